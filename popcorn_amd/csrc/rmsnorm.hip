// RMSNorm forward and backward: row passes that read each operand from HBM
// once.
//
// Fast path (cols a multiple of the 16-byte pack and at most 256*8 packs):
// a row is held in registers by TPR lanes (64 = one wavefront per row, or 256
// = the whole 4-wave block), each lane owning VPT packs strided by TPR so a
// wave's loads are contiguous. The sum of squares is a DPP/shuffle wave
// reduction plus, for TPR=256, a 4-entry LDS exchange. Any other shape takes
// a one-block-per-row kernel that loops over the row twice.
//
// Backward keeps w and the running dw / dbias columns in registers for a
// block that walks a contiguous run of rows, prefetching the next row's x and
// dy while the current row's dot product is reduced. Per-block fp32 partial
// rows go to a workspace and one more kernel sums them in a fixed order, so dw
// is deterministic.
#include "api.h"
#include "common.h"

namespace pk {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxVpt = 8;
constexpr int kBwdMaxBlocks = 1024;

// Sum over the TPR lanes that share a row. TPR=64: one wave. TPR=256: the
// block; `red` holds one slot per wave and the call is a block barrier.
template <int TPR> __device__ __forceinline__ float row_sum(float v, float* red) {
  v = wave_sum(v);
  if constexpr (TPR == 64) {
    return v;
  } else {
    static_assert(TPR == kThreads, "rows span one wave or the whole block");
    const int wave = threadIdx.x / 64;
    __syncthreads();  // previous readers of `red` are done
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) t += red[i];
    return t;
  }
}

// torch: rms = (h * rsqrt(mean(h^2) + eps)).to(T); y = rms * w; y = y + bias.
template <typename T, bool BIAS> __device__ __forceinline__ T fwd_elem(float xv, float r, float wv, float bv) {
  float y = round_to<T>(xv * r) * wv;
  if constexpr (BIAS) y = round_to<T>(y) + bv;
  return from_f32<T>(y);
}

template <typename T, int TPR, int VPT, bool BIAS>
__global__ __launch_bounds__(kThreads) void rmsnorm_fwd_vec(const T* __restrict__ x, const T* __restrict__ w,
                                                            const T* __restrict__ bias, T* __restrict__ y,
                                                            float* __restrict__ rstd, int64_t rows, int cols,
                                                            float eps, float inv_cols) {
  constexpr int P = Vec<T>::N;
  constexpr int RPB = kThreads / TPR;
  __shared__ float red[kWaves];
  const int lane = threadIdx.x % TPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
  const bool live = row < rows;
  const int nvec = cols / P;
  const T* xr = x + row * cols;

  Vec<T> xv[VPT];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int v = lane + k * TPR;
    if (live && v < nvec) {
      xv[k] = ld16_stream(xr + v * P);
#pragma unroll
      for (int j = 0; j < P; ++j) {
        const float f = to_f32(xv[k].v[j]);
        ss += f * f;
      }
    }
  }
  ss = row_sum<TPR>(ss, red);
  if (!live) return;
  const float r = 1.0f / sqrtf(ss * inv_cols + eps);
  if (rstd != nullptr && lane == 0) rstd[row] = r;

  T* yr = y + row * cols;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int v = lane + k * TPR;
    if (v < nvec) {
      const Vec<T> wv = ld16(w + v * P);
      Vec<T> bv;
      if constexpr (BIAS) bv = ld16(bias + v * P);
      Vec<T> out;
#pragma unroll
      for (int j = 0; j < P; ++j)
        out.v[j] = fwd_elem<T, BIAS>(to_f32(xv[k].v[j]), r, to_f32(wv.v[j]), BIAS ? to_f32(bv.v[j]) : 0.f);
      st16_stream(yr + v * P, out);
    }
  }
}

// Any row width, any alignment: one block per row, two passes over x.
template <typename T, bool BIAS>
__global__ __launch_bounds__(kThreads) void rmsnorm_fwd_any(const T* __restrict__ x, const T* __restrict__ w,
                                                            const T* __restrict__ bias, T* __restrict__ y,
                                                            float* __restrict__ rstd, int64_t rows, int cols,
                                                            float eps, float inv_cols) {
  __shared__ float red[kWaves];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * cols;
  float ss = 0.f;
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    const float f = to_f32(xr[c]);
    ss += f * f;
  }
  ss = row_sum<kThreads>(ss, red);
  const float r = 1.0f / sqrtf(ss * inv_cols + eps);
  if (rstd != nullptr && threadIdx.x == 0) rstd[row] = r;
  T* yr = y + row * cols;
  for (int c = threadIdx.x; c < cols; c += kThreads)
    yr[c] = fwd_elem<T, BIAS>(to_f32(xr[c]), r, to_f32(w[c]), BIAS ? to_f32(bias[c]) : 0.f);
}

// ---------------------------------------------------------------------------
// backward

template <typename T, int TPR, int VPT, bool BIAS>
__global__ __launch_bounds__(kThreads) void rmsnorm_bwd_vec(const T* __restrict__ x, const T* __restrict__ w,
                                                            const float* __restrict__ rstd,
                                                            const T* __restrict__ dy, T* __restrict__ dx,
                                                            float* __restrict__ dw_part,
                                                            float* __restrict__ db_part, int64_t rows, int cols,
                                                            float inv_cols, int64_t rows_per_block) {
  constexpr int P = Vec<T>::N;
  constexpr int RPB = kThreads / TPR;
  __shared__ float red[kWaves];
  const int lane = threadIdx.x % TPR;
  const int slot = threadIdx.x / TPR;
  const int nvec = cols / P;

  float wf[VPT][P], dwa[VPT][P], dba[VPT][P];
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int v = lane + k * TPR;
    Vec<T> wv;
    if (v < nvec) wv = ld16(w + v * P);
#pragma unroll
    for (int j = 0; j < P; ++j) {
      wf[k][j] = v < nvec ? to_f32(wv.v[j]) : 0.f;
      dwa[k][j] = 0.f;
      dba[k][j] = 0.f;
    }
  }

  // This block owns rows [row0, row_end); slot s takes row0 + s, + RPB, ...
  const int64_t row0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t row_end = row0 + rows_per_block < rows ? row0 + rows_per_block : rows;
  // Every slot runs the same trip count so the TPR=256 barriers line up.
  const int64_t trips = (row_end - row0 + RPB - 1) / RPB;

  Vec<T> xv[VPT], gv[VPT], xn[VPT], gn[VPT];
  auto fetch = [&](int64_t row, Vec<T>* xo, Vec<T>* go) {
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int v = lane + k * TPR;
      if (row < row_end && v < nvec) {
        xo[k] = ld16_stream(x + row * cols + v * P);
        go[k] = ld16_stream(dy + row * cols + v * P);
      }
    }
  };
  fetch(row0 + slot, xv, gv);

  for (int64_t t = 0; t < trips; ++t) {
    const int64_t row = row0 + slot + t * RPB;
    const bool live = row < row_end;
    fetch(row + RPB, xn, gn);  // next row of this slot, in flight during the reduction
    const float r = live ? rstd[row] : 0.f;
    float dot = 0.f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int v = lane + k * TPR;
      if (live && v < nvec) {
#pragma unroll
        for (int j = 0; j < P; ++j) dot += to_f32(gv[k].v[j]) * wf[k][j] * (to_f32(xv[k].v[j]) * r);
      }
    }
    dot = row_sum<TPR>(dot, red) * inv_cols;
    if (live) {
#pragma unroll
      for (int k = 0; k < VPT; ++k) {
        const int v = lane + k * TPR;
        if (v < nvec) {
          Vec<T> out;
#pragma unroll
          for (int j = 0; j < P; ++j) {
            const float g = to_f32(gv[k].v[j]);
            const float n = to_f32(xv[k].v[j]) * r;
            out.v[j] = from_f32<T>(r * (g * wf[k][j] - n * dot));
            dwa[k][j] += g * n;
            if constexpr (BIAS) dba[k][j] += g;
          }
          st16_stream(dx + row * cols + v * P, out);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      xv[k] = xn[k];
      gv[k] = gn[k];
    }
  }

  // One partial row per (block, slot).
  const int64_t prow = (int64_t)blockIdx.x * RPB + slot;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int v = lane + k * TPR;
    if (v < nvec) {
      float* dst = dw_part + prow * cols + v * P;
#pragma unroll
      for (int j = 0; j < P; j += 4)
        *reinterpret_cast<float4*>(dst + j) = make_float4(dwa[k][j], dwa[k][j + 1], dwa[k][j + 2], dwa[k][j + 3]);
      if constexpr (BIAS) {
        float* bdst = db_part + prow * cols + v * P;
#pragma unroll
        for (int j = 0; j < P; j += 4)
          *reinterpret_cast<float4*>(bdst + j) =
              make_float4(dba[k][j], dba[k][j + 1], dba[k][j + 2], dba[k][j + 3]);
      }
    }
  }
}

// Any row width: one block walks rows_per_block rows, one column per thread
// per step, partial rows as above (one per block).
template <typename T, bool BIAS>
__global__ __launch_bounds__(kThreads) void rmsnorm_bwd_any(const T* __restrict__ x, const T* __restrict__ w,
                                                            const float* __restrict__ rstd,
                                                            const T* __restrict__ dy, T* __restrict__ dx,
                                                            float* __restrict__ dw_part,
                                                            float* __restrict__ db_part, int64_t rows, int cols,
                                                            float inv_cols, int64_t rows_per_block) {
  __shared__ float red[kWaves];
  const int64_t row0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t row_end = row0 + rows_per_block < rows ? row0 + rows_per_block : rows;
  float* dwp = dw_part + (int64_t)blockIdx.x * cols;
  float* dbp = BIAS ? db_part + (int64_t)blockIdx.x * cols : nullptr;
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    dwp[c] = 0.f;
    if constexpr (BIAS) dbp[c] = 0.f;
  }
  for (int64_t row = row0; row < row_end; ++row) {
    const float r = rstd[row];
    const T* xr = x + row * cols;
    const T* gr = dy + row * cols;
    float dot = 0.f;
    for (int c = threadIdx.x; c < cols; c += kThreads) dot += to_f32(gr[c]) * to_f32(w[c]) * (to_f32(xr[c]) * r);
    dot = row_sum<kThreads>(dot, red) * inv_cols;
    T* dxr = dx + row * cols;
    for (int c = threadIdx.x; c < cols; c += kThreads) {
      const float g = to_f32(gr[c]);
      const float n = to_f32(xr[c]) * r;
      dxr[c] = from_f32<T>(r * (g * to_f32(w[c]) - n * dot));
      dwp[c] += g * n;  // column c is only ever touched by this thread
      if constexpr (BIAS) dbp[c] += g;
    }
  }
}

// dw[c] = sum over parts of part[p][c], in a fixed order. 64 columns per
// block, 4 waves splitting the parts, combined through LDS.
template <typename T>
__global__ __launch_bounds__(kThreads) void column_sum(const float* __restrict__ part, T* __restrict__ out,
                                                       int64_t parts, int cols) {
  __shared__ float acc[kWaves][64];
  const int c = blockIdx.x * 64 + (threadIdx.x & 63);
  const int wave = threadIdx.x / 64;
  float s = 0.f;
  if (c < cols)
    for (int64_t p = wave; p < parts; p += kWaves) s += part[p * cols + c];
  acc[wave][threadIdx.x & 63] = s;
  __syncthreads();
  if (wave == 0 && c < cols) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) t += acc[i][threadIdx.x];
    out[c] = from_f32<T>(t);
  }
}

// ---------------------------------------------------------------------------
// launch planning

struct Plan {
  bool vec;  // fast path usable
  int tpr;   // 64 or 256
  int vpt;   // 1, 2, 4, 8
};

Plan plan_for(int64_t cols, int esize, bool aligned) {
  const int P = 16 / esize;
  Plan p{false, kThreads, 1};
  if (!aligned || cols % P != 0) return p;
  const int64_t nvec = cols / P;
  if (nvec > (int64_t)kThreads * kMaxVpt) return p;
  p.vec = true;
  p.tpr = nvec <= 64 * kMaxVpt ? 64 : kThreads;
  int64_t need = (nvec + p.tpr - 1) / p.tpr;
  p.vpt = need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : 8;
  return p;
}

int64_t bwd_blocks(int64_t rows, const Plan& p) {
  const int64_t rpb = p.vec ? kThreads / p.tpr : 1;
  const int64_t want = (rows + rpb - 1) / rpb;
  return want < kBwdMaxBlocks ? want : kBwdMaxBlocks;
}

int64_t bwd_parts(int64_t rows, const Plan& p) { return bwd_blocks(rows, p) * (p.vec ? kThreads / p.tpr : 1); }

template <typename T, bool BIAS, int TPR, int VPT>
void launch_fwd_vec(int64_t rows, const void* x, const void* w, const void* b, void* y, float* rstd, int cols,
                    float eps, hipStream_t s) {
  constexpr int RPB = kThreads / TPR;
  hipLaunchKernelGGL((rmsnorm_fwd_vec<T, TPR, VPT, BIAS>), dim3((rows + RPB - 1) / RPB), dim3(kThreads), 0, s,
                     static_cast<const T*>(x), static_cast<const T*>(w), static_cast<const T*>(b),
                     static_cast<T*>(y), rstd, rows, cols, eps, 1.0f / (float)cols);
}

template <typename T, bool BIAS, int TPR>
void dispatch_fwd_vpt(int vpt, int64_t rows, const void* x, const void* w, const void* b, void* y, float* rstd,
                      int cols, float eps, hipStream_t s) {
  switch (vpt) {
    case 1: return launch_fwd_vec<T, BIAS, TPR, 1>(rows, x, w, b, y, rstd, cols, eps, s);
    case 2: return launch_fwd_vec<T, BIAS, TPR, 2>(rows, x, w, b, y, rstd, cols, eps, s);
    case 4: return launch_fwd_vec<T, BIAS, TPR, 4>(rows, x, w, b, y, rstd, cols, eps, s);
    default: return launch_fwd_vec<T, BIAS, TPR, 8>(rows, x, w, b, y, rstd, cols, eps, s);
  }
}

template <typename T, bool BIAS>
int fwd(const void* x, const void* w, const void* b, void* y, float* rstd, int64_t rows, int64_t cols, float eps,
        hipStream_t s) {
  const bool aligned = aligned16(x) && aligned16(w) && aligned16(y) && (!BIAS || aligned16(b));
  const Plan p = plan_for(cols, sizeof(T), aligned);
  if (!p.vec) {
    hipLaunchKernelGGL((rmsnorm_fwd_any<T, BIAS>), dim3(rows), dim3(kThreads), 0, s, static_cast<const T*>(x),
                       static_cast<const T*>(w), static_cast<const T*>(b), static_cast<T*>(y), rstd, rows,
                       (int)cols, eps, 1.0f / (float)cols);
  } else if (p.tpr == 64) {
    dispatch_fwd_vpt<T, BIAS, 64>(p.vpt, rows, x, w, b, y, rstd, (int)cols, eps, s);
  } else {
    dispatch_fwd_vpt<T, BIAS, kThreads>(p.vpt, rows, x, w, b, y, rstd, (int)cols, eps, s);
  }
  return launched("pk_rmsnorm_fwd");
}

struct BwdArgs {
  const void *x, *w, *dy;
  const float* rstd;
  void *dx, *dw, *db;
  float *dw_part, *db_part;
  int64_t rows;
  int cols;
  hipStream_t s;
};

template <typename T, bool BIAS, int TPR, int VPT> void launch_bwd_vec(const BwdArgs& a, int64_t blocks) {
  const int64_t per = (a.rows + blocks - 1) / blocks;
  hipLaunchKernelGGL((rmsnorm_bwd_vec<T, TPR, VPT, BIAS>), dim3(blocks), dim3(kThreads), 0, a.s,
                     static_cast<const T*>(a.x), static_cast<const T*>(a.w), a.rstd, static_cast<const T*>(a.dy),
                     static_cast<T*>(a.dx), a.dw_part, a.db_part, a.rows, a.cols, 1.0f / (float)a.cols, per);
}

template <typename T, bool BIAS, int TPR> void dispatch_bwd_vpt(int vpt, const BwdArgs& a, int64_t blocks) {
  switch (vpt) {
    case 1: return launch_bwd_vec<T, BIAS, TPR, 1>(a, blocks);
    case 2: return launch_bwd_vec<T, BIAS, TPR, 2>(a, blocks);
    case 4: return launch_bwd_vec<T, BIAS, TPR, 4>(a, blocks);
    default: return launch_bwd_vec<T, BIAS, TPR, 8>(a, blocks);
  }
}

template <typename T, bool BIAS> int bwd(const BwdArgs& a) {
  const bool aligned = aligned16(a.x) && aligned16(a.w) && aligned16(a.dy) && aligned16(a.dx);
  const Plan p = plan_for(a.cols, sizeof(T), aligned);
  const int64_t blocks = bwd_blocks(a.rows, p);
  if (!p.vec) {
    const int64_t per = (a.rows + blocks - 1) / blocks;
    hipLaunchKernelGGL((rmsnorm_bwd_any<T, BIAS>), dim3(blocks), dim3(kThreads), 0, a.s, static_cast<const T*>(a.x),
                       static_cast<const T*>(a.w), a.rstd, static_cast<const T*>(a.dy), static_cast<T*>(a.dx),
                       a.dw_part, a.db_part, a.rows, a.cols, 1.0f / (float)a.cols, per);
  } else if (p.tpr == 64) {
    dispatch_bwd_vpt<T, BIAS, 64>(p.vpt, a, blocks);
  } else {
    dispatch_bwd_vpt<T, BIAS, kThreads>(p.vpt, a, blocks);
  }
  const int64_t parts = bwd_parts(a.rows, p);
  const dim3 grid((a.cols + 63) / 64);
  hipLaunchKernelGGL(column_sum<T>, grid, dim3(kThreads), 0, a.s, a.dw_part, static_cast<T*>(a.dw), parts, a.cols);
  if (BIAS)
    hipLaunchKernelGGL(column_sum<T>, grid, dim3(kThreads), 0, a.s, a.db_part, static_cast<T*>(a.db), parts, a.cols);
  return launched("pk_rmsnorm_bwd");
}

int64_t workspace_bytes(int64_t rows, int64_t cols, int dtype, bool bias) {
  // Plan with alignment assumed: the vec plan needs at least as many parts
  // as the fallback, so the size covers both.
  const Plan p = plan_for(cols, elem_size(dtype), true);
  const int64_t parts = bwd_parts(rows, p);
  int64_t one = parts * cols * (int64_t)sizeof(float);
  one = (one + 255) / 256 * 256;
  return bias ? 2 * one : one;
}

int check_shape(const char* who, int64_t rows, int64_t cols, int dtype) {
  if (rows < 0 || cols < 0) return fail(PK_ERR_INVALID, "%s: negative shape (%lld, %lld)", who, (long long)rows,
                                        (long long)cols);
  if (cols > (int64_t)1 << 30) return fail(PK_ERR_UNSUPPORTED, "%s: %lld columns", who, (long long)cols);
  if (!known_dtype(dtype)) return fail(PK_ERR_UNSUPPORTED, "%s: dtype code %d", who, dtype);
  return PK_OK;
}

}  // namespace
}  // namespace pk

extern "C" {

int pk_rmsnorm_fwd(const void* x, const void* w, const void* bias, void* y, float* rstd, int64_t rows, int64_t cols,
                   float eps, int dtype, void* stream) {
  using namespace pk;
  if (int st = check_shape("pk_rmsnorm_fwd", rows, cols, dtype)) return st;
  if (rows == 0) return PK_OK;
  if (cols == 0) return fail(PK_ERR_INVALID, "pk_rmsnorm_fwd: zero-width rows");
  if (!x || !w || !y) return fail(PK_ERR_INVALID, "pk_rmsnorm_fwd: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool b = bias != nullptr;
  switch (dtype) {
    case PK_F32: return b ? fwd<float, true>(x, w, bias, y, rstd, rows, cols, eps, s)
                          : fwd<float, false>(x, w, bias, y, rstd, rows, cols, eps, s);
    case PK_BF16: return b ? fwd<bf16, true>(x, w, bias, y, rstd, rows, cols, eps, s)
                           : fwd<bf16, false>(x, w, bias, y, rstd, rows, cols, eps, s);
    default: return b ? fwd<f16, true>(x, w, bias, y, rstd, rows, cols, eps, s)
                      : fwd<f16, false>(x, w, bias, y, rstd, rows, cols, eps, s);
  }
}

int64_t pk_rmsnorm_bwd_workspace(int64_t rows, int64_t cols, int dtype) {
  using namespace pk;
  if (rows <= 0 || cols <= 0 || !known_dtype(dtype)) return 0;
  return workspace_bytes(rows, cols, dtype, true);
}

int pk_rmsnorm_bwd(const void* x, const void* w, const float* rstd, const void* dy, void* dx, void* dw, void* dbias,
                   void* workspace, int64_t workspace_bytes, int64_t rows, int64_t cols, int dtype, void* stream) {
  using namespace pk;
  if (int st = check_shape("pk_rmsnorm_bwd", rows, cols, dtype)) return st;
  if (cols == 0) return fail(PK_ERR_INVALID, "pk_rmsnorm_bwd: zero-width rows");
  if (!x || !w || !rstd || !dy || !dx || !dw || !workspace)
    return fail(PK_ERR_INVALID, "pk_rmsnorm_bwd: null pointer");
  const bool b = dbias != nullptr;
  if (rows == 0) return fail(PK_ERR_UNSUPPORTED, "pk_rmsnorm_bwd: zero rows (dw is all zeros; fill it host-side)");
  const int64_t need = pk::workspace_bytes(rows, cols, dtype, b);
  if (workspace_bytes < need)
    return fail(PK_ERR_INVALID, "pk_rmsnorm_bwd: workspace of %lld bytes, need %lld", (long long)workspace_bytes,
                (long long)need);
  if (!aligned16(workspace)) return fail(PK_ERR_INVALID, "pk_rmsnorm_bwd: workspace not 16-byte aligned");
  const int64_t half = need / (b ? 2 : 1);
  BwdArgs a{x,
            w,
            dy,
            rstd,
            dx,
            dw,
            dbias,
            static_cast<float*>(workspace),
            b ? reinterpret_cast<float*>(static_cast<char*>(workspace) + half) : nullptr,
            rows,
            (int)cols,
            static_cast<hipStream_t>(stream)};
  switch (dtype) {
    case PK_F32: return b ? bwd<float, true>(a) : bwd<float, false>(a);
    case PK_BF16: return b ? bwd<bf16, true>(a) : bwd<bf16, false>(a);
    default: return b ? bwd<f16, true>(a) : bwd<f16, false>(a);
  }
}

}  // extern "C"
