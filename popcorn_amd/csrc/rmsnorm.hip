// RMSNorm forward and backward: row passes that read each operand from HBM
// once.
//
// Fast path (cols a multiple of the 16-byte pack, at most 1024*16 packs): a
// row is held in registers by TPR lanes, each owning VPT packs strided by TPR
// so a wave's loads are contiguous. TPR = 64 is one wavefront per row (several
// rows per block, sum of squares by wave shuffles alone); TPR = NTB is the
// whole block (a wave reduction plus one LDS exchange). Any other shape takes
// a one-block-per-row kernel that loops over the row twice.
//
// Forward launches one block per row group, except for row counts that fit in
// a few waves of resident blocks: there a persistent grid takes rows in grid
// stride with w in registers and the next row prefetched (measured faster on
// MI355X for such short launches, slower for long ones).
//
// Backward is a persistent grid (a few blocks per CU): block b takes rows
// b, b + G, b + 2G, ... (G = grid size; the blocks together sweep the tensors
// front to back, which measured 13% faster than contiguous runs of rows per
// block) with w and its running dw / dbias columns in registers, prefetching
// the next row's x and dy while the current row's dot product is reduced.
// Blocks leave one fp32 partial row each (the rows of a block's wavefront
// slots are combined through LDS first), and a two-stage column reduction
// sums the partials in a fixed order, so dw is deterministic.
#include "api.h"
#include "common.h"

namespace pk {
namespace {

constexpr int kThreads = 256;    // fallback kernels and column sums
constexpr int kMaxVpt = 16;
constexpr int kColSplit = 32;    // partial rows summed per block in the first column-sum stage

// Sum over the TPR lanes that share a row: TPR = 64 is one wave; TPR = NTB is
// the block, `red` holds one slot per wave and the call is a block barrier.
template <int NTB, int TPR> __device__ __forceinline__ float row_sum(float v, float* red) {
  v = wave_sum(v);
  if constexpr (TPR == 64) {
    return v;
  } else {
    static_assert(TPR == NTB, "rows span one wave or the whole block");
    constexpr int W = NTB / 64;
    const int wave = threadIdx.x / 64;
    __syncthreads();  // previous readers of `red` are done
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < W; ++i) t += red[i];
    return t;
  }
}

// torch: rms = (h * rsqrt(mean(h^2) + eps)).to(T); y = rms * w; y = y + bias.
template <typename T, bool BIAS> __device__ __forceinline__ T fwd_elem(float xv, float r, float wv, float bv) {
  float y = round_to<T>(xv * r) * wv;
  if constexpr (BIAS) y = round_to<T>(y) + bv;
  return from_f32<T>(y);
}

// One row per TPR lanes, RPB = NTB / TPR rows per block.
template <typename T, int NTB, int TPR, int VPT, bool BIAS>
__global__ __launch_bounds__(NTB) void rmsnorm_fwd_vec(const T* __restrict__ x, const T* __restrict__ w,
                                                       const T* __restrict__ bias, T* __restrict__ y,
                                                       float* __restrict__ rstd, int64_t rows, int cols, float eps,
                                                       float inv_cols) {
  constexpr int P = Vec<T>::N;
  constexpr int RPB = NTB / TPR;
  __shared__ float red[NTB / 64];
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
  ss = row_sum<NTB, TPR>(ss, red);
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

// Persistent form of rmsnorm_fwd_vec for short launches: slot s of block b
// takes rows b * RPB + s + k * stride, with w (and bias) in registers and the
// next row's x in flight while the current row is reduced.
template <typename T, int NTB, int TPR, int VPT, bool BIAS>
__global__ __launch_bounds__(NTB) void rmsnorm_fwd_grid(const T* __restrict__ x, const T* __restrict__ w,
                                                        const T* __restrict__ bias, T* __restrict__ y,
                                                        float* __restrict__ rstd, int64_t rows, int cols, float eps,
                                                        float inv_cols) {
  constexpr int P = Vec<T>::N;
  constexpr int RPB = NTB / TPR;
  __shared__ float red[NTB / 64];
  const int lane = threadIdx.x % TPR;
  const int nvec = cols / P;
  const int64_t stride = (int64_t)gridDim.x * RPB;
  const int64_t first = (int64_t)blockIdx.x * RPB;
  const int64_t row0 = first + threadIdx.x / TPR;
  const int64_t trips = (rows - first + stride - 1) / stride;  // the same for every slot: barriers line up
  Vec<T> wv[VPT], bv[VPT];
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int v = lane + k * TPR;
    if (v < nvec) {
      wv[k] = ld16(w + v * P);
      if constexpr (BIAS) bv[k] = ld16(bias + v * P);
    }
  }
  Vec<T> xv[VPT], xn[VPT];
  auto fetch = [&](int64_t row, Vec<T>* xo) {
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int v = lane + k * TPR;
      if (row < rows && v < nvec) xo[k] = ld16_stream(x + row * cols + v * P);
    }
  };
  fetch(row0, xv);
  for (int64_t t = 0; t < trips; ++t) {
    const int64_t row = row0 + t * stride;
    fetch(row + stride, xn);
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int v = lane + k * TPR;
      if (row < rows && v < nvec)
#pragma unroll
        for (int j = 0; j < P; ++j) {
          const float f = to_f32(xv[k].v[j]);
          ss += f * f;
        }
    }
    ss = row_sum<NTB, TPR>(ss, red);
    if (row < rows) {
      const float r = 1.0f / sqrtf(ss * inv_cols + eps);
      if (rstd != nullptr && lane == 0) rstd[row] = r;
#pragma unroll
      for (int k = 0; k < VPT; ++k) {
        const int v = lane + k * TPR;
        if (v < nvec) {
          Vec<T> out;
#pragma unroll
          for (int j = 0; j < P; ++j)
            out.v[j] = fwd_elem<T, BIAS>(to_f32(xv[k].v[j]), r, to_f32(wv[k].v[j]), BIAS ? to_f32(bv[k].v[j]) : 0.f);
          st16_stream(y + row * cols + v * P, out);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < VPT; ++k) xv[k] = xn[k];
  }
}

// Any row width, any alignment: one block per row, two passes over x.
template <typename T, bool BIAS>
__global__ __launch_bounds__(kThreads) void rmsnorm_fwd_any(const T* __restrict__ x, const T* __restrict__ w,
                                                            const T* __restrict__ bias, T* __restrict__ y,
                                                            float* __restrict__ rstd, int64_t rows, int cols,
                                                            float eps, float inv_cols) {
  __shared__ float red[kThreads / 64];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * cols;
  float ss = 0.f;
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    const float f = to_f32(xr[c]);
    ss += f * f;
  }
  ss = row_sum<kThreads, kThreads>(ss, red);
  const float r = 1.0f / sqrtf(ss * inv_cols + eps);
  if (rstd != nullptr && threadIdx.x == 0) rstd[row] = r;
  T* yr = y + row * cols;
  for (int c = threadIdx.x; c < cols; c += kThreads)
    yr[c] = fwd_elem<T, BIAS>(to_f32(xr[c]), r, to_f32(w[c]), BIAS ? to_f32(bias[c]) : 0.f);
}

// ---------------------------------------------------------------------------
// backward

// Adds this lane's VPT*P column values into the block's partial row in LDS
// (slot by slot, so the order is fixed) and lets slot 0 write it out.
template <int NTB, int TPR, int VPT, int P>
__device__ __forceinline__ void flush_partial(float (&acc)[VPT][P], float* lds_row, float* __restrict__ dst,
                                              int nvec) {
  constexpr int RPB = NTB / TPR;
  const int lane = threadIdx.x % TPR;
  const int slot = threadIdx.x / TPR;
  if constexpr (RPB > 1) {
    for (int s = RPB - 1; s >= 1; --s) {
      if (slot == s) {
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
          const int v = lane + k * TPR;
          if (v < nvec)
#pragma unroll
            for (int j = 0; j < P; ++j) lds_row[v * P + j] = (s == RPB - 1 ? 0.f : lds_row[v * P + j]) + acc[k][j];
        }
      }
      __syncthreads();
    }
  }
  if (slot == 0) {
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int v = lane + k * TPR;
      if (v < nvec) {
#pragma unroll
        for (int j = 0; j < P; j += 4) {
          float4 o = make_float4(acc[k][j], acc[k][j + 1], acc[k][j + 2], acc[k][j + 3]);
          if constexpr (RPB > 1) {
            o.x += lds_row[v * P + j];
            o.y += lds_row[v * P + j + 1];
            o.z += lds_row[v * P + j + 2];
            o.w += lds_row[v * P + j + 3];
          }
          *reinterpret_cast<float4*>(dst + v * P + j) = o;
        }
      }
    }
  }
}

template <typename T, int NTB, int TPR, int VPT, bool BIAS>
__global__ __launch_bounds__(NTB) void rmsnorm_bwd_vec(const T* __restrict__ x, const T* __restrict__ w,
                                                       const float* __restrict__ rstd, const T* __restrict__ dy,
                                                       T* __restrict__ dx, float* __restrict__ dw_part,
                                                       float* __restrict__ db_part, int64_t rows, int cols,
                                                       float inv_cols) {
  constexpr int P = Vec<T>::N;
  constexpr int RPB = NTB / TPR;
  __shared__ float red[NTB / 64];
  extern __shared__ float lds_row[];  // cols floats when RPB > 1
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

  // Slot s of block b takes rows b * RPB + s + k * stride; every slot runs
  // the same trip count so block-wide barriers line up.
  const int64_t stride = (int64_t)gridDim.x * RPB;
  const int64_t row0 = (int64_t)blockIdx.x * RPB;
  const int64_t trips = (rows - row0 + stride - 1) / stride;

  Vec<T> xv[VPT], gv[VPT], xn[VPT], gn[VPT];
  auto fetch = [&](int64_t row, Vec<T>* xo, Vec<T>* go) {
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int v = lane + k * TPR;
      if (row < rows && v < nvec) {
        xo[k] = ld16_stream(x + row * cols + v * P);
        go[k] = ld16_stream(dy + row * cols + v * P);
      }
    }
  };
  fetch(row0 + slot, xv, gv);

  for (int64_t t = 0; t < trips; ++t) {
    const int64_t row = row0 + slot + t * stride;
    const bool live = row < rows;
    fetch(row + stride, xn, gn);  // next row of this slot, in flight during the reduction
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
    dot = row_sum<NTB, TPR>(dot, red) * inv_cols;
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

  flush_partial<NTB, TPR, VPT, P>(dwa, lds_row, dw_part + (int64_t)blockIdx.x * cols, nvec);
  if constexpr (BIAS) {
    if constexpr (RPB > 1) __syncthreads();  // lds_row is reused
    flush_partial<NTB, TPR, VPT, P>(dba, lds_row, db_part + (int64_t)blockIdx.x * cols, nvec);
  }
}

// Any row width: block b walks rows b, b + G, ..., one column per thread per
// step, one partial row per block.
template <typename T, bool BIAS>
__global__ __launch_bounds__(kThreads) void rmsnorm_bwd_any(const T* __restrict__ x, const T* __restrict__ w,
                                                            const float* __restrict__ rstd,
                                                            const T* __restrict__ dy, T* __restrict__ dx,
                                                            float* __restrict__ dw_part,
                                                            float* __restrict__ db_part, int64_t rows, int cols,
                                                            float inv_cols) {
  __shared__ float red[kThreads / 64];
  float* dwp = dw_part + (int64_t)blockIdx.x * cols;
  float* dbp = BIAS ? db_part + (int64_t)blockIdx.x * cols : nullptr;
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    dwp[c] = 0.f;
    if constexpr (BIAS) dbp[c] = 0.f;
  }
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const float r = rstd[row];
    const T* xr = x + row * cols;
    const T* gr = dy + row * cols;
    float dot = 0.f;
    for (int c = threadIdx.x; c < cols; c += kThreads) dot += to_f32(gr[c]) * to_f32(w[c]) * (to_f32(xr[c]) * r);
    dot = row_sum<kThreads, kThreads>(dot, red) * inv_cols;
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

// Column sums of a [parts, cols] fp32 array in a fixed order. Stage one:
// block (cx, s) sums parts [s*kColSplit, (s+1)*kColSplit) of 256 columns into
// stage[s]; stage two sums the stage rows and rounds to T.
__global__ __launch_bounds__(kThreads) void column_sum_stage(const float* __restrict__ part,
                                                            float* __restrict__ stage, int64_t parts, int cols) {
  const int c = blockIdx.x * kThreads + threadIdx.x;
  const int64_t p0 = (int64_t)blockIdx.y * kColSplit;
  const int64_t p1 = p0 + kColSplit < parts ? p0 + kColSplit : parts;
  if (c >= cols) return;
  float s = 0.f;
  for (int64_t p = p0; p < p1; ++p) s += part[p * cols + c];
  stage[(int64_t)blockIdx.y * cols + c] = s;
}

template <typename T>
__global__ __launch_bounds__(kThreads) void column_sum_final(const float* __restrict__ stage, T* __restrict__ out,
                                                            int64_t n, int cols) {
  const int c = blockIdx.x * kThreads + threadIdx.x;
  if (c >= cols) return;
  float s = 0.f;
  for (int64_t p = 0; p < n; ++p) s += stage[p * cols + c];
  out[c] = from_f32<T>(s);
}

// ---------------------------------------------------------------------------
// launch planning

struct Plan {
  bool vec;  // fast path usable
  int ntb;   // threads per block
  int tpr;   // threads per row: 64 or ntb
  int vpt;   // 16-byte packs per thread: 1, 2, 4, 8, 16
};

int pow2_at_least(int64_t n) {
  int p = 1;
  while (p < n) p *= 2;
  return p;
}

// Launch shape for rows of `cols` elements of `esize` bytes: one row per
// wavefront up to 4 packs per lane, wider rows over a block at 4 packs per
// thread (forward) or 2 (backward, which also keeps dw columns in
// registers). Measured on MI355X these beat one-wave rows of 16 packs and
// blocks of 128 / 512 / 1024 threads for 4096-wide fp32 and 8192-wide bf16
// rows.
Plan plan_for(int64_t cols, int esize, bool aligned, bool backward) {
  const int P = 16 / esize;
  Plan p{false, kThreads, kThreads, 1};
  if (!aligned || cols % P != 0) return p;
  const int64_t nvec = cols / P;
  const int wave_max = 4;
  const int block_vpt = backward ? 2 : 4;
  if (nvec > (int64_t)1024 * kMaxVpt) return p;
  p.vec = true;
  if (nvec <= 64 * wave_max) {  // one wave per row, 4 rows per block
    p.ntb = 256;
    p.tpr = 64;
    p.vpt = pow2_at_least((nvec + 63) / 64);
  } else {  // a block per row
    p.vpt = block_vpt;
    p.ntb = p.tpr = pow2_at_least((nvec + p.vpt - 1) / p.vpt);
    if (p.ntb > 1024) {
      p.ntb = p.tpr = 1024;
      p.vpt = pow2_at_least((nvec + 1023) / 1024);
    }
  }
  return p;
}

// Resident blocks per CU of a kernel at this launch shape (queried once per
// instantiation; each CU of an MI355X is alike).
template <typename K> int resident_per_cu(K kernel, int threads, size_t lds) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, lds) != hipSuccess || n < 1) n = 1;
  return n;
}

template <typename T, bool BIAS, int NTB, int TPR, int VPT> int bwd_resident(int cols) {
  // dynamic LDS of a 4-rows-per-block shape: one fp32 row of at most 64*4*8 columns
  static const int n = resident_per_cu(rmsnorm_bwd_vec<T, NTB, TPR, VPT, BIAS>, NTB,
                                       NTB / TPR > 1 ? (size_t)64 * 4 * 8 * sizeof(float) : 0);
  (void)cols;
  return n;
}

template <typename T, bool BIAS> int bwd_any_resident() {
  static const int n = resident_per_cu(rmsnorm_bwd_any<T, BIAS>, kThreads, 0);
  return n;
}

template <typename T, bool BIAS, int NTB, int TPR, int VPT>
void launch_fwd_vec(int64_t rows, const void* x, const void* w, const void* b, void* y, float* rstd, int cols,
                    float eps, hipStream_t s) {
  constexpr int RPB = NTB / TPR;
  const int64_t groups = (rows + RPB - 1) / RPB;
  // Up to four waves of resident blocks: the persistent grid.
  static const int per_cu = resident_per_cu(rmsnorm_fwd_vec<T, NTB, TPR, VPT, BIAS>, NTB, 0);
  static const int per_cu_grid = resident_per_cu(rmsnorm_fwd_grid<T, NTB, TPR, VPT, BIAS>, NTB, 0);
  if (groups <= (int64_t)4 * cu_count() * per_cu) {
    const int64_t slots = (int64_t)cu_count() * per_cu_grid;
    hipLaunchKernelGGL((rmsnorm_fwd_grid<T, NTB, TPR, VPT, BIAS>), dim3(groups < slots ? groups : slots), dim3(NTB), 0,
                       s, static_cast<const T*>(x), static_cast<const T*>(w), static_cast<const T*>(b),
                       static_cast<T*>(y), rstd, rows, cols, eps, 1.0f / (float)cols);
    return;
  }
  hipLaunchKernelGGL((rmsnorm_fwd_vec<T, NTB, TPR, VPT, BIAS>), dim3(groups), dim3(NTB), 0, s,
                     static_cast<const T*>(x), static_cast<const T*>(w), static_cast<const T*>(b),
                     static_cast<T*>(y), rstd, rows, cols, eps, 1.0f / (float)cols);
}

struct BwdArgs {
  const void *x, *w, *dy;
  const float* rstd;
  void *dx, *dw, *db;
  float *dw_part, *db_part, *stage;
  int64_t rows;
  int cols;
  hipStream_t s;
};

template <typename T, bool BIAS, int NTB, int TPR, int VPT> void launch_bwd_vec(const BwdArgs& a, int64_t blocks) {
  constexpr int RPB = NTB / TPR;
  const size_t lds = RPB > 1 ? (size_t)a.cols * sizeof(float) : 0;
  hipLaunchKernelGGL((rmsnorm_bwd_vec<T, NTB, TPR, VPT, BIAS>), dim3(blocks), dim3(NTB), lds, a.s,
                     static_cast<const T*>(a.x), static_cast<const T*>(a.w), a.rstd, static_cast<const T*>(a.dy),
                     static_cast<T*>(a.dx), a.dw_part, a.db_part, a.rows, a.cols, 1.0f / (float)a.cols);
}

// Every (ntb, tpr, vpt) the planner can return.
#define PK_RMS_FWD_SHAPES(X) X(256, 64, 1) X(256, 64, 2) X(256, 64, 4) X(128, 128, 4) X(256, 256, 4) X(512, 512, 4) \
  X(1024, 1024, 4) X(1024, 1024, 8) X(1024, 1024, 16)
#define PK_RMS_BWD_SHAPES(X) X(256, 64, 1) X(256, 64, 2) X(256, 64, 4) X(256, 256, 2) X(512, 512, 2) \
  X(1024, 1024, 2) X(1024, 1024, 4) X(1024, 1024, 8) X(1024, 1024, 16)

template <typename T, bool BIAS>
int fwd(const void* x, const void* w, const void* b, void* y, float* rstd, int64_t rows, int64_t cols, float eps,
        hipStream_t s) {
  const bool aligned = aligned16(x) && aligned16(w) && aligned16(y) && (!BIAS || aligned16(b));
  const Plan p = plan_for(cols, sizeof(T), aligned, false);
  bool done = false;
#define PK_FWD_CASE(NTB, TPR, VPT)                                                         \
  if (!done && p.vec && p.ntb == NTB && p.tpr == TPR && p.vpt == VPT) {                   \
    launch_fwd_vec<T, BIAS, NTB, TPR, VPT>(rows, x, w, b, y, rstd, (int)cols, eps, s);    \
    done = true;                                                                           \
  }
  PK_RMS_FWD_SHAPES(PK_FWD_CASE)
#undef PK_FWD_CASE
  if (!done)
    hipLaunchKernelGGL((rmsnorm_fwd_any<T, BIAS>), dim3(rows), dim3(kThreads), 0, s, static_cast<const T*>(x),
                       static_cast<const T*>(w), static_cast<const T*>(b), static_cast<T*>(y), rstd, rows,
                       (int)cols, eps, 1.0f / (float)cols);
  return launched("pk_rmsnorm_fwd");
}

// Persistent backward grid: every resident block slot of the device, never
// more blocks than the rows need.
template <typename T, bool BIAS> int64_t bwd_blocks(int64_t rows, const Plan& p) {
  int per_cu = 0;
  int64_t rpb = 1;
#define PK_RES_CASE(NTB, TPR, VPT)                                                         \
  if (!per_cu && p.vec && p.ntb == NTB && p.tpr == TPR && p.vpt == VPT) {                 \
    per_cu = bwd_resident<T, BIAS, NTB, TPR, VPT>(0);                                     \
    rpb = NTB / TPR;                                                                       \
  }
  PK_RMS_BWD_SHAPES(PK_RES_CASE)
#undef PK_RES_CASE
  if (!per_cu) per_cu = bwd_any_resident<T, BIAS>();
  const int64_t want = (rows + rpb - 1) / rpb;
  const int64_t cap = (int64_t)cu_count() * per_cu;
  return want < cap ? want : cap;
}

int64_t stage_rows(int64_t parts) { return (parts + kColSplit - 1) / kColSplit; }

template <typename T> void column_sums(const float* part, float* stage, T* out, int64_t parts, int cols,
                                       hipStream_t s) {
  const int64_t n = stage_rows(parts);
  const int cx = (cols + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(column_sum_stage, dim3(cx, (unsigned)n), dim3(kThreads), 0, s, part, stage, parts, cols);
  hipLaunchKernelGGL(column_sum_final<T>, dim3(cx), dim3(kThreads), 0, s, stage, out, n, cols);
}

template <typename T, bool BIAS> int bwd(const BwdArgs& a) {
  const bool aligned = aligned16(a.x) && aligned16(a.w) && aligned16(a.dy) && aligned16(a.dx);
  const Plan p = plan_for(a.cols, sizeof(T), aligned, true);
  const int64_t blocks = bwd_blocks<T, BIAS>(a.rows, p);
  bool done = false;
#define PK_BWD_CASE(NTB, TPR, VPT)                                                         \
  if (!done && p.vec && p.ntb == NTB && p.tpr == TPR && p.vpt == VPT) {                   \
    launch_bwd_vec<T, BIAS, NTB, TPR, VPT>(a, blocks);                                    \
    done = true;                                                                           \
  }
  PK_RMS_BWD_SHAPES(PK_BWD_CASE)
#undef PK_BWD_CASE
  if (!done)
    hipLaunchKernelGGL((rmsnorm_bwd_any<T, BIAS>), dim3(blocks), dim3(kThreads), 0, a.s, static_cast<const T*>(a.x),
                       static_cast<const T*>(a.w), a.rstd, static_cast<const T*>(a.dy), static_cast<T*>(a.dx),
                       a.dw_part, a.db_part, a.rows, a.cols, 1.0f / (float)a.cols);
  column_sums<T>(a.dw_part, a.stage, static_cast<T*>(a.dw), blocks, a.cols, a.s);
  if (BIAS) column_sums<T>(a.db_part, a.stage, static_cast<T*>(a.db), blocks, a.cols, a.s);
  return launched("pk_rmsnorm_bwd");
}

// Workspace: [blocks, cols] dw partials, the same for dbias, and the
// [stage_rows, cols] first-stage column sums, each rounded up to 256 bytes.
struct Layout {
  int64_t part, stage, total;
};

template <typename T, bool BIAS> Layout layout_for(int64_t rows, int64_t cols) {
  // The aligned plan and the fallback may use different grids: size for the larger.
  const int64_t b1 = bwd_blocks<T, BIAS>(rows, plan_for(cols, sizeof(T), true, true));
  const int64_t b2 = bwd_blocks<T, BIAS>(rows, plan_for(cols, sizeof(T), false, true));
  const int64_t blocks = b1 > b2 ? b1 : b2;
  auto up = [](int64_t n) { return (n + 255) / 256 * 256; };
  Layout l;
  l.part = up(blocks * cols * (int64_t)sizeof(float));
  l.stage = up(stage_rows(blocks) * cols * (int64_t)sizeof(float));
  l.total = l.part * (BIAS ? 2 : 1) + l.stage;
  return l;
}

Layout workspace_layout(int64_t rows, int64_t cols, int dtype, bool bias) {
  switch (dtype) {
    case PK_F32: return bias ? layout_for<float, true>(rows, cols) : layout_for<float, false>(rows, cols);
    case PK_BF16: return bias ? layout_for<bf16, true>(rows, cols) : layout_for<bf16, false>(rows, cols);
    default: return bias ? layout_for<f16, true>(rows, cols) : layout_for<f16, false>(rows, cols);
  }
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
  return workspace_layout(rows, cols, dtype, true).total;
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
  const Layout l = workspace_layout(rows, cols, dtype, b);
  if (workspace_bytes < l.total)
    return fail(PK_ERR_INVALID, "pk_rmsnorm_bwd: workspace of %lld bytes, need %lld", (long long)workspace_bytes,
                (long long)l.total);
  if (!aligned16(workspace)) return fail(PK_ERR_INVALID, "pk_rmsnorm_bwd: workspace not 16-byte aligned");
  char* base = static_cast<char*>(workspace);
  BwdArgs a{x,
            w,
            dy,
            rstd,
            dx,
            dw,
            dbias,
            reinterpret_cast<float*>(base),
            b ? reinterpret_cast<float*>(base + l.part) : nullptr,
            reinterpret_cast<float*>(base + l.part * (b ? 2 : 1)),
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
