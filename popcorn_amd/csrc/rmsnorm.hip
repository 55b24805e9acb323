// RMSNorm forward and backward: row passes that read each operand from HBM
// once.
//
// Fast path (cols a multiple of the 16-byte pack, at most 1024*16 packs): a
// row is held in registers by TPR lanes, each owning VPT packs (contiguous per
// wave in the one-shot forward, else strided by TPR) so a wave's loads are
// contiguous. TPR = 64 is one wavefront per row (several
// rows per block, sum of squares by wave shuffles alone); TPR = NTB is the
// whole block (a wave reduction plus one LDS exchange). Any other shape takes
// a one-block-per-row kernel that loops over the row twice.
//
// Forward launches one block per row group, the even and the odd XCDs each
// sweeping one half of the rows, except for row counts that fit in a few waves
// of resident blocks: there a persistent grid takes rows in grid stride with w
// in registers and the next row prefetched (measured faster on MI355X for such
// short launches, slower for long ones).
//
// Backward is a persistent grid (a few blocks per CU): block b takes rows
// b, b + G, b + 2G, ... (G = grid size; the blocks together sweep the tensors
// front to back, which measured 13% faster than contiguous runs of rows per
// block) with w and its running dw / dbias columns in registers, prefetching
// the next row's x and dy while the current row's dot product is reduced.
// Blocks leave one fp32 partial row each (the rows of a block's wavefront
// slots are combined through LDS first), and a two-stage column reduction
// sums the partials in a fixed order, so dw is deterministic.
//
// Types: T is x's type (and dx's); W is the weight's, which is also the type
// of the bias, of y and of dy, and of dw / dbias: W = T, or fp32 with a 16-bit
// x (torch's promotion of a 16-bit normalised row times an fp32 weight gives
// an fp32 result, unrounded).
#include <math.h>

#include <mutex>

#include "api.h"
#include "colsum.h"
#include "common.h"

namespace pk {
namespace {

constexpr int kThreads = 256;    // fallback kernels and column sums
constexpr int kMaxVpt = 16;

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

// Pack (16-byte vector) of a row held by slot k of `lane` in the one-shot
// forward. A row of one wave interleaves its packs over the lanes; a row
// spanning the block gives wave w the contiguous packs [w*64*VPT,
// (w+1)*64*VPT), each load of a wave then covering 1 KB in order. With the
// XCD split below, 1.5% faster at 65536 x 8192 bf16 than packs interleaved
// over the whole block; the persistent grid kernel keeps the interleaved
// order, which measured 4% faster there (4096 x 4096 fp32).
template <int NTB, int TPR, int VPT> __device__ __forceinline__ int fwd_pack(int lane, int k) {
  if constexpr (TPR == NTB && NTB > 64) return (lane / 64) * (64 * VPT) + k * 64 + lane % 64;
  else return lane + k * TPR;
}

// Row group of block b in a one-shot launch over `units` groups. Dispatch
// places block b on XCD b % 8; the four even XCDs sweep the first 4*qe groups
// and the four odd XCDs the rest, each front to back (qe = ceil(units / 8),
// grid 8*qe). Returns -1 for the few blocks past the end.
__device__ __forceinline__ int64_t xcd_split_unit(int64_t b, int64_t units) {
  const int64_t qe = (units + 7) / 8;
  const int64_t x = b & 7, local = b >> 3;
  const int64_t u = (x & 1) ? 4 * qe + local * 4 + (x >> 1) : local * 4 + (x >> 1);
  return u < units ? u : -1;
}
inline int64_t xcd_split_grid(int64_t units) { return 8 * ((units + 7) / 8); }

// torch: rms = (h * rsqrt(mean(h^2) + eps)).to(T); y = rms * w; y = y + bias.
// Kernel modes: the plain norm, the norm plus bias, and the residual-add form
// (s = x + residual is formed, written out and normalised, with weight + offset).
constexpr int kPlain = 0, kBias = 1, kAdd = 2;

// s = round(x + residual): the sum torch forms at T before normalising it
template <typename T> __device__ __forceinline__ void add_residual(Vec<T>& xv, const Vec<T>& rv) {
#pragma unroll
  for (int j = 0; j < Vec<T>::N; ++j) xv.v[j] = from_f32<T>(to_f32(xv.v[j]) + to_f32(rv.v[j]));
}
// w + offset, rounded to the weight's type like the reference's `weight + offset`
template <typename W, int N> __device__ __forceinline__ Lane<W, N> offset_weight(Lane<W, N> wv, float offset) {
#pragma unroll
  for (int j = 0; j < N; ++j) wv.v[j] = from_f32<W>(to_f32(wv.v[j]) + offset);
  return wv;
}

// torch: n = (h * r).to(T); y = n * w (at W); y = y + bias. With W = T every
// op rounds to T; with W = fp32 only n is rounded.
template <typename T, typename W, bool BIAS> __device__ __forceinline__ W fwd_elem(float xv, float r, float wv, float bv) {
  float y = round_to<T>(xv * r) * wv;
  if constexpr (BIAS) y = round_to<W>(y) + bv;
  return from_f32<W>(y);
}

// One row per TPR lanes, RPB = NTB / TPR rows per block.
template <typename T, typename W, int NTB, int TPR, int VPT, int MODE>
__global__ __launch_bounds__(NTB) void rmsnorm_fwd_vec(const T* __restrict__ x, const W* __restrict__ w,
                                                       const W* __restrict__ bias, const T* __restrict__ res,
                                                       T* __restrict__ s_out, float offset, W* __restrict__ y,
                                                       float* __restrict__ rstd, int64_t rows, int cols, float eps,
                                                       float inv_cols) {
  constexpr bool BIAS = MODE == kBias;
  constexpr int P = Vec<T>::N;
  constexpr int RPB = NTB / TPR;
  __shared__ float red[NTB / 64];
  const int lane = threadIdx.x % TPR;
  const int64_t group = xcd_split_unit(blockIdx.x, (rows + RPB - 1) / RPB);
  if (group < 0) return;  // whole block, before any barrier
  const int64_t row = group * RPB + threadIdx.x / TPR;
  const bool live = row < rows;
  const int nvec = cols / P;
  const T* xr = x + row * cols;

  Vec<T> xv[VPT];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int v = fwd_pack<NTB, TPR, VPT>(lane, k);
    if (live && v < nvec) {
      xv[k] = ld16_stream(xr + v * P);
      if constexpr (MODE == kAdd) {
        add_residual(xv[k], ld16_stream(res + row * cols + v * P));
        st16_stream(s_out + row * cols + v * P, xv[k]);
      }
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

  W* yr = y + row * cols;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int v = fwd_pack<NTB, TPR, VPT>(lane, k);
    if (v < nvec) {
      Lane<W, P> wv = ld_lane<W, P>(w + v * P);
      if constexpr (MODE == kAdd) wv = offset_weight(wv, offset);
      Lane<W, P> bv;
      if constexpr (BIAS) bv = ld_lane<W, P>(bias + v * P);
      Lane<W, P> out;
#pragma unroll
      for (int j = 0; j < P; ++j)
        out.v[j] = fwd_elem<T, W, BIAS>(to_f32(xv[k].v[j]), r, to_f32(wv.v[j]), BIAS ? to_f32(bv.v[j]) : 0.f);
      st_lane_stream(yr + v * P, out);
    }
  }
}

// Persistent form of rmsnorm_fwd_vec for short launches: slot s of block b
// takes rows b * RPB + s + k * stride, with w (and bias) in registers and the
// next row's x in flight while the current row is reduced.
template <typename T, typename W, int NTB, int TPR, int VPT, int MODE>
__global__ __launch_bounds__(NTB) void rmsnorm_fwd_grid(const T* __restrict__ x, const W* __restrict__ w,
                                                        const W* __restrict__ bias, const T* __restrict__ res,
                                                        T* __restrict__ s_out, float offset, W* __restrict__ y,
                                                        float* __restrict__ rstd, int64_t rows, int cols, float eps,
                                                        float inv_cols) {
  constexpr bool BIAS = MODE == kBias;
  constexpr int P = Vec<T>::N;
  constexpr int RPB = NTB / TPR;
  __shared__ float red[NTB / 64];
  const int lane = threadIdx.x % TPR;
  const int nvec = cols / P;
  const int64_t stride = (int64_t)gridDim.x * RPB;
  const int64_t first = (int64_t)blockIdx.x * RPB;
  const int64_t row0 = first + threadIdx.x / TPR;
  const int64_t trips = (rows - first + stride - 1) / stride;  // the same for every slot: barriers line up
  Lane<W, P> wv[VPT], bv[VPT];
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int v = lane + k * TPR;
    if (v < nvec) {
      wv[k] = ld_lane<W, P>(w + v * P);
      if constexpr (MODE == kAdd) wv[k] = offset_weight(wv[k], offset);
      if constexpr (BIAS) bv[k] = ld_lane<W, P>(bias + v * P);
    }
  }
  Vec<T> xv[VPT], xn[VPT];
  Vec<T> rv[MODE == kAdd ? VPT : 1], rn[MODE == kAdd ? VPT : 1];
  auto fetch = [&](int64_t row, Vec<T>* xo, Vec<T>* ro) {
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int v = lane + k * TPR;
      if (row < rows && v < nvec) {
        xo[k] = ld16_stream(x + row * cols + v * P);
        if constexpr (MODE == kAdd) ro[k] = ld16_stream(res + row * cols + v * P);
      }
    }
  };
  fetch(row0, xv, rv);
  for (int64_t t = 0; t < trips; ++t) {
    const int64_t row = row0 + t * stride;
    fetch(row + stride, xn, rn);
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int v = lane + k * TPR;
      if (row < rows && v < nvec) {
        if constexpr (MODE == kAdd) {
          add_residual(xv[k], rv[k]);
          st16_stream(s_out + row * cols + v * P, xv[k]);
        }
#pragma unroll
        for (int j = 0; j < P; ++j) {
          const float f = to_f32(xv[k].v[j]);
          ss += f * f;
        }
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
          Lane<W, P> out;
#pragma unroll
          for (int j = 0; j < P; ++j)
            out.v[j] = fwd_elem<T, W, BIAS>(to_f32(xv[k].v[j]), r, to_f32(wv[k].v[j]), BIAS ? to_f32(bv[k].v[j]) : 0.f);
          st_lane_stream(y + row * cols + v * P, out);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      xv[k] = xn[k];
      if constexpr (MODE == kAdd) rv[k] = rn[k];
    }
  }
}

// Any row width, any alignment: one block per row, two passes over x.
template <typename T, typename W, int MODE>
__global__ __launch_bounds__(kThreads) void rmsnorm_fwd_any(const T* __restrict__ x, const W* __restrict__ w,
                                                            const W* __restrict__ bias, const T* __restrict__ res,
                                                            T* __restrict__ s_out, float offset, W* __restrict__ y,
                                                            float* __restrict__ rstd, int64_t rows, int cols,
                                                            float eps, float inv_cols) {
  constexpr bool BIAS = MODE == kBias;
  __shared__ float red[kThreads / 64];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * cols;
  float ss = 0.f;
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    float f = to_f32(xr[c]);
    if constexpr (MODE == kAdd) {
      const T sv = from_f32<T>(f + to_f32(res[row * cols + c]));
      s_out[row * cols + c] = sv;  // re-read below by this same thread
      f = to_f32(sv);
    }
    ss += f * f;
  }
  ss = row_sum<kThreads, kThreads>(ss, red);
  const float r = 1.0f / sqrtf(ss * inv_cols + eps);
  if (rstd != nullptr && threadIdx.x == 0) rstd[row] = r;
  W* yr = y + row * cols;
  const T* sr = MODE == kAdd ? s_out + row * cols : xr;
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    const float wv = MODE == kAdd ? to_f32(from_f32<W>(to_f32(w[c]) + offset)) : to_f32(w[c]);
    yr[c] = fwd_elem<T, W, BIAS>(to_f32(sr[c]), r, wv, BIAS ? to_f32(bias[c]) : 0.f);
  }
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

// MODE kAdd: x is the residual sum s, w is used as w + offset, and ds (the
// gradient reaching s from its second use, may be NULL) is added to dx.
template <typename T, typename W, int NTB, int TPR, int VPT, int MODE>
__global__ __launch_bounds__(NTB) void rmsnorm_bwd_vec(const T* __restrict__ x, const W* __restrict__ w,
                                                       const float* __restrict__ rstd, const W* __restrict__ dy,
                                                       const T* __restrict__ ds, float offset, T* __restrict__ dx,
                                                       float* __restrict__ dw_part, float* __restrict__ db_part,
                                                       int64_t rows, int cols, float inv_cols) {
  constexpr bool BIAS = MODE == kBias;
  constexpr bool ADD = MODE == kAdd;
  const bool has_ds = ADD && ds != nullptr;
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
    Lane<W, P> wv;
    if (v < nvec) wv = ld_lane<W, P>(w + v * P);
    if constexpr (ADD) wv = offset_weight(wv, offset);
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

  Vec<T> xv[VPT], xn[VPT];
  Lane<W, P> gv[VPT], gn[VPT];
  Vec<T> sv[ADD ? VPT : 1], sn[ADD ? VPT : 1];
  auto fetch = [&](int64_t row, Vec<T>* xo, Lane<W, P>* go, Vec<T>* so) {
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int v = lane + k * TPR;
      if (row < rows && v < nvec) {
        xo[k] = ld16_stream(x + row * cols + v * P);
        go[k] = ld_lane_stream<W, P>(dy + row * cols + v * P);
        if (has_ds) so[k] = ld16_stream(ds + row * cols + v * P);
      }
    }
  };
  fetch(row0 + slot, xv, gv, sv);

  for (int64_t t = 0; t < trips; ++t) {
    const int64_t row = row0 + slot + t * stride;
    const bool live = row < rows;
    fetch(row + stride, xn, gn, sn);  // next row of this slot, in flight during the reduction
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
            float d = r * (g * wf[k][j] - n * dot);
            if constexpr (ADD) d += has_ds ? to_f32(sv[k].v[j]) : 0.f;
            out.v[j] = from_f32<T>(d);
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
      if constexpr (ADD) sv[k] = sn[k];
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
template <typename T, typename W, int MODE>
__global__ __launch_bounds__(kThreads) void rmsnorm_bwd_any(const T* __restrict__ x, const W* __restrict__ w,
                                                            const float* __restrict__ rstd,
                                                            const W* __restrict__ dy, const T* __restrict__ ds,
                                                            float offset, T* __restrict__ dx,
                                                            float* __restrict__ dw_part,
                                                            float* __restrict__ db_part, int64_t rows, int cols,
                                                            float inv_cols) {
  constexpr bool BIAS = MODE == kBias;
  constexpr bool ADD = MODE == kAdd;
  const bool has_ds = ADD && ds != nullptr;
  // weight as the forward used it: w, or w + offset rounded to its type
  auto wc = [&](int c) { return ADD ? to_f32(from_f32<W>(to_f32(w[c]) + offset)) : to_f32(w[c]); };
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
    const W* gr = dy + row * cols;
    float dot = 0.f;
    for (int c = threadIdx.x; c < cols; c += kThreads) dot += to_f32(gr[c]) * wc(c) * (to_f32(xr[c]) * r);
    dot = row_sum<kThreads, kThreads>(dot, red) * inv_cols;
    T* dxr = dx + row * cols;
    for (int c = threadIdx.x; c < cols; c += kThreads) {
      const float g = to_f32(gr[c]);
      const float n = to_f32(xr[c]) * r;
      float d = r * (g * wc(c) - n * dot);
      if (has_ds) d += to_f32(ds[row * cols + c]);
      dxr[c] = from_f32<T>(d);
      dwp[c] += g * n;  // column c is only ever touched by this thread
      if constexpr (BIAS) dbp[c] += g;
    }
  }
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

template <typename T, typename W, int MODE, int NTB, int TPR, int VPT> int bwd_resident() {
  // dynamic LDS of a 4-rows-per-block shape: one fp32 row of at most 64*4*8 columns
  static const int n = resident_per_cu(rmsnorm_bwd_vec<T, W, NTB, TPR, VPT, MODE>, NTB,
                                       NTB / TPR > 1 ? (size_t)64 * 4 * 8 * sizeof(float) : 0);
  return n;
}

template <typename T, typename W, int MODE> int bwd_any_resident() {
  static const int n = resident_per_cu(rmsnorm_bwd_any<T, W, MODE>, kThreads, 0);
  return n;
}

struct FwdArgs {
  const void *x, *w, *b, *res;
  void* s_out;
  float offset;
  void* y;
  float* rstd;
  int64_t rows;
  int cols;
  float eps;
  hipStream_t s;
};

template <typename T, typename W, int MODE, int NTB, int TPR, int VPT> void launch_fwd_vec(const FwdArgs& a) {
  constexpr int RPB = NTB / TPR;
  const int64_t groups = (a.rows + RPB - 1) / RPB;
  const T *x = static_cast<const T*>(a.x), *res = static_cast<const T*>(a.res);
  const W *w = static_cast<const W*>(a.w), *b = static_cast<const W*>(a.b);
  T* s_out = static_cast<T*>(a.s_out);
  W* y = static_cast<W*>(a.y);
  // Up to four waves of resident blocks: the persistent grid.
  static const int per_cu = resident_per_cu(rmsnorm_fwd_vec<T, W, NTB, TPR, VPT, MODE>, NTB, 0);
  static const int per_cu_grid = resident_per_cu(rmsnorm_fwd_grid<T, W, NTB, TPR, VPT, MODE>, NTB, 0);
  if (groups <= (int64_t)4 * cu_count() * per_cu) {
    const int64_t slots = (int64_t)cu_count() * per_cu_grid;
    hipLaunchKernelGGL((rmsnorm_fwd_grid<T, W, NTB, TPR, VPT, MODE>), dim3(groups < slots ? groups : slots), dim3(NTB),
                       0, a.s, x, w, b, res, s_out, a.offset, y, a.rstd, a.rows, a.cols, a.eps, 1.0f / (float)a.cols);
    return;
  }
  hipLaunchKernelGGL((rmsnorm_fwd_vec<T, W, NTB, TPR, VPT, MODE>), dim3(xcd_split_grid(groups)), dim3(NTB), 0, a.s, x,
                     w, b, res, s_out, a.offset, y, a.rstd, a.rows, a.cols, a.eps, 1.0f / (float)a.cols);
}

struct BwdArgs {
  const void *x, *w, *dy, *ds;
  float offset;
  const float* rstd;
  void *dx, *dw, *db;
  float *dw_part, *db_part, *stage;
  int64_t rows;
  int cols;
  hipStream_t s;
};

template <typename T, typename W, int MODE, int NTB, int TPR, int VPT>
void launch_bwd_vec(const BwdArgs& a, int64_t blocks) {
  constexpr int RPB = NTB / TPR;
  const size_t lds = RPB > 1 ? (size_t)a.cols * sizeof(float) : 0;
  hipLaunchKernelGGL((rmsnorm_bwd_vec<T, W, NTB, TPR, VPT, MODE>), dim3(blocks), dim3(NTB), lds, a.s,
                     static_cast<const T*>(a.x), static_cast<const W*>(a.w), a.rstd, static_cast<const W*>(a.dy),
                     static_cast<const T*>(a.ds), a.offset, static_cast<T*>(a.dx), a.dw_part, a.db_part, a.rows,
                     a.cols, 1.0f / (float)a.cols);
}

// Every (ntb, tpr, vpt) the planner can return.
#define PK_RMS_FWD_SHAPES(X) X(256, 64, 1) X(256, 64, 2) X(256, 64, 4) X(128, 128, 4) X(256, 256, 4) X(512, 512, 4) \
  X(1024, 1024, 4) X(1024, 1024, 8) X(1024, 1024, 16)
#define PK_RMS_BWD_SHAPES(X) X(256, 64, 1) X(256, 64, 2) X(256, 64, 4) X(256, 256, 2) X(512, 512, 2) \
  X(1024, 1024, 2) X(1024, 1024, 4) X(1024, 1024, 8) X(1024, 1024, 16)

template <typename T, typename W, int MODE> int fwd(const FwdArgs& a, const char* who) {
  const bool aligned = aligned16(a.x) && aligned16(a.w) && aligned16(a.y) && (MODE != kBias || aligned16(a.b)) &&
                       (MODE != kAdd || (aligned16(a.res) && aligned16(a.s_out)));
  const Plan p = plan_for(a.cols, sizeof(T), aligned, false);
  bool done = false;
#define PK_FWD_CASE(NTB, TPR, VPT)                                                         \
  if (!done && p.vec && p.ntb == NTB && p.tpr == TPR && p.vpt == VPT) {                   \
    launch_fwd_vec<T, W, MODE, NTB, TPR, VPT>(a);                                         \
    done = true;                                                                           \
  }
  PK_RMS_FWD_SHAPES(PK_FWD_CASE)
#undef PK_FWD_CASE
  if (!done)
    hipLaunchKernelGGL((rmsnorm_fwd_any<T, W, MODE>), dim3(a.rows), dim3(kThreads), 0, a.s,
                       static_cast<const T*>(a.x), static_cast<const W*>(a.w), static_cast<const W*>(a.b),
                       static_cast<const T*>(a.res), static_cast<T*>(a.s_out), a.offset, static_cast<W*>(a.y),
                       a.rstd, a.rows, a.cols, a.eps, 1.0f / (float)a.cols);
  return launched(who);
}

// Persistent backward grid: every resident block slot of the device, never
// more blocks than the rows need.
template <typename T, typename W, int MODE> int64_t bwd_blocks(int64_t rows, const Plan& p) {
  int per_cu = 0;
  int64_t rpb = 1;
#define PK_RES_CASE(NTB, TPR, VPT)                                                         \
  if (!per_cu && p.vec && p.ntb == NTB && p.tpr == TPR && p.vpt == VPT) {                 \
    per_cu = bwd_resident<T, W, MODE, NTB, TPR, VPT>();                                   \
    rpb = NTB / TPR;                                                                       \
  }
  PK_RMS_BWD_SHAPES(PK_RES_CASE)
#undef PK_RES_CASE
  if (!per_cu) per_cu = bwd_any_resident<T, W, MODE>();
  const int64_t want = (rows + rpb - 1) / rpb;
  const int64_t cap = (int64_t)cu_count() * per_cu;
  return want < cap ? want : cap;
}

template <typename T, typename W, int MODE> int bwd(const BwdArgs& a, const char* who) {
  const bool aligned = aligned16(a.x) && aligned16(a.w) && aligned16(a.dy) && aligned16(a.dx) &&
                       (a.ds == nullptr || aligned16(a.ds));
  const Plan p = plan_for(a.cols, sizeof(T), aligned, true);
  const int64_t blocks = bwd_blocks<T, W, MODE>(a.rows, p);
  bool done = false;
#define PK_BWD_CASE(NTB, TPR, VPT)                                                         \
  if (!done && p.vec && p.ntb == NTB && p.tpr == TPR && p.vpt == VPT) {                   \
    launch_bwd_vec<T, W, MODE, NTB, TPR, VPT>(a, blocks);                                 \
    done = true;                                                                           \
  }
  PK_RMS_BWD_SHAPES(PK_BWD_CASE)
#undef PK_BWD_CASE
  if (!done)
    hipLaunchKernelGGL((rmsnorm_bwd_any<T, W, MODE>), dim3(blocks), dim3(kThreads), 0, a.s,
                       static_cast<const T*>(a.x), static_cast<const W*>(a.w), a.rstd, static_cast<const W*>(a.dy),
                       static_cast<const T*>(a.ds), a.offset, static_cast<T*>(a.dx), a.dw_part, a.db_part, a.rows,
                       a.cols, 1.0f / (float)a.cols);
  column_sums<W>(a.dw_part, a.stage, static_cast<W*>(a.dw), blocks, a.cols, a.s);
  if (MODE == kBias) column_sums<W>(a.db_part, a.stage, static_cast<W*>(a.db), blocks, a.cols, a.s);
  return launched(who);
}

// Workspace: [blocks, cols] dw partials, the same for dbias, and the
// [stage_rows, cols] first-stage column sums, each rounded up to 256 bytes.
struct Layout {
  int64_t part, stage, total;
};

template <typename T, typename W, int MODE> Layout layout_for(int64_t rows, int64_t cols) {
  // The aligned plan and the fallback may use different grids: size for the larger.
  const int64_t b1 = bwd_blocks<T, W, MODE>(rows, plan_for(cols, sizeof(T), true, true));
  const int64_t b2 = bwd_blocks<T, W, MODE>(rows, plan_for(cols, sizeof(T), false, true));
  const int64_t blocks = b1 > b2 ? b1 : b2;
  auto up = [](int64_t n) { return (n + 255) / 256 * 256; };
  Layout l;
  l.part = up(blocks * cols * (int64_t)sizeof(float));
  l.stage = up(stage_rows(blocks) * cols * (int64_t)sizeof(float));
  l.total = l.part * (MODE == kBias ? 2 : 1) + l.stage;
  return l;
}

// (x dtype, weight dtype) pairs the kernels implement, in every mode: one
// dtype, or a 16-bit x (with its residual and sum, in the residual-add mode)
// with an fp32 weight.
bool supported_pair(int dtype, int wdtype, int /*mode*/) {
  if (wdtype == dtype) return known_dtype(dtype);
  return wdtype == PK_F32 && (dtype == PK_BF16 || dtype == PK_F16);
}

template <int MODE> Layout layout_of(int64_t rows, int64_t cols, int dtype, int wdtype) {
  if (wdtype != dtype) return dtype == PK_BF16 ? layout_for<bf16, float, MODE>(rows, cols)
                                               : layout_for<f16, float, MODE>(rows, cols);
  switch (dtype) {
    case PK_F32: return layout_for<float, float, MODE>(rows, cols);
    case PK_BF16: return layout_for<bf16, bf16, MODE>(rows, cols);
    default: return layout_for<f16, f16, MODE>(rows, cols);
  }
}

Layout workspace_layout(int64_t rows, int64_t cols, int dtype, int wdtype, int mode) {
  return mode == kBias ? layout_of<kBias>(rows, cols, dtype, wdtype)
                       : mode == kAdd ? layout_of<kAdd>(rows, cols, dtype, wdtype)
                                      : layout_of<kPlain>(rows, cols, dtype, wdtype);
}

// One workspace size serves every backward entry point, mode and weight dtype.
int64_t workspace_bytes(int64_t rows, int64_t cols, int dtype) {
  int64_t n = 0;
  for (int wdtype : {dtype, (int)PK_F32})
    for (int mode : {kPlain, kBias, kAdd}) {
      if (!supported_pair(dtype, wdtype, mode)) continue;
      const int64_t t = workspace_layout(rows, cols, dtype, wdtype, mode).total;
      n = t > n ? t : n;
    }
  return n;
}

template <int MODE> int fwd_dispatch(const FwdArgs& a, int dtype, int wdtype, const char* who) {
  if (wdtype != dtype) return dtype == PK_BF16 ? fwd<bf16, float, MODE>(a, who) : fwd<f16, float, MODE>(a, who);
  switch (dtype) {
    case PK_F32: return fwd<float, float, MODE>(a, who);
    case PK_BF16: return fwd<bf16, bf16, MODE>(a, who);
    default: return fwd<f16, f16, MODE>(a, who);
  }
}

template <int MODE> int bwd_dispatch(const BwdArgs& a, int dtype, int wdtype, const char* who) {
  if (wdtype != dtype) return dtype == PK_BF16 ? bwd<bf16, float, MODE>(a, who) : bwd<f16, float, MODE>(a, who);
  switch (dtype) {
    case PK_F32: return bwd<float, float, MODE>(a, who);
    case PK_BF16: return bwd<bf16, bf16, MODE>(a, who);
    default: return bwd<f16, f16, MODE>(a, who);
  }
}

// Splits the caller's workspace for a backward call of this mode.
int carve(const char* who, void* workspace, int64_t workspace_bytes, int64_t rows, int64_t cols, int dtype,
          int wdtype, int mode, BwdArgs& a) {
  const Layout l = workspace_layout(rows, cols, dtype, wdtype, mode);
  if (workspace_bytes < l.total)
    return fail(PK_ERR_INVALID, "%s: workspace of %lld bytes, need %lld", who, (long long)workspace_bytes,
                (long long)l.total);
  if (!aligned16(workspace)) return fail(PK_ERR_INVALID, "%s: workspace not 16-byte aligned", who);
  char* base = static_cast<char*>(workspace);
  a.dw_part = reinterpret_cast<float*>(base);
  a.db_part = mode == kBias ? reinterpret_cast<float*>(base + l.part) : nullptr;
  a.stage = reinterpret_cast<float*>(base + l.part * (mode == kBias ? 2 : 1));
  return PK_OK;
}

int check_shape(const char* who, int64_t rows, int64_t cols, int dtype, int wdtype = -1, int mode = kPlain) {
  if (rows < 0 || cols < 0) return fail(PK_ERR_INVALID, "%s: negative shape (%lld, %lld)", who, (long long)rows,
                                        (long long)cols);
  if (cols > (int64_t)1 << 30) return fail(PK_ERR_UNSUPPORTED, "%s: %lld columns", who, (long long)cols);
  if (!known_dtype(dtype)) return fail(PK_ERR_UNSUPPORTED, "%s: dtype code %d", who, dtype);
  if (!supported_pair(dtype, wdtype < 0 ? dtype : wdtype, mode))
    return fail(PK_ERR_UNSUPPORTED, "%s: x dtype code %d with weight dtype code %d (one dtype, or a 16-bit x with an "
                "fp32 weight)", who, dtype, wdtype);
  return PK_OK;
}

}  // namespace
}  // namespace pk

// ---------------------------------------------------------------------------
// Fixed scratch for pk_rmsnorm_bwd_noalloc: the dw / dbias partial rows and
// the column-sum stage of one backward call. Every GPU the library runs on
// holds its own copy from module load until the process ends. Each block
// writes its whole partial row and the first column-sum stage writes every
// stage row it covers, so nothing needs clearing between calls; two calls that
// overlap on one GPU (on different streams, or from different threads) share
// the array and race.
static constexpr int64_t kScratchBytes = (int64_t)96 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace pk {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void* g_scratch_addr[kMaxDevices];  // device address of `scratch` per device, once looked up

// Device address of the current device's scratch array. The array's host-side
// name is only a stand-in for the symbol: its device address is looked up
// once per device with that device current and kept.
int scratch_address(const char* who, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(PK_ERR_HIP, "%s: no current HIP device", who);
  std::lock_guard<std::mutex> hold(g_scratch_lock);
  if (g_scratch_addr[dev] == nullptr) {
    void* addr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || addr == nullptr)
      return fail(PK_ERR_HIP, "%s: hipGetSymbolAddress(scratch) on device %d failed: %s", who, dev,
                  hipGetErrorString(err));
    g_scratch_addr[dev] = addr;
  }
  *out = g_scratch_addr[dev];
  return PK_OK;
}

}  // namespace
}  // namespace pk

extern "C" {

int pk_rmsnorm_fwd(const void* x, const void* w, const void* bias, void* y, float* rstd, int64_t rows, int64_t cols,
                   float eps, int dtype, int w_dtype, void* stream) {
  using namespace pk;
  if (int st = check_shape("pk_rmsnorm_fwd", rows, cols, dtype, w_dtype)) return st;
  if (rows == 0) return PK_OK;
  if (cols == 0) return fail(PK_ERR_INVALID, "pk_rmsnorm_fwd: zero-width rows");
  if (!x || !w || !y) return fail(PK_ERR_INVALID, "pk_rmsnorm_fwd: null pointer");
  const FwdArgs a{x, w, bias, nullptr, nullptr, 0.f, y, rstd, rows, (int)cols, eps, static_cast<hipStream_t>(stream)};
  return bias != nullptr ? fwd_dispatch<kBias>(a, dtype, w_dtype, "pk_rmsnorm_fwd")
                         : fwd_dispatch<kPlain>(a, dtype, w_dtype, "pk_rmsnorm_fwd");
}

int64_t pk_rmsnorm_bwd_workspace(int64_t rows, int64_t cols, int dtype) {
  using namespace pk;
  if (rows <= 0 || cols <= 0 || !known_dtype(dtype)) return 0;
  return workspace_bytes(rows, cols, dtype);
}

int pk_rmsnorm_bwd(const void* x, const void* w, const float* rstd, const void* dy, void* dx, void* dw, void* dbias,
                   void* workspace, int64_t workspace_bytes, int64_t rows, int64_t cols, int dtype, int w_dtype,
                   void* stream) {
  using namespace pk;
  const char* who = "pk_rmsnorm_bwd";
  if (int st = check_shape(who, rows, cols, dtype, w_dtype)) return st;
  if (cols == 0) return fail(PK_ERR_INVALID, "pk_rmsnorm_bwd: zero-width rows");
  if (!x || !w || !rstd || !dy || !dx || !dw || !workspace)
    return fail(PK_ERR_INVALID, "pk_rmsnorm_bwd: null pointer");
  if (rows == 0) return fail(PK_ERR_UNSUPPORTED, "pk_rmsnorm_bwd: zero rows (dw is all zeros; fill it host-side)");
  const int mode = dbias != nullptr ? kBias : kPlain;
  BwdArgs a{x, w, dy, nullptr, 0.f, rstd, dx, dw, dbias, nullptr, nullptr, nullptr, rows, (int)cols,
            static_cast<hipStream_t>(stream)};
  if (int st = carve(who, workspace, workspace_bytes, rows, cols, dtype, w_dtype, mode, a)) return st;
  return mode == kBias ? bwd_dispatch<kBias>(a, dtype, w_dtype, who) : bwd_dispatch<kPlain>(a, dtype, w_dtype, who);
}

int pk_rmsnorm_bwd_noalloc(const void* x, const void* w, const float* rstd, const void* dy, void* dx, void* dw,
                           void* dbias, int64_t rows, int64_t cols, int dtype, int w_dtype, void* stream) {
  using namespace pk;
  const char* who = "pk_rmsnorm_bwd_noalloc";
  if (int st = check_shape(who, rows, cols, dtype, w_dtype)) return st;
  if (cols == 0) return fail(PK_ERR_INVALID, "%s: zero-width rows", who);
  if (rows == 0) return fail(PK_ERR_UNSUPPORTED, "%s: zero rows (dw is all zeros; fill it host-side)", who);
  // The size limit is checked before the pointers, so a caller can probe it
  // with null pointers: a call past the limit then never reaches a launch,
  // even if this check were wrong (the null check below refuses it).
  const int mode = dbias != nullptr ? kBias : kPlain;
  const int64_t need = workspace_layout(rows, cols, dtype, w_dtype, mode).total;
  if (need > kScratchBytes)
    return fail(PK_ERR_UNSUPPORTED, "%s: shape (%lld, %lld) needs %lld bytes of scratch, the fixed array holds %lld",
                who, (long long)rows, (long long)cols, (long long)need, (long long)kScratchBytes);
  if (!x || !w || !rstd || !dy || !dx || !dw) return fail(PK_ERR_INVALID, "%s: null pointer", who);
  void* base = nullptr;
  if (int st = scratch_address(who, &base)) return st;
  BwdArgs a{x, w, dy, nullptr, 0.f, rstd, dx, dw, dbias, nullptr, nullptr, nullptr, rows, (int)cols,
            static_cast<hipStream_t>(stream)};
  if (int st = carve(who, base, kScratchBytes, rows, cols, dtype, w_dtype, mode, a)) return st;
  return mode == kBias ? bwd_dispatch<kBias>(a, dtype, w_dtype, who) : bwd_dispatch<kPlain>(a, dtype, w_dtype, who);
}

int pk_add_rmsnorm_fwd(const void* x, const void* residual, const void* w, void* y, void* s, float* rstd,
                       int64_t rows, int64_t cols, float eps, float offset, int dtype, int w_dtype, void* stream) {
  using namespace pk;
  const char* who = "pk_add_rmsnorm_fwd";
  if (int st = check_shape(who, rows, cols, dtype, w_dtype, kAdd)) return st;
  if (rows == 0) return PK_OK;
  if (cols == 0) return fail(PK_ERR_INVALID, "pk_add_rmsnorm_fwd: zero-width rows");
  if (!x || !residual || !w || !y || !s) return fail(PK_ERR_INVALID, "pk_add_rmsnorm_fwd: null pointer");
  if (!isfinite(offset)) return fail(PK_ERR_INVALID, "pk_add_rmsnorm_fwd: offset is not finite");
  const FwdArgs a{x, w, nullptr, residual, s, offset, y, rstd, rows, (int)cols, eps, static_cast<hipStream_t>(stream)};
  return fwd_dispatch<kAdd>(a, dtype, w_dtype, who);
}

int pk_add_rmsnorm_bwd(const void* s, const void* w, const float* rstd, const void* dy, const void* ds, void* dx,
                       void* dw, void* workspace, int64_t workspace_bytes, int64_t rows, int64_t cols, float offset,
                       int dtype, int w_dtype, void* stream) {
  using namespace pk;
  const char* who = "pk_add_rmsnorm_bwd";
  if (int st = check_shape(who, rows, cols, dtype, w_dtype, kAdd)) return st;
  if (cols == 0) return fail(PK_ERR_INVALID, "pk_add_rmsnorm_bwd: zero-width rows");
  if (!s || !w || !rstd || !dy || !dx || !dw || !workspace)
    return fail(PK_ERR_INVALID, "pk_add_rmsnorm_bwd: null pointer");
  if (rows == 0) return fail(PK_ERR_UNSUPPORTED, "pk_add_rmsnorm_bwd: zero rows (dw is all zeros; fill it host-side)");
  if (!isfinite(offset)) return fail(PK_ERR_INVALID, "pk_add_rmsnorm_bwd: offset is not finite");
  BwdArgs a{s, w, dy, ds, offset, rstd, dx, dw, nullptr, nullptr, nullptr, nullptr, rows, (int)cols,
            static_cast<hipStream_t>(stream)};
  if (int st = carve(who, workspace, workspace_bytes, rows, cols, dtype, w_dtype, kAdd, a)) return st;
  return bwd_dispatch<kAdd>(a, dtype, w_dtype, who);
}

}  // extern "C"
