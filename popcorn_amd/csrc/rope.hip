// Paired rotary embedding of q [batch, q_heads, seq, head_dim] and
// k [batch, kv_heads, seq, head_dim] with full-width tables
// cos, sin [cos_batch, seq, head_dim] (cos_batch 1 or batch), in one launch:
//
//   y[j]     = x[j]     cos[j]     - x[j + h] sin[j]        (j < h = head_dim/2)
//   y[j + h] = x[j + h] cos[j + h] + x[j]     sin[j + h]
//
// i.e. x cos + rotate_half(x) sin with rotate_half(x) = (-x2, x1); the
// transpose (the backward) is dx[j] = dy[j] cos[j] + dy[j + h] sin[j + h],
// dx[j + h] = dy[j + h] cos[j + h] - dy[j] sin[j]. The two halves of a table
// row need not be equal. Arithmetic is fp32 with one rounding per output.
// Inputs and outputs may differ in type: 16-bit q/k with fp32 tables give fp32
// outputs (torch's promotion), whose backward reads fp32 cotangents and writes
// 16-bit gradients.
//
// A block takes a tile of positions of one batch row and a group of heads
// (q heads first, then k heads); a thread owns one (position, chunk) of the
// tile, a chunk being VEC consecutive pairs (one 16-byte access of each half
// when they fill it). It loads its cos/sin values once into registers and
// then streams its chunk of every head of the group, U heads' loads in flight
// at a time, so table reads are amortised over the group instead of repeated
// per head. Consecutive threads take consecutive chunks, then positions: a
// wave streams contiguous rows of one head.
#include "api.h"
#include "colsum.h"
#include "common.h"

namespace pk {
namespace {

constexpr int kThreads = 256;

struct RopeArgs {
  const void* x[2];
  void* y[2];
  int64_t xs[2][3], ys[2][3];  // (batch, head, seq) strides of q, k and of their outputs
  int heads[2];
  int batch, seq, half, cos_batch;
  int chunks;  // chunks per row (half / VEC)
  int rows;    // positions per block tile
  int tiles;   // tiles per batch row, ceil(seq / rows)
  int group;   // heads per block (of q_heads + kv_heads)
};

// VEC elements of T: whole 16-byte non-temporal accesses when they fill them
// (one or two, when a wider type lines up with a 16-bit one), else elements.
template <typename T, int VEC> struct alignas(16) Pack {
  static constexpr bool kWhole = VEC * sizeof(T) % 16 == 0;
  T v[VEC];
  __device__ __forceinline__ void load(const T* p) {
    if constexpr (kWhole) {
#pragma unroll
      for (int i = 0; i < (int)(VEC * sizeof(T) / 16); ++i)
        reinterpret_cast<u32x4*>(v)[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p) + i);
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) v[j] = p[j];
    }
  }
  __device__ __forceinline__ void store(T* p) const {
    if constexpr (kWhole) {
#pragma unroll
      for (int i = 0; i < (int)(VEC * sizeof(T) / 16); ++i)
        __builtin_nontemporal_store(reinterpret_cast<const u32x4*>(v)[i], reinterpret_cast<u32x4*>(p) + i);
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) p[j] = v[j];
    }
  }
};

// table values as fp32, cacheable loads (reused across heads)
template <typename C, int N> __device__ __forceinline__ void table(const C* p, float (&out)[N]) {
  if constexpr (N * sizeof(C) % 16 == 0) {
    constexpr int PER = 16 / sizeof(C);
#pragma unroll
    for (int i = 0; i < N; i += PER) {
      const uint4 raw = *reinterpret_cast<const uint4*>(p + i);
      const C* e = reinterpret_cast<const C*>(&raw);
#pragma unroll
      for (int j = 0; j < PER; ++j) out[i + j] = to_f32(e[j]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) out[j] = to_f32(p[j]);
  }
}

template <typename TI, typename TO, typename C, int VEC, int U, bool TRANSPOSE>
__global__ __launch_bounds__(kThreads) void rope_kernel(const C* __restrict__ cosp, const C* __restrict__ sinp,
                                                        RopeArgs a) {
  // block -> (head group, batch, tile); consecutive blocks take consecutive tiles
  unsigned blk = blockIdx.x;
  const int tile = (int)(blk % (unsigned)a.tiles);
  blk /= (unsigned)a.tiles;
  const int b = (int)(blk % (unsigned)a.batch);
  const int h_begin = (int)(blk / (unsigned)a.batch) * a.group;
  const int all_heads = a.heads[0] + a.heads[1];
  const int h_end = h_begin + a.group < all_heads ? h_begin + a.group : all_heads;
  const int64_t hd = 2 * (int64_t)a.half;
  const int64_t tb = (int64_t)(a.cos_batch == 1 ? 0 : b) * a.seq * hd;
  const int per_tile = a.rows * a.chunks;
  for (int it = threadIdx.x; it < per_tile; it += kThreads) {
    const int r = it / a.chunks;
    const int j = (it - r * a.chunks) * VEC;
    const int s = tile * a.rows + r;
    if (s >= a.seq) break;
    const int64_t trow = tb + (int64_t)s * hd + j;
    float c1[VEC], c2[VEC], s1[VEC], s2[VEC];
    table(cosp + trow, c1);
    table(cosp + trow + a.half, c2);
    table(sinp + trow, s1);
    table(sinp + trow + a.half, s2);
    // this chunk's element offset at head 0 of q (side 0) and k (side 1)
    const int64_t xo[2] = {b * a.xs[0][0] + s * a.xs[0][2] + j, b * a.xs[1][0] + s * a.xs[1][2] + j};
    const int64_t yo[2] = {b * a.ys[0][0] + s * a.ys[0][2] + j, b * a.ys[1][0] + s * a.ys[1][2] + j};
    for (int hh = h_begin; hh < h_end; hh += U) {
      Pack<TI, VEC> x1[U], x2[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int g = hh + u;
        if (g >= h_end) break;
        const int t = g >= a.heads[0];
        const int h = t ? g - a.heads[0] : g;
        const TI* xr = static_cast<const TI*>(a.x[t]) + xo[t] + h * a.xs[t][1];
        x1[u].load(xr);
        x2[u].load(xr + a.half);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int g = hh + u;
        if (g >= h_end) break;
        const int t = g >= a.heads[0];
        const int h = t ? g - a.heads[0] : g;
        Pack<TO, VEC> y1, y2;
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
          const float p = to_f32(x1[u].v[k]), q = to_f32(x2[u].v[k]);
          if constexpr (!TRANSPOSE) {
            y1.v[k] = from_f32<TO>(p * c1[k] - q * s1[k]);
            y2.v[k] = from_f32<TO>(q * c2[k] + p * s2[k]);
          } else {
            y1.v[k] = from_f32<TO>(p * c1[k] + q * s2[k]);
            y2.v[k] = from_f32<TO>(q * c2[k] - p * s1[k]);
          }
        }
        TO* yr = static_cast<TO*>(a.y[t]) + yo[t] + h * a.ys[t][1];
        y1.store(yr);
        y2.store(yr + a.half);
      }
    }
  }
}

template <typename TI, typename TO, typename C, int VEC>
int launch(const void* cs, const void* sn, RopeArgs a, int transpose, hipStream_t s) {
  constexpr int U = 4;
  a.chunks = a.half / VEC;
  // a tile is one pass of the block's threads over whole rows (at least one row)
  a.rows = kThreads / a.chunks > 0 ? kThreads / a.chunks : 1;
  a.tiles = (a.seq + a.rows - 1) / a.rows;
  // split the heads into the fewest groups that still give about eight blocks per CU
  const int all_heads = a.heads[0] + a.heads[1];
  const int64_t tiles = (int64_t)a.batch * a.tiles;
  constexpr int64_t kBlocksPerCu = 8;
  int64_t groups = (kBlocksPerCu * cu_count() + tiles - 1) / tiles;
  groups = groups < 1 ? 1 : (groups > all_heads ? all_heads : groups);
  a.group = (int)((all_heads + groups - 1) / groups);
  groups = (all_heads + a.group - 1) / a.group;
  const int64_t blocks = tiles * groups;
  if (blocks == 0) return PK_OK;
  if (blocks > INT32_MAX) return fail(PK_ERR_UNSUPPORTED, "pk_rope: %lld blocks exceed the grid", (long long)blocks);
  if (transpose)
    hipLaunchKernelGGL((rope_kernel<TI, TO, C, VEC, U, true>), dim3((unsigned)blocks), dim3(kThreads), 0, s,
                       static_cast<const C*>(cs), static_cast<const C*>(sn), a);
  else
    hipLaunchKernelGGL((rope_kernel<TI, TO, C, VEC, U, false>), dim3((unsigned)blocks), dim3(kThreads), 0, s,
                       static_cast<const C*>(cs), static_cast<const C*>(sn), a);
  return launched("pk_rope");
}

// Chunks are 16 bytes of the narrower of the input and output types.
template <typename TI, typename TO> constexpr int kRopeVec = 16 / (sizeof(TI) < sizeof(TO) ? sizeof(TI) : sizeof(TO));

template <typename TI, typename TO, typename C>
int run(bool vec, const void* cs, const void* sn, const RopeArgs& a, int tr, hipStream_t s) {
  return vec ? launch<TI, TO, C, kRopeVec<TI, TO>>(cs, sn, a, tr, s) : launch<TI, TO, C, 1>(cs, sn, a, tr, s);
}

template <typename TI, typename TO>
int run_cs(int cs_dtype, bool vec, const void* cs, const void* sn, const RopeArgs& a, int tr, hipStream_t s) {
  switch (cs_dtype) {
    case PK_F32: return run<TI, TO, float>(vec, cs, sn, a, tr, s);
    case PK_BF16: return run<TI, TO, bf16>(vec, cs, sn, a, tr, s);
    default: return run<TI, TO, f16>(vec, cs, sn, a, tr, s);
  }
}

// Input/output type pairs: one type, or a 16-bit type with fp32 either way.
bool rope_pair(int in_dtype, int out_dtype) {
  if (!known_dtype(in_dtype) || !known_dtype(out_dtype)) return false;
  return in_dtype == out_dtype || in_dtype == PK_F32 || out_dtype == PK_F32;
}

int run_types(int in_dtype, int out_dtype, int cs_dtype, bool vec, const void* cs, const void* sn, const RopeArgs& a,
              int tr, hipStream_t s) {
  if (in_dtype == out_dtype) {
    switch (in_dtype) {
      case PK_F32: return run_cs<float, float>(cs_dtype, vec, cs, sn, a, tr, s);
      case PK_BF16: return run_cs<bf16, bf16>(cs_dtype, vec, cs, sn, a, tr, s);
      default: return run_cs<f16, f16>(cs_dtype, vec, cs, sn, a, tr, s);
    }
  }
  if (out_dtype == PK_F32)
    return in_dtype == PK_BF16 ? run_cs<bf16, float>(cs_dtype, vec, cs, sn, a, tr, s)
                               : run_cs<f16, float>(cs_dtype, vec, cs, sn, a, tr, s);
  return out_dtype == PK_BF16 ? run_cs<float, bf16>(cs_dtype, vec, cs, sn, a, tr, s)
                              : run_cs<float, f16>(cs_dtype, vec, cs, sn, a, tr, s);
}

// ---------------------------------------------------------------------------
// qk_norm_rope: per-head RMSNorm of the q and k rows (each side with its own
// weight over head_dim), then the rotation above, in one pass:
//
//   r = 1 / sqrt(mean(x^2) + eps),  n = x r w,  y = n cos + rotate_half(n) sin
//
// and its backward, which recomputes n from x and the saved r:
//
//   g = rotation^T(dy),  u = g w,  dx = r (u - x r^2 <u, x> / head_dim),
//   dw = sum over rows of g x r.
//
// Same tiling as rope_kernel, with two restrictions that keep every row
// inside one wavefront: 16-byte chunks only, and chunks per row a power of
// two up to 64, so the row's lanes are consecutive and aligned and its sums
// are butterflies over them. A head group never mixes q and k heads, so a
// block holds one weight vector and one dw accumulator. dw is reduced without
// atomics: lanes of one chunk column in a wave, then the four waves through
// LDS, into one [2 * head_dim] partial row per block (the other side's half
// zero), summed over blocks in a fixed order by column_sums.

struct NormArgs {
  const void* x[2];   // q, k
  void* y[2];         // forward: outputs; backward: dq, dk
  const void* g[2];   // backward: cotangents dyq, dyk
  const void* w[2];   // q_weight, k_weight [head_dim]
  float* rstd[2];     // [batch, heads, seq] per side: written forward, read backward
  int64_t xs[2][3], ys[2][3], gs[2][3];  // (batch, head, seq) strides
  int heads[2];
  int batch, seq, half, cos_batch;
  int chunks, shift;  // chunks per row (a power of two) and its log2
  int rows, tiles;    // positions per block tile, tiles per batch row
  int group[2];       // heads per block of q and of k
  int groups_q;       // head groups of q; groups [groups_q, groups_q + groups_k) are k's
  float eps, inv_d;
  float* part;        // backward: [blocks, 2 * head_dim] partial dw rows
};

struct NormPlan {
  int rows, tiles, group[2], groups_q, groups_k;
  int64_t blocks;
};

// Head groups sized for about eight 256-thread blocks per CU, as rope_kernel,
// then evened out on each side: a side of n heads in g groups takes groups of
// ceil(n / g), so no block carries a short remainder (32 q heads in groups of
// at most 10 become four groups of 8, not 10, 10, 10 and 2).
NormPlan norm_plan(int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq, int chunks) {
  NormPlan p{};
  p.rows = kThreads / chunks;
  p.tiles = (int)((seq + p.rows - 1) / p.rows);
  const int64_t all = q_heads + kv_heads;
  const int64_t tiles = batch * p.tiles;
  if (all == 0 || tiles == 0) return p;
  int64_t groups = (8 * (int64_t)cu_count() + tiles - 1) / tiles;
  groups = groups < 1 ? 1 : (groups > all ? all : groups);
  const int64_t most = (all + groups - 1) / groups;  // heads per block at most
  const int64_t heads[2] = {q_heads, kv_heads};
  int n[2];
  for (int t = 0; t < 2; ++t) {
    n[t] = (int)((heads[t] + most - 1) / most);
    p.group[t] = n[t] > 0 ? (int)((heads[t] + n[t] - 1) / n[t]) : 1;
  }
  p.groups_q = n[0];
  p.groups_k = n[1];
  p.blocks = tiles * (p.groups_q + p.groups_k);
  return p;
}

// Sum over the `width` consecutive lanes (a power of two, aligned) that hold one row.
__device__ __forceinline__ float row_sum(float v, int width) {
  for (int m = 1; m < width; m <<= 1) v += __shfl_xor(v, m, 64);
  return v;
}

struct NormBlock {
  int t, b, h_begin, h_end, s, j;
};

__device__ __forceinline__ NormBlock norm_block(const NormArgs& a) {
  NormBlock nb;
  unsigned blk = blockIdx.x;
  const int tile = (int)(blk % (unsigned)a.tiles);
  blk /= (unsigned)a.tiles;
  nb.b = (int)(blk % (unsigned)a.batch);
  int gi = (int)(blk / (unsigned)a.batch);
  nb.t = gi >= a.groups_q;
  if (nb.t) gi -= a.groups_q;
  nb.h_begin = gi * a.group[nb.t];
  nb.h_end = nb.h_begin + a.group[nb.t] < a.heads[nb.t] ? nb.h_begin + a.group[nb.t] : a.heads[nb.t];
  nb.s = tile * a.rows + (int)(threadIdx.x >> a.shift);
  nb.j = (int)(threadIdx.x & (a.chunks - 1));
  return nb;
}

// T: q and k; TO: the outputs (T, or fp32 beside fp32 tables or weights); W: the weights (T, or fp32)
template <typename T, typename TO, typename C, typename W, int VEC, int U>
__global__ __launch_bounds__(kThreads) void qk_norm_rope_fwd_kernel(const C* __restrict__ cosp,
                                                                    const C* __restrict__ sinp, NormArgs a) {
  const NormBlock nb = norm_block(a);
  if (nb.s >= a.seq) return;  // whole rows drop out together; no barrier below
  const int t = nb.t, j = nb.j * VEC;
  const int64_t hd = 2 * (int64_t)a.half;
  const int64_t trow = ((int64_t)(a.cos_batch == 1 ? 0 : nb.b) * a.seq + nb.s) * hd + j;
  float c1[VEC], c2[VEC], s1[VEC], s2[VEC], w1[VEC], w2[VEC];
  table(cosp + trow, c1);
  table(cosp + trow + a.half, c2);
  table(sinp + trow, s1);
  table(sinp + trow + a.half, s2);
  const W* wp = static_cast<const W*>(a.w[t]);
  table(wp + j, w1);
  table(wp + a.half + j, w2);
  const T* xb = static_cast<const T*>(a.x[t]) + nb.b * a.xs[t][0] + nb.s * a.xs[t][2] + j;
  TO* yb = static_cast<TO*>(a.y[t]) + nb.b * a.ys[t][0] + nb.s * a.ys[t][2] + j;
  float* rb = a.rstd[t] + ((int64_t)nb.b * a.heads[t]) * a.seq + nb.s;
  for (int h0 = nb.h_begin; h0 < nb.h_end; h0 += U) {
    Pack<T, VEC> x1[U], x2[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (h0 + u >= nb.h_end) break;
      const T* xr = xb + (h0 + u) * a.xs[t][1];
      x1[u].load(xr);
      x2[u].load(xr + a.half);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (h0 + u >= nb.h_end) break;
      float ss = 0.f;
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        const float p = to_f32(x1[u].v[k]), q = to_f32(x2[u].v[k]);
        ss += p * p + q * q;
      }
      const float r = rsqrtf(row_sum(ss, a.chunks) * a.inv_d + a.eps);
      Pack<TO, VEC> y1, y2;
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        const float n1 = to_f32(x1[u].v[k]) * r * w1[k], n2 = to_f32(x2[u].v[k]) * r * w2[k];
        y1.v[k] = from_f32<TO>(n1 * c1[k] - n2 * s1[k]);
        y2.v[k] = from_f32<TO>(n2 * c2[k] + n1 * s2[k]);
      }
      TO* yr = yb + (h0 + u) * a.ys[t][1];
      y1.store(yr);
      y2.store(yr + a.half);
      if (nb.j == 0) rb[(int64_t)(h0 + u) * a.seq] = r;
    }
  }
}

// T: q, k and their gradients; TG: the cotangents (the forward's output type); W: the weights
// and their gradients
template <typename T, typename TG, typename C, typename W, int VEC, int U>
__global__ __launch_bounds__(kThreads) void qk_norm_rope_bwd_kernel(const C* __restrict__ cosp,
                                                                    const C* __restrict__ sinp, NormArgs a) {
  extern __shared__ float red[];  // [4 waves][2 * half]
  const NormBlock nb = norm_block(a);
  const int t = nb.t, j = nb.j * VEC;
  float dw1[VEC], dw2[VEC];
#pragma unroll
  for (int k = 0; k < VEC; ++k) dw1[k] = dw2[k] = 0.f;
  if (nb.s < a.seq) {  // rows past the end keep zero partials but join the reduction
    const int64_t hd = 2 * (int64_t)a.half;
    const int64_t trow = ((int64_t)(a.cos_batch == 1 ? 0 : nb.b) * a.seq + nb.s) * hd + j;
    float c1[VEC], c2[VEC], s1[VEC], s2[VEC], w1[VEC], w2[VEC];
    table(cosp + trow, c1);
    table(cosp + trow + a.half, c2);
    table(sinp + trow, s1);
    table(sinp + trow + a.half, s2);
    const W* wp = static_cast<const W*>(a.w[t]);
    table(wp + j, w1);
    table(wp + a.half + j, w2);
    const T* xb = static_cast<const T*>(a.x[t]) + nb.b * a.xs[t][0] + nb.s * a.xs[t][2] + j;
    const TG* gb = static_cast<const TG*>(a.g[t]) + nb.b * a.gs[t][0] + nb.s * a.gs[t][2] + j;
    T* db = static_cast<T*>(a.y[t]) + nb.b * a.ys[t][0] + nb.s * a.ys[t][2] + j;
    const float* rb = a.rstd[t] + ((int64_t)nb.b * a.heads[t]) * a.seq + nb.s;
    for (int h0 = nb.h_begin; h0 < nb.h_end; h0 += U) {
      Pack<T, VEC> x1[U], x2[U];
      Pack<TG, VEC> g1[U], g2[U];
      float r[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (h0 + u >= nb.h_end) break;
        const T* xr = xb + (h0 + u) * a.xs[t][1];
        const TG* gr = gb + (h0 + u) * a.gs[t][1];
        x1[u].load(xr);
        x2[u].load(xr + a.half);
        g1[u].load(gr);
        g2[u].load(gr + a.half);
        r[u] = rb[(int64_t)(h0 + u) * a.seq];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (h0 + u >= nb.h_end) break;
        float e1[VEC], e2[VEC], u1[VEC], u2[VEC];
        float dot = 0.f;
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
          const float d1 = to_f32(g1[u].v[k]), d2 = to_f32(g2[u].v[k]);
          e1[k] = d1 * c1[k] + d2 * s2[k];  // gradient reaching n (transposed rotation)
          e2[k] = d2 * c2[k] - d1 * s1[k];
          u1[k] = e1[k] * w1[k];
          u2[k] = e2[k] * w2[k];
          dot += u1[k] * to_f32(x1[u].v[k]) + u2[k] * to_f32(x2[u].v[k]);
        }
        const float rr = r[u];
        const float coef = rr * rr * row_sum(dot, a.chunks) * a.inv_d;
        Pack<T, VEC> o1, o2;
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
          const float p = to_f32(x1[u].v[k]), q = to_f32(x2[u].v[k]);
          o1.v[k] = from_f32<T>(rr * (u1[k] - p * coef));
          o2.v[k] = from_f32<T>(rr * (u2[k] - q * coef));
          dw1[k] += e1[k] * p * rr;
          dw2[k] += e2[k] * q * rr;
        }
        T* dr = db + (h0 + u) * a.ys[t][1];
        o1.store(dr);
        o2.store(dr + a.half);
      }
    }
  }
  // dw: lanes of one chunk column within the wave, then the four waves
#pragma unroll
  for (int k = 0; k < VEC; ++k) {
    for (int m = a.chunks; m < 64; m <<= 1) {
      dw1[k] += __shfl_xor(dw1[k], m, 64);
      dw2[k] += __shfl_xor(dw2[k], m, 64);
    }
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int hd = 2 * a.half;
  if (lane < a.chunks) {
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      red[wave * hd + j + k] = dw1[k];
      red[wave * hd + a.half + j + k] = dw2[k];
    }
  }
  __syncthreads();
  float* out = a.part + (int64_t)blockIdx.x * 2 * hd;
  for (int c = threadIdx.x; c < 2 * hd; c += kThreads) {
    const int side = c >= hd, col = c - side * hd;
    float v = 0.f;
    if (side == t) v = ((red[col] + red[hd + col]) + red[2 * hd + col]) + red[3 * hd + col];
    out[c] = v;
  }
}

// 16-byte chunks with a power-of-two count per row, at most 64; 0 when unsupported.
int norm_chunks(int64_t head_dim, int x_dtype) {
  const int64_t V = 16 / elem_size(x_dtype);
  const int64_t half = head_dim / 2;
  if (head_dim % 2 != 0 || half % V != 0) return 0;
  const int64_t c = half / V;
  return (c >= 1 && c <= 64 && (c & (c - 1)) == 0) ? (int)c : 0;
}

int64_t norm_workspace(const NormPlan& p, int64_t head_dim) {
  auto up = [](int64_t n) { return (n + 255) / 256 * 256; };
  const int64_t cols = 2 * head_dim;
  return up(p.blocks * cols * (int64_t)sizeof(float)) + up(stage_rows(p.blocks) * cols * (int64_t)sizeof(float));
}

// TY: the forward's output type, which is the backward's cotangent type; W: the weights' type
template <typename T, typename TY, typename C, typename W>
int norm_launch(bool backward, const void* cs, const void* sn, NormArgs a, const NormPlan& p, void* dw, void* ws,
                hipStream_t s) {
  constexpr int VEC = 16 / sizeof(T);
  const C* c = static_cast<const C*>(cs);
  const C* n = static_cast<const C*>(sn);
  if (!backward) {
    if (p.blocks > 0)
      hipLaunchKernelGGL((qk_norm_rope_fwd_kernel<T, TY, C, W, VEC, 4>), dim3((unsigned)p.blocks), dim3(kThreads), 0, s,
                         c, n, a);
    return launched("pk_qk_norm_rope_fwd");
  }
  const int cols = 4 * a.half;
  auto up = [](int64_t v) { return (v + 255) / 256 * 256; };
  a.part = static_cast<float*>(ws);
  float* stage = reinterpret_cast<float*>(static_cast<char*>(ws) + up(p.blocks * cols * (int64_t)sizeof(float)));
  if (p.blocks > 0) {
    const size_t lds = 4 * (size_t)(2 * a.half) * sizeof(float);
    hipLaunchKernelGGL((qk_norm_rope_bwd_kernel<T, TY, C, W, VEC, 2>), dim3((unsigned)p.blocks), dim3(kThreads), lds,
                       s, c, n, a);
    column_sums<W>(a.part, stage, static_cast<W*>(dw), p.blocks, cols, s);
  } else {  // nothing to sum: dw is zero
    hipLaunchKernelGGL(column_sum_final<W>, dim3((cols + kFinalCols - 1) / kFinalCols), dim3(kColThreads), 0, s,
                       stage, static_cast<W*>(dw), (int64_t)0, cols);
  }
  return launched("pk_qk_norm_rope_bwd");
}

// Shared validation and argument set-up of the two entry points.
int norm_setup(const char* who, NormArgs& a, NormPlan& p, const void* q, const void* k, const void* qw,
               const void* kw, const void* cos, const void* sin, const int64_t* strides, int nstrides, int64_t batch,
               int64_t q_heads, int64_t kv_heads, int64_t seq, int64_t head_dim, int64_t cos_batch, int x_dtype,
               int cs_dtype) {
  if (batch < 0 || q_heads < 0 || kv_heads < 0 || seq < 0 || head_dim < 0)
    return fail(PK_ERR_INVALID, "%s: negative size", who);
  if (cos_batch != 1 && cos_batch != batch)
    return fail(PK_ERR_INVALID, "%s: cos_batch=%lld is neither 1 nor batch=%lld", who, (long long)cos_batch,
                (long long)batch);
  if (!known_dtype(x_dtype) || !known_dtype(cs_dtype))
    return fail(PK_ERR_UNSUPPORTED, "%s: dtype codes %d/%d", who, x_dtype, cs_dtype);
  if (batch > INT32_MAX || seq > INT32_MAX || q_heads + kv_heads > INT32_MAX || head_dim > INT32_MAX)
    return fail(PK_ERR_UNSUPPORTED, "%s: shape too large", who);
  const int chunks = norm_chunks(head_dim, x_dtype);
  if (head_dim > 0 && chunks == 0)
    return fail(PK_ERR_UNSUPPORTED, "%s: head_dim=%lld is not 2 * (16-byte packs) * 2^k with at most 64 packs", who,
                (long long)head_dim);
  a = NormArgs{};
  a.chunks = chunks > 0 ? chunks : 1;
  while ((1 << a.shift) < a.chunks) ++a.shift;
  p = norm_plan(batch, q_heads, kv_heads, seq, a.chunks);
  if (p.blocks > INT32_MAX) return fail(PK_ERR_UNSUPPORTED, "%s: %lld blocks exceed the grid", who, (long long)p.blocks);
  a.heads[0] = (int)q_heads;
  a.heads[1] = (int)kv_heads;
  a.batch = (int)batch;
  a.seq = (int)seq;
  a.half = (int)(head_dim / 2);
  a.cos_batch = (int)cos_batch;
  a.rows = p.rows;
  a.tiles = p.tiles;
  a.group[0] = p.group[0];
  a.group[1] = p.group[1];
  a.groups_q = p.groups_q;
  a.inv_d = head_dim > 0 ? 1.0f / (float)head_dim : 0.f;
  if (p.blocks == 0) return PK_OK;  // nothing to read (a backward still zeroes dw)
  if (!cos || !sin || !strides || (q_heads > 0 && (!q || !qw)) || (kv_heads > 0 && (!k || !kw)))
    return fail(PK_ERR_INVALID, "%s: null pointer", who);
  const void* ptrs[] = {q, k, qw, kw};
  for (const void* ptr : ptrs)
    if (ptr && !aligned16(ptr)) return fail(PK_ERR_UNSUPPORTED, "%s: q, k and the weights must be 16-byte aligned", who);
  if ((16 / elem_size(x_dtype) * elem_size(cs_dtype)) % 16 == 0 && !(aligned16(cos) && aligned16(sin)))
    return fail(PK_ERR_UNSUPPORTED, "%s: cos and sin must be 16-byte aligned", who);
  const int64_t V = 16 / elem_size(x_dtype);
  for (int i = 0; i < nstrides; ++i)
    if (strides[i] % V != 0) return fail(PK_ERR_UNSUPPORTED, "%s: strides must be multiples of %lld", who, (long long)V);
  a.x[0] = q;
  a.x[1] = k;
  a.w[0] = qw;
  a.w[1] = kw;
  return PK_OK;
}

template <typename T, typename TY, typename W>
int norm_run_cs(int cs_dtype, bool backward, const void* cs, const void* sn, const NormArgs& a, const NormPlan& p,
                void* dw, void* ws, hipStream_t s) {
  switch (cs_dtype) {
    case PK_F32: return norm_launch<T, TY, float, W>(backward, cs, sn, a, p, dw, ws, s);
    case PK_BF16: return norm_launch<T, TY, bf16, W>(backward, cs, sn, a, p, dw, ws, s);
    default: return norm_launch<T, TY, f16, W>(backward, cs, sn, a, p, dw, ws, s);
  }
}

// Type codes the kernels take: the weights are x's type, or fp32 beside a
// 16-bit x; the output (or cotangent) is x's type, or fp32 with a 16-bit x,
// and fp32 whenever the weights are (their product with x promotes).
bool norm_types(int x_dtype, int y_dtype, int w_dtype) {
  if (!known_dtype(x_dtype)) return false;
  const bool half = x_dtype != PK_F32;
  if (w_dtype != x_dtype && !(half && w_dtype == PK_F32)) return false;
  if (w_dtype != x_dtype) return y_dtype == PK_F32;
  return y_dtype == x_dtype || (half && y_dtype == PK_F32);
}

int norm_run(int x_dtype, int y_dtype, int cs_dtype, int w_dtype, bool backward, const void* cs, const void* sn,
             const NormArgs& a, const NormPlan& p, void* dw, void* ws, hipStream_t s) {
  if (w_dtype != x_dtype)
    return x_dtype == PK_BF16 ? norm_run_cs<bf16, float, float>(cs_dtype, backward, cs, sn, a, p, dw, ws, s)
                              : norm_run_cs<f16, float, float>(cs_dtype, backward, cs, sn, a, p, dw, ws, s);
  if (y_dtype != x_dtype)
    return x_dtype == PK_BF16 ? norm_run_cs<bf16, float, bf16>(cs_dtype, backward, cs, sn, a, p, dw, ws, s)
                              : norm_run_cs<f16, float, f16>(cs_dtype, backward, cs, sn, a, p, dw, ws, s);
  switch (x_dtype) {
    case PK_F32: return norm_run_cs<float, float, float>(cs_dtype, backward, cs, sn, a, p, dw, ws, s);
    case PK_BF16: return norm_run_cs<bf16, bf16, bf16>(cs_dtype, backward, cs, sn, a, p, dw, ws, s);
    default: return norm_run_cs<f16, f16, f16>(cs_dtype, backward, cs, sn, a, p, dw, ws, s);
  }
}

}  // namespace
}  // namespace pk

extern "C" {

int pk_rope(const void* q, const void* k, const void* cos, const void* sin, void* yq, void* yk,
            const int64_t* strides, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq, int64_t head_dim,
            int64_t cos_batch, int x_dtype, int y_dtype, int cs_dtype, int transpose, void* stream) {
  using namespace pk;
  if (batch < 0 || q_heads < 0 || kv_heads < 0 || seq < 0 || head_dim < 0)
    return fail(PK_ERR_INVALID, "pk_rope: negative size");
  if (head_dim % 2 != 0) return fail(PK_ERR_INVALID, "pk_rope: head_dim=%lld is odd", (long long)head_dim);
  if (cos_batch != 1 && cos_batch != batch)
    return fail(PK_ERR_INVALID, "pk_rope: cos_batch=%lld is neither 1 nor batch=%lld", (long long)cos_batch,
                (long long)batch);
  if (batch == 0 || seq == 0 || head_dim == 0 || q_heads + kv_heads == 0) return PK_OK;
  if (!cos || !sin || !strides || (q_heads > 0 && (!q || !yq)) || (kv_heads > 0 && (!k || !yk)))
    return fail(PK_ERR_INVALID, "pk_rope: null pointer");
  if (!known_dtype(cs_dtype) || !rope_pair(x_dtype, y_dtype))
    return fail(PK_ERR_UNSUPPORTED, "pk_rope: dtype codes %d -> %d with tables %d", x_dtype, y_dtype, cs_dtype);
  if (batch > INT32_MAX || seq > INT32_MAX || q_heads > INT32_MAX || kv_heads > INT32_MAX || head_dim > INT32_MAX)
    return fail(PK_ERR_UNSUPPORTED, "pk_rope: shape too large");
  if (q_heads + kv_heads > INT32_MAX) return fail(PK_ERR_UNSUPPORTED, "pk_rope: too many heads");
  RopeArgs a{};
  a.x[0] = q;
  a.x[1] = k;
  a.y[0] = yq;
  a.y[1] = yk;
  for (int i = 0; i < 3; ++i) {
    a.xs[0][i] = strides[i];
    a.xs[1][i] = strides[3 + i];
    a.ys[0][i] = strides[6 + i];
    a.ys[1][i] = strides[9 + i];
  }
  a.heads[0] = (int)q_heads;
  a.heads[1] = (int)kv_heads;
  a.batch = (int)batch;
  a.seq = (int)seq;
  a.half = (int)(head_dim / 2);
  a.cos_batch = (int)cos_batch;
  // 16-byte packs of the narrower of x and y when every row start and both
  // halves are 16-byte aligned (half a multiple of V and strides multiples of
  // V); a pack's table entries are then 16-byte loads too whenever they fill
  // whole 16 bytes, which needs only the table bases aligned.
  const int narrow = elem_size(x_dtype) < elem_size(y_dtype) ? elem_size(x_dtype) : elem_size(y_dtype);
  const int64_t V = 16 / narrow;
  bool vec = a.half % V == 0;
  const void* ptrs[] = {q, k, yq, yk};
  for (const void* p : ptrs) vec = vec && (p == nullptr || aligned16(p));
  for (int i = 0; i < 12; ++i) vec = vec && strides[i] % V == 0;
  if ((V * elem_size(cs_dtype)) % 16 == 0) vec = vec && aligned16(cos) && aligned16(sin);
  return run_types(x_dtype, y_dtype, cs_dtype, vec, cos, sin, a, transpose, static_cast<hipStream_t>(stream));
}

int pk_qk_norm_rope_fwd(const void* q, const void* k, const void* q_weight, const void* k_weight, const void* cos,
                        const void* sin, void* yq, void* yk, float* rstd_q, float* rstd_k, const int64_t* strides,
                        int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq, int64_t head_dim,
                        int64_t cos_batch, float eps, int x_dtype, int y_dtype, int cs_dtype, int w_dtype,
                        void* stream) {
  using namespace pk;
  if (!norm_types(x_dtype, y_dtype, w_dtype))
    return fail(PK_ERR_UNSUPPORTED,
                "pk_qk_norm_rope_fwd: dtype codes %d -> %d with weights %d (x's; fp32 from 16 bits; fp32 weights "
                "with 16 bits give fp32)", x_dtype, y_dtype, w_dtype);
  NormArgs a;
  NormPlan p;
  int rc = norm_setup("pk_qk_norm_rope_fwd", a, p, q, k, q_weight, k_weight, cos, sin, strides, 12, batch, q_heads,
                      kv_heads, seq, head_dim, cos_batch, x_dtype, cs_dtype);
  if (rc != PK_OK || p.blocks == 0) return rc;
  if ((q_heads > 0 && (!yq || !rstd_q)) || (kv_heads > 0 && (!yk || !rstd_k)))
    return fail(PK_ERR_INVALID, "pk_qk_norm_rope_fwd: null output");
  if ((yq && !aligned16(yq)) || (yk && !aligned16(yk)))
    return fail(PK_ERR_UNSUPPORTED, "pk_qk_norm_rope_fwd: outputs must be 16-byte aligned");
  a.y[0] = yq;
  a.y[1] = yk;
  a.rstd[0] = rstd_q;
  a.rstd[1] = rstd_k;
  for (int i = 0; i < 3; ++i) {
    a.xs[0][i] = strides[i];
    a.xs[1][i] = strides[3 + i];
    a.ys[0][i] = strides[6 + i];
    a.ys[1][i] = strides[9 + i];
  }
  a.eps = eps;
  return norm_run(x_dtype, y_dtype, cs_dtype, w_dtype, false, cos, sin, a, p, nullptr, nullptr,
                  static_cast<hipStream_t>(stream));
}

int64_t pk_qk_norm_rope_bwd_workspace(int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq,
                                      int64_t head_dim, int x_dtype) {
  using namespace pk;
  if (batch < 0 || q_heads < 0 || kv_heads < 0 || seq < 0 || head_dim < 0 || !known_dtype(x_dtype)) return -1;
  const int chunks = norm_chunks(head_dim, x_dtype);
  if (head_dim > 0 && chunks == 0) return -1;
  const NormPlan p = norm_plan(batch, q_heads, kv_heads, seq, chunks > 0 ? chunks : 1);
  return norm_workspace(p, head_dim);
}

int pk_qk_norm_rope_bwd(const void* q, const void* k, const void* q_weight, const void* k_weight, const void* cos,
                        const void* sin, const float* rstd_q, const float* rstd_k, const void* dyq, const void* dyk,
                        void* dq, void* dk, void* dw, void* workspace, int64_t workspace_bytes,
                        const int64_t* strides, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq,
                        int64_t head_dim, int64_t cos_batch, int x_dtype, int dy_dtype, int cs_dtype, int w_dtype,
                        void* stream) {
  using namespace pk;
  if (!norm_types(x_dtype, dy_dtype, w_dtype))
    return fail(PK_ERR_UNSUPPORTED,
                "pk_qk_norm_rope_bwd: dtype codes %d / %d with weights %d (cotangents x's; fp32 from 16 bits; fp32 "
                "with fp32 weights)", x_dtype, dy_dtype, w_dtype);
  NormArgs a;
  NormPlan p;
  int rc = norm_setup("pk_qk_norm_rope_bwd", a, p, q, k, q_weight, k_weight, cos, sin, strides, 18, batch, q_heads,
                      kv_heads, seq, head_dim, cos_batch, x_dtype, cs_dtype);
  if (rc != PK_OK || head_dim == 0) return rc;
  if (!dw) return fail(PK_ERR_INVALID, "pk_qk_norm_rope_bwd: null dw");
  const int64_t need = norm_workspace(p, head_dim);
  if ((need > 0 && !workspace) || workspace_bytes < need)
    return fail(PK_ERR_INVALID, "pk_qk_norm_rope_bwd: workspace of %lld bytes, need %lld", (long long)workspace_bytes,
                (long long)need);
  if (p.blocks > 0) {
    if ((q_heads > 0 && (!dyq || !dq || !rstd_q)) || (kv_heads > 0 && (!dyk || !dk || !rstd_k)))
      return fail(PK_ERR_INVALID, "pk_qk_norm_rope_bwd: null pointer");
    const void* outs[] = {dyq, dyk, dq, dk};
    for (const void* ptr : outs)
      if (ptr && !aligned16(ptr)) return fail(PK_ERR_UNSUPPORTED, "pk_qk_norm_rope_bwd: 16-byte alignment required");
    a.g[0] = dyq;
    a.g[1] = dyk;
    a.y[0] = dq;
    a.y[1] = dk;
    a.rstd[0] = const_cast<float*>(rstd_q);
    a.rstd[1] = const_cast<float*>(rstd_k);
    for (int i = 0; i < 3; ++i) {
      a.xs[0][i] = strides[i];
      a.xs[1][i] = strides[3 + i];
      a.gs[0][i] = strides[6 + i];
      a.gs[1][i] = strides[9 + i];
      a.ys[0][i] = strides[12 + i];
      a.ys[1][i] = strides[15 + i];
    }
  }
  return norm_run(x_dtype, dy_dtype, cs_dtype, w_dtype, true, cos, sin, a, p, dw, workspace,
                  static_cast<hipStream_t>(stream));
}

}  // extern "C"
