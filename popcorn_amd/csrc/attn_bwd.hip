// Attention backward (grouped-query, optional causal mask, dense batches or
// packed sequences) on gfx950 matrix cores, in two deterministic kernels
// that never add into shared memory of another block:
//
//   dq kernel   one block = 4 waves x 32 query rows of one (sequence, q head),
//               keys streamed through LDS in tiles of 32. Per tile each wave
//               recomputes S^T = K Q^T and dP^T = V dO^T, forms
//               P = exp2(s*c - lse2) from the forward's log-sum-exp and
//               dS = P (dP - D), and accumulates dQ^T += K^T dS^T. Its prologue
//               also computes D = rowsum(dO * O) for its rows and stores it for
//               the second kernel.
//   dkdv kernel one block = 4 waves x 32 keys of one (sequence, kv head),
//               holding its K and V fragments in registers; query tiles of 32
//               rows (over every q head of the group) stream through LDS. Per
//               tile each wave computes S = Q K^T and dP = dO V^T, whose result
//               layout puts one key per lane column, so P and dS go straight
//               into dV^T += dO^T P and dK^T += Q^T dS as B operands.
//
// With scores z = scale * q.k: dS = dL/dz, dQ = scale * dS K,
// dK = scale * dS^T Q, dV = P^T dO. A negative scale is applied as in the
// forward (Q negated on load, c = |scale| log2 e), so dK uses |scale| and
// dQ the signed scale.
//
// LDS tiles are row-major 16-byte chunks. For head_dim 128 chunk c of row r
// sits at c ^ (4 (r % 4) + (r / 4) % 4): the 16-byte fragment reads (16 rows,
// one chunk) and the transposing ds_read_b64_tr_b16 reads (4 rows x 4 chunks
// per pair of 16-lane groups) both land on 64 distinct banks. head_dim 64
// rows are padded to 72 elements instead.
#include <math.h>

#include "api.h"
#include "attn_common.h"

namespace pk {
namespace {

using namespace attn;

constexpr int NT = 256;
constexpr int BM = 128;  // dq kernel: query rows per block
constexpr int BN = 32;   // dq kernel: keys per tile
constexpr int BK = 128;  // dkdv kernel: keys per block
constexpr int BQ = 32;   // dkdv kernel: query rows per tile

struct BwdArgs {
  const void *q, *k, *v, *o, *dout;
  const float* lse;  // natural log, laid out like dsum
  float* dsum;       // D = rowsum(dO * O): element (b, h, token t of b) at b*lse_bs + h*lse_hs + t (+ start)
  void *dq, *dk, *dv;
  const int* cu;  // packed sequences (see pk_attn_varlen_fwd) or NULL
  int total;
  int64_t qs[3], ks[3], vs[3], os[3], gs[3], dqs[3], dks[3], dvs[3];  // (batch, token, head) strides
  int64_t lse_bs, lse_hs;
  int B, S, Hq, Hkv, group;
  float scale;  // signed softmax scale
  float c;      // |scale| * log2(e), at least 1e-30
  uint32_t q_flip;
};

// LDS tile layout: element offset of (row, dim), dim a multiple of 4
template <int D> struct Tile {
  static constexpr int ST = D == 128 ? 128 : D + 8;
  static __device__ __forceinline__ int at(int row, int dim) {
    if constexpr (D == 128)
      return row * 128 + ((((dim >> 3) ^ (4 * (row & 3) + ((row >> 2) & 3))) << 3) | (dim & 7));
    else
      return row * ST + dim;
  }
};

__device__ __forceinline__ void seq_bounds(const BwdArgs& a, int b, int& start, int& S) {
  S = a.S;
  start = 0;
  if (a.cu != nullptr) {
    start = min(max(a.cu[b], 0), a.total);
    S = min(min(max(a.cu[b + 1], start), a.total) - start, a.S);
  }
}

__device__ __forceinline__ uint4 flip(uint4 v, uint32_t f) { return make_uint4(v.x ^ f, v.y ^ f, v.z ^ f, v.w ^ f); }

// ------------------------------------------------------------------ dq kernel

template <typename T, int D, bool CAUSAL>
__global__ __attribute__((amdgpu_flat_work_group_size(NT, NT), amdgpu_waves_per_eu(2))) void attn_bwd_dq_kernel(
    BwdArgs a) {
  using Frag = typename Mma<T>::frag;
  using L = Tile<D>;
  constexpr int KCH = D / 8;
  constexpr int ROWS = NT / KCH;     // tile rows staged per pass
  constexpr int PASSES = BN / ROWS;  // 2 (D = 128) or 1 (D = 64)
  constexpr int KK = D / 16;
  constexpr int DT = D / 32;
  __shared__ __attribute__((aligned(16))) T Ks[2][BN * L::ST];
  __shared__ __attribute__((aligned(16))) T Vs[2][BN * L::ST];

  const int m_tiles = (a.S + BM - 1) / BM;
  const int w = blockIdx.x;
  const int per_tile = a.B * a.Hq;
  const int m_tile = m_tiles - 1 - w / per_tile;  // longest causal rows first
  const int b = (w % per_tile) / a.Hq;
  const int hq = w % a.Hq;
  const int hkv = hq / a.group;
  int start, S;
  seq_bounds(a, b, start, S);
  const int m0 = m_tile * BM;
  if (m0 >= S) return;  // whole block, before any barrier

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r32 = lane & 31;
  const int g = lane >> 5;
  const int wave_first = m0 + wave * 32;
  const int q_row = wave_first + r32;
  const bool row_ok = q_row < S;

  const T* qbase = static_cast<const T*>(a.q) + b * a.qs[0] + hq * a.qs[2] + start * a.qs[1];
  const T* obase = static_cast<const T*>(a.o) + b * a.os[0] + hq * a.os[2] + start * a.os[1];
  const T* gbase = static_cast<const T*>(a.dout) + b * a.gs[0] + hq * a.gs[2] + start * a.gs[1];
  const T* kbase = static_cast<const T*>(a.k) + b * a.ks[0] + hkv * a.ks[2] + start * a.ks[1];
  const T* vbase = static_cast<const T*>(a.v) + b * a.vs[0] + hkv * a.vs[2] + start * a.vs[1];
  const int k_bytes = (int)(((int64_t)(S - 1) * a.ks[1] + D) * (int)sizeof(T));
  const int v_bytes = (int)(((int64_t)(S - 1) * a.vs[1] + D) * (int)sizeof(T));
  const __amdgpu_buffer_rsrc_t krsrc = __builtin_amdgcn_make_buffer_rsrc((void*)kbase, (short)0, k_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrsrc = __builtin_amdgcn_make_buffer_rsrc((void*)vbase, (short)0, v_bytes, 0x00020000);

  // Q^T and dO^T fragments of this lane's row (B operands), and D = rowsum(dO * O)
  Frag qf[KK], gf[KK];
  float dsum = 0.f;
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
    uint4 qr = make_uint4(0, 0, 0, 0), gr = qr, orr = qr;
    if (row_ok) {
      const int64_t col = 16 * kk + 8 * g;
      qr = *reinterpret_cast<const uint4*>(qbase + (int64_t)q_row * a.qs[1] + col);
      gr = *reinterpret_cast<const uint4*>(gbase + (int64_t)q_row * a.gs[1] + col);
      orr = *reinterpret_cast<const uint4*>(obase + (int64_t)q_row * a.os[1] + col);
    }
    qf[kk] = __builtin_bit_cast(Frag, flip(qr, a.q_flip));
    gf[kk] = __builtin_bit_cast(Frag, gr);
    const Frag of = __builtin_bit_cast(Frag, orr);
#pragma unroll
    for (int j = 0; j < 8; ++j) dsum += to_f32(gf[kk][j]) * to_f32(of[j]);
  }
  dsum += __shfl_xor(dsum, 32, 64);
  const int64_t lidx = b * a.lse_bs + hq * a.lse_hs + start + q_row;
  // rows past the end: lse2 = +inf makes every p zero
  const float lse2 = row_ok ? a.lse[lidx] * 1.4426950408889634f : INFINITY;
  if (row_ok && g == 0) a.dsum[lidx] = dsum;

  const int kv_end = CAUSAL ? min(m0 + BM, S) : S;
  const int n_tiles = (kv_end + BN - 1) / BN;

  const int kc = tid % KCH, kr = tid / KCH;
  uint4 kreg[PASSES], vreg[PASSES];
  auto load = [&](int t) {
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int row = t * BN + kr + p * ROWS;
      kreg[p] = ld_buf(krsrc, (kc * 8) * (int)sizeof(T), row * (int)a.ks[1] * (int)sizeof(T));
      vreg[p] = ld_buf(vrsrc, (kc * 8) * (int)sizeof(T), row * (int)a.vs[1] * (int)sizeof(T));
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int off = L::at(kr + p * ROWS, kc * 8);
      *reinterpret_cast<uint4*>(Ks[buf] + off) = kreg[p];
      *reinterpret_cast<uint4*>(Vs[buf] + off) = vreg[p];
    }
  };
  // lane offsets: K / V fragment kk (A operand: row r32, dims 16kk + 8g) and the
  // transposing K reads (rows 4g + (lane%16)/4 [+8], dims 32dt + 16((lane/16)%2) + 4(lane%4))
  int a_lane[KK], t_lane[2][DT];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) a_lane[kk] = L::at(r32, 16 * kk + 8 * g);
#pragma unroll
  for (int hi = 0; hi < 2; ++hi)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      t_lane[hi][dt] = L::at(8 * hi + 4 * g + ((lane & 15) >> 2), 32 * dt + 16 * ((lane >> 4) & 1) + 4 * (lane & 3));

  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[dt][r] = 0.f;

  load(0);
  store(0);
  __syncthreads();
  for (int t = 0; t < n_tiles; ++t) {
    const int buf = t & 1;
    load(min(t + 1, n_tiles - 1));
    const int kv0 = t * BN;
    if (!(CAUSAL && kv0 > wave_first + 31)) {
      const T* ks = Ks[buf];
      const T* vs = Vs[buf];
      f32x16 s, dp;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        s = Mma<T>::run(*reinterpret_cast<const Frag*>(ks + a_lane[kk]), qf[kk], s);
        dp = Mma<T>::run(*reinterpret_cast<const Frag*>(vs + a_lane[kk]), gf[kk], dp);
      }
      const bool need_mask = (CAUSAL && kv0 + BN - 1 > wave_first) || kv0 + BN > S;
      const int lim = CAUSAL ? min(q_row, S - 1) : S - 1;
      Frag dsf[2];
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int r = 8 * c + j;
          float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], a.c, -lse2));
          if (need_mask) p = kv0 + 8 * (r >> 2) + 4 * g + (r & 3) <= lim ? p : 0.f;
          dsf[c][j] = (T)(p * (dp[r] - dsum));
        }
      // dQ^T += K^T dS^T: K^T fragments from transposing reads of the K tile
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(ks + t_lane[0][dt] + 16 * c * L::ST));
          const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(ks + t_lane[1][dt] + 16 * c * L::ST));
          acc[dt] = Mma<T>::run(__builtin_bit_cast(Frag, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7)),
                                dsf[c], acc[dt]);
        }
    }
    store(buf ^ 1);
    __syncthreads();
  }

  if (row_ok) {
    T* drow = static_cast<T*>(a.dq) + b * a.dqs[0] + hq * a.dqs[2] + (int64_t)(start + q_row) * a.dqs[1];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq)
        *reinterpret_cast<uint2*>(drow + dt * 32 + 8 * rq + 4 * g) =
            pack4<T>(acc[dt][4 * rq] * a.scale, acc[dt][4 * rq + 1] * a.scale, acc[dt][4 * rq + 2] * a.scale,
                     acc[dt][4 * rq + 3] * a.scale);
  }
}

// ---------------------------------------------------------------- dkdv kernel

template <typename T, int D, bool CAUSAL>
__global__ __attribute__((amdgpu_flat_work_group_size(NT, NT), amdgpu_waves_per_eu(1))) void attn_bwd_dkdv_kernel(
    BwdArgs a) {
  using Frag = typename Mma<T>::frag;
  using L = Tile<D>;
  constexpr int KCH = D / 8;
  constexpr int PER = BQ * KCH / NT;  // chunks of each of Q and dO per thread: 2 (D = 128) or 1
  constexpr int KK = D / 16;
  constexpr int DT = D / 32;
  __shared__ __attribute__((aligned(16))) T Qs[2][BQ * L::ST];
  __shared__ __attribute__((aligned(16))) T Gs[2][BQ * L::ST];
  __shared__ __attribute__((aligned(16))) float Ls[2][BQ];  // lse2 of the tile's rows (+inf past the end)
  __shared__ __attribute__((aligned(16))) float Dsm[2][BQ];

  const int kv_tiles = (a.S + BK - 1) / BK;
  const int w = blockIdx.x;
  const int per_tile = a.B * a.Hkv;
  const int kv_tile = w / per_tile;  // first key tiles (the most causal work) first
  (void)kv_tiles;
  const int b = (w % per_tile) / a.Hkv;
  const int hkv = w % a.Hkv;
  int start, S;
  seq_bounds(a, b, start, S);
  const int kb0 = kv_tile * BK;
  if (kb0 >= S) return;  // whole block, before any barrier

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r32 = lane & 31;
  const int g = lane >> 5;
  const int kw0 = kb0 + wave * 32;
  const int key = kw0 + r32;
  const bool key_ok = key < S;

  // this lane's key as the B operand of S = Q K^T and dP = dO V^T
  Frag kf[KK], vf[KK];
  {
    const T* krow = static_cast<const T*>(a.k) + b * a.ks[0] + hkv * a.ks[2] + (int64_t)(start + key) * a.ks[1];
    const T* vrow = static_cast<const T*>(a.v) + b * a.vs[0] + hkv * a.vs[2] + (int64_t)(start + key) * a.vs[1];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      uint4 kr = make_uint4(0, 0, 0, 0), vr = kr;
      if (key_ok) {
        kr = *reinterpret_cast<const uint4*>(krow + 16 * kk + 8 * g);
        vr = *reinterpret_cast<const uint4*>(vrow + 16 * kk + 8 * g);
      }
      kf[kk] = __builtin_bit_cast(Frag, kr);
      vf[kk] = __builtin_bit_cast(Frag, vr);
    }
  }

  // query tiles: every q head of the group, rows from the block's first key on (causal)
  const int u0 = CAUSAL ? kb0 / BQ : 0;
  const int n_u = (S + BQ - 1) / BQ - u0;
  const int n_it = a.group * n_u;

  const int kc = tid % KCH, kr = tid / KCH;  // staging: row kr (+ NT / KCH per pass), chunk kc
  constexpr int ROWS = NT / KCH;
  uint4 qreg[PER], greg[PER];
  float lreg = INFINITY, dreg = 0.f;
  auto load = [&](int it) {
    const int hq = hkv * a.group + it / n_u;
    const int u = u0 + it % n_u;
    const T* qb = static_cast<const T*>(a.q) + b * a.qs[0] + hq * a.qs[2] + start * a.qs[1];
    const T* gb = static_cast<const T*>(a.dout) + b * a.gs[0] + hq * a.gs[2] + start * a.gs[1];
    const __amdgpu_buffer_rsrc_t qrs =
        __builtin_amdgcn_make_buffer_rsrc((void*)qb, (short)0, (int)(((int64_t)(S - 1) * a.qs[1] + D) * (int)sizeof(T)),
                                          0x00020000);
    const __amdgpu_buffer_rsrc_t grs =
        __builtin_amdgcn_make_buffer_rsrc((void*)gb, (short)0, (int)(((int64_t)(S - 1) * a.gs[1] + D) * (int)sizeof(T)),
                                          0x00020000);
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int row = u * BQ + kr + p * ROWS;
      qreg[p] = flip(ld_buf(qrs, kc * 8 * (int)sizeof(T), row * (int)a.qs[1] * (int)sizeof(T)), a.q_flip);
      greg[p] = ld_buf(grs, kc * 8 * (int)sizeof(T), row * (int)a.gs[1] * (int)sizeof(T));
    }
    if (tid < BQ) {
      const int row = u * BQ + tid;
      const int64_t li = b * a.lse_bs + hq * a.lse_hs + start + row;
      lreg = row < S ? a.lse[li] * 1.4426950408889634f : INFINITY;
      dreg = row < S ? a.dsum[li] : 0.f;
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int off = L::at(kr + p * ROWS, kc * 8);
      *reinterpret_cast<uint4*>(Qs[buf] + off) = qreg[p];
      *reinterpret_cast<uint4*>(Gs[buf] + off) = greg[p];
    }
    if (tid < BQ) {
      Ls[buf][tid] = lreg;
      Dsm[buf][tid] = dreg;
    }
  };

  int a_lane[KK], t_lane[2][DT];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) a_lane[kk] = L::at(r32, 16 * kk + 8 * g);
#pragma unroll
  for (int hi = 0; hi < 2; ++hi)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      t_lane[hi][dt] = L::at(8 * hi + 4 * g + ((lane & 15) >> 2), 32 * dt + 16 * ((lane >> 4) & 1) + 4 * (lane & 3));

  f32x16 dv[DT], dk[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) dv[dt][r] = dk[dt][r] = 0.f;

  load(0);
  store(0);
  __syncthreads();
  for (int it = 0; it < n_it; ++it) {
    const int buf = it & 1;
    load(min(it + 1, n_it - 1));
    const int q0 = (u0 + it % n_u) * BQ;
    // skip tiles whose every query precedes every key of this wave
    if (!(CAUSAL && q0 + BQ - 1 < kw0)) {
      const T* qs = Qs[buf];
      const T* gs = Gs[buf];
      f32x16 s, dp;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        s = Mma<T>::run(*reinterpret_cast<const Frag*>(qs + a_lane[kk]), kf[kk], s);
        dp = Mma<T>::run(*reinterpret_cast<const Frag*>(gs + a_lane[kk]), vf[kk], dp);
      }
      // this lane's 16 queries: rows 8j + 4g + i of the tile (r = 4j + i)
      float l2[16], dd[16];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 lv = *reinterpret_cast<const float4*>(&Ls[buf][8 * j + 4 * g]);
        const float4 dv4 = *reinterpret_cast<const float4*>(&Dsm[buf][8 * j + 4 * g]);
        l2[4 * j] = lv.x;
        l2[4 * j + 1] = lv.y;
        l2[4 * j + 2] = lv.z;
        l2[4 * j + 3] = lv.w;
        dd[4 * j] = dv4.x;
        dd[4 * j + 1] = dv4.y;
        dd[4 * j + 2] = dv4.z;
        dd[4 * j + 3] = dv4.w;
      }
      const bool need_mask = (CAUSAL && q0 < kw0 + 32) || !key_ok;
      Frag pf[2], dsf[2];
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int r = 8 * c + j;
          float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], a.c, -l2[r]));
          if (need_mask) {
            const int qrow = q0 + 8 * (r >> 2) + 4 * g + (r & 3);
            p = key_ok && (!CAUSAL || key <= qrow) ? p : 0.f;
          }
          pf[c][j] = (T)p;
          dsf[c][j] = (T)(p * (dp[r] - dd[r]));
        }
      // dV^T += dO^T P and dK^T += Q^T dS, A operands from transposing reads
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const s16x4 glo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(gs + t_lane[0][dt] + 16 * c * L::ST));
          const s16x4 ghi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(gs + t_lane[1][dt] + 16 * c * L::ST));
          dv[dt] = Mma<T>::run(__builtin_bit_cast(Frag, __builtin_shufflevector(glo, ghi, 0, 1, 2, 3, 4, 5, 6, 7)),
                               pf[c], dv[dt]);
          const s16x4 qlo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(qs + t_lane[0][dt] + 16 * c * L::ST));
          const s16x4 qhi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(qs + t_lane[1][dt] + 16 * c * L::ST));
          dk[dt] = Mma<T>::run(__builtin_bit_cast(Frag, __builtin_shufflevector(qlo, qhi, 0, 1, 2, 3, 4, 5, 6, 7)),
                               dsf[c], dk[dt]);
        }
    }
    store(buf ^ 1);
    __syncthreads();
  }

  if (key_ok) {
    const float ks = fabsf(a.scale);
    T* dkrow = static_cast<T*>(a.dk) + b * a.dks[0] + hkv * a.dks[2] + (int64_t)(start + key) * a.dks[1];
    T* dvrow = static_cast<T*>(a.dv) + b * a.dvs[0] + hkv * a.dvs[2] + (int64_t)(start + key) * a.dvs[1];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int d0 = dt * 32 + 8 * rq + 4 * g;
        *reinterpret_cast<uint2*>(dvrow + d0) =
            pack4<T>(dv[dt][4 * rq], dv[dt][4 * rq + 1], dv[dt][4 * rq + 2], dv[dt][4 * rq + 3]);
        *reinterpret_cast<uint2*>(dkrow + d0) = pack4<T>(dk[dt][4 * rq] * ks, dk[dt][4 * rq + 1] * ks,
                                                         dk[dt][4 * rq + 2] * ks, dk[dt][4 * rq + 3] * ks);
      }
  }
}

template <typename T, int D>
int launch(const BwdArgs& a, bool causal, hipStream_t s) {
  const int64_t dq_blocks = (int64_t)((a.S + BM - 1) / BM) * a.B * a.Hq;
  const int64_t kv_blocks = (int64_t)((a.S + BK - 1) / BK) * a.B * a.Hkv;
  if (causal) {
    hipLaunchKernelGGL((attn_bwd_dq_kernel<T, D, true>), dim3(dq_blocks), dim3(NT), 0, s, a);
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<T, D, true>), dim3(kv_blocks), dim3(NT), 0, s, a);
  } else {
    hipLaunchKernelGGL((attn_bwd_dq_kernel<T, D, false>), dim3(dq_blocks), dim3(NT), 0, s, a);
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<T, D, false>), dim3(kv_blocks), dim3(NT), 0, s, a);
  }
  return launched("pk_attn_bwd");
}

// strides[24] = q, k, v, o, dout, dq, dk, dv (batch, token, head)
int bwd_launch(const char* who, BwdArgs a, const int64_t* strides, int64_t batch, int64_t seq, int64_t q_heads,
               int64_t kv_heads, int64_t head_dim, float softmax_scale, int causal, int dtype, void* stream) {
  if (batch < 0 || seq < 0 || q_heads < 0 || kv_heads < 0 || head_dim < 0)
    return fail(PK_ERR_INVALID, "%s: negative size", who);
  if (batch == 0 || seq == 0 || q_heads == 0) return PK_OK;
  if (!a.q || !a.k || !a.v || !a.o || !a.dout || !a.lse || !a.dsum || !a.dq || !a.dk || !a.dv || !strides)
    return fail(PK_ERR_INVALID, "%s: null pointer", who);
  if (kv_heads == 0 || q_heads % kv_heads != 0)
    return fail(PK_ERR_INVALID, "%s: q_heads=%lld is not a multiple of kv_heads=%lld", who, (long long)q_heads,
                (long long)kv_heads);
  if (dtype != PK_BF16 && dtype != PK_F16) return fail(PK_ERR_UNSUPPORTED, "%s: dtype code %d (bf16/fp16 only)", who, dtype);
  if (head_dim != 64 && head_dim != 128)
    return fail(PK_ERR_UNSUPPORTED, "%s: head_dim=%lld (64 or 128 only)", who, (long long)head_dim);
  if (!isfinite(softmax_scale)) return fail(PK_ERR_INVALID, "%s: softmax_scale is not finite", who);
  if (seq > (1 << 30) || batch * q_heads > (1 << 20)) return fail(PK_ERR_UNSUPPORTED, "%s: shape too large", who);
  const void* ptrs[] = {a.q, a.k, a.v, a.o, a.dout, a.dq, a.dk, a.dv};
  for (const void* p : ptrs)
    if (!aligned16(p)) return fail(PK_ERR_INVALID, "%s: tensors must be 16-byte aligned", who);
  for (int i = 0; i < 24; ++i)
    if (strides[i] % 8 != 0 || strides[i] < 0)
      return fail(PK_ERR_INVALID, "%s: stride %d = %lld is not a non-negative multiple of 8", who, i,
                  (long long)strides[i]);
  int64_t* dst[] = {a.qs, a.ks, a.vs, a.os, a.gs, a.dqs, a.dks, a.dvs};
  for (int t = 0; t < 8; ++t)
    for (int i = 0; i < 3; ++i) dst[t][i] = strides[3 * t + i];
  // buffer offsets are 32-bit: rows of one sequence (plus a tile past the end) must fit
  int64_t widest = 0;
  for (int t = 0; t < 5; ++t) widest = dst[t][1] > widest ? dst[t][1] : widest;
  if ((seq + 2 * BK) * widest * 2 + head_dim * 2 > INT32_MAX)
    return fail(PK_ERR_UNSUPPORTED, "%s: rows span more than 2 GiB per head", who);
  a.B = (int)batch;
  a.S = (int)seq;
  a.Hq = (int)q_heads;
  a.Hkv = (int)kv_heads;
  a.group = (int)(q_heads / kv_heads);
  a.scale = softmax_scale;
  a.c = fmaxf(fabsf(softmax_scale) * 1.4426950408889634f, 1e-30f);
  a.q_flip = softmax_scale < 0.f ? 0x80008000u : 0u;
  if ((seq + BM - 1) / BM * batch * q_heads > INT32_MAX) return fail(PK_ERR_UNSUPPORTED, "%s: grid too large", who);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == PK_BF16) return head_dim == 64 ? launch<bf16, 64>(a, causal, s) : launch<bf16, 128>(a, causal, s);
  return head_dim == 64 ? launch<f16, 64>(a, causal, s) : launch<f16, 128>(a, causal, s);
}

}  // namespace
}  // namespace pk

extern "C" {

int pk_attn_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout, const float* lse,
                float* dsum, void* dq, void* dk, void* dv, const int64_t* strides, int64_t batch, int64_t seq,
                int64_t q_heads, int64_t kv_heads, int64_t head_dim, float softmax_scale, int causal, int dtype,
                void* stream) {
  using namespace pk;
  BwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.dout = dout;
  a.lse = lse;
  a.dsum = dsum;
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  a.cu = nullptr;
  a.lse_bs = q_heads * seq;  // [batch, q_heads, seq]
  a.lse_hs = seq;
  return bwd_launch("pk_attn_bwd", a, strides, batch, seq, q_heads, kv_heads, head_dim, softmax_scale, causal, dtype,
                    stream);
}

int pk_attn_varlen_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout, const float* lse,
                       float* dsum, void* dq, void* dk, void* dv, const int* cu_seqlens, const int64_t* strides,
                       int64_t num_seqs, int64_t total, int64_t max_seqlen, int64_t q_heads, int64_t kv_heads,
                       int64_t head_dim, float softmax_scale, int causal, int dtype, void* stream) {
  using namespace pk;
  const char* who = "pk_attn_varlen_bwd";
  if (num_seqs < 0 || total < 0 || max_seqlen < 0) return fail(PK_ERR_INVALID, "%s: negative size", who);
  if (num_seqs == 0 || total == 0 || max_seqlen == 0) return PK_OK;
  if (!cu_seqlens || !strides) return fail(PK_ERR_INVALID, "%s: null pointer", who);
  if (total > INT32_MAX || max_seqlen > total)
    return fail(PK_ERR_INVALID, "%s: max_seqlen %lld exceeds total %lld", who, (long long)max_seqlen, (long long)total);
  // packed tensors have no batch dimension: strides[16] are (token, head) of q, k, v, o, dout, dq, dk, dv
  int64_t dense[24];
  for (int t = 0; t < 8; ++t) {
    dense[3 * t] = 0;
    dense[3 * t + 1] = strides[2 * t];
    dense[3 * t + 2] = strides[2 * t + 1];
  }
  BwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.dout = dout;
  a.lse = lse;
  a.dsum = dsum;
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  a.cu = cu_seqlens;
  a.total = (int)total;
  a.lse_bs = 0;  // [q_heads, total]
  a.lse_hs = total;
  return bwd_launch(who, a, dense, num_seqs, max_seqlen, q_heads, kv_heads, head_dim, softmax_scale, causal, dtype,
                    stream);
}

}  // extern "C"
