// Attention backward (grouped-query, optional causal mask, dense batches or
// packed sequences) on gfx950 matrix cores, in two deterministic kernels
// that never add into shared memory of another block:
//
//   dq kernel   one block = 4 waves x 32 query rows over one (sequence, kv
//               head): gp of its q heads x 4/gp row groups, as in the
//               forward; keys streamed through LDS in tiles of 32. Per tile
//               each wave recomputes S^T = K Q^T and dP^T = V dO^T, forms
//               P = exp2(s*c - lse2) from the forward's log-sum-exp and
//               dS = P (dP - D), and accumulates dQ^T += K^T dS^T, with the
//               dQ products of one tile interleaved with the S and dP
//               products of the next (software-pipelined). Its prologue
//               also computes D = rowsum(dO * O) for its rows and stores it,
//               with lse2 = lse * log2(e), for the second kernel.
//   dkdv kernel one block = 128 keys of one (sequence, kv head) in four
//               32-key slices, two waves per slice sharing a SIMD; query tiles
//               of 32 rows (over every q head of the group) stream through
//               LDS. The slice's role-0 wave holds K and computes S = Q K^T,
//               whose result layout puts one key per lane column, so
//               P = exp2(s*c - lse2) goes straight into dV^T += dO^T P as the
//               B operand; it also leaves P (as fp16) in LDS. The role-1 wave
//               holds V, computes dP = dO V^T one step later, reads that P,
//               forms dS = P (dP - D) and accumulates dK^T += Q^T dS. Splitting
//               the roles halves each wave's registers (one fragment set, one
//               accumulator), which is what lets two waves share each SIMD
//               (four at head_dim 64, whose kernel fits 128 registers, so
//               two blocks share a CU).
//               Each step is software-pipelined: a wave forms the factors of
//               one tile from the score block it computed in the step before,
//               then runs that tile's accumulation interleaved with the next
//               tile's score block. Query tiles (with their lse2 and D rows)
//               arrive through six LDS stages, two tiles in flight beyond the
//               three a step reads. A block walks its q heads' tiles one
//               after another, so when the grid is too small to fill the
//               device the q heads of each group are split over several blocks
//               that leave fp32 partials, and a third kernel adds them in
//               split order (still deterministic).
//
// Both kernels stage tiles with buffer loads that write LDS directly (16
// bytes per lane at the wave's LDS base + 16 * lane): each lane fetches the
// global chunk that its LDS slot holds under the swizzle below, so no staging
// registers or LDS stores are needed. Rows past the end read as zero.
//
// With scores z = scale * q.k: dS = dL/dz, dQ = scale * dS K,
// dK = scale * dS^T Q, dV = P^T dO. In the dq kernel a negative scale is
// applied as in the forward (Q negated on load, c = |scale| log2 e), so dQ
// takes the signed scale; the dkdv kernel stages Q unchanged and uses the
// signed c and the signed scale for dK.
//
// LDS tiles are unpadded rows of 16-byte chunks, chunk c of row r stored at
// c ^ swz(r): swz(r) = 4 (r % 4) + (r / 4) % 4 for head_dim 128 and 256 (rows
// span all 64 banks, or twice) and 4 ((r / 2) % 2) + (r / 4) % 4 for head_dim
// 64 (two rows per bank sweep). Either way the 16-byte fragment reads (16
// rows, one chunk) and the transposing ds_read_b64_tr_b16 reads (4 rows x 4
// chunks per pair of 16-lane groups) land on 64 distinct banks.
//
// head_dim 256 (attn_bwd_wide.h) keeps this dq kernel, at one wave per SIMD,
// and replaces the dkdv kernel, whose six stages would not fit in LDS at that
// width, with a single-role kernel.
#include <math.h>

#include <type_traits>

#include "api.h"
#include "attn_common.h"

namespace pk {
namespace {

using namespace attn;

constexpr int NT = 256;
constexpr int BM = 128;  // dq kernel: query rows per block times q heads per block
constexpr int BN = 32;   // dq kernel: keys per tile
constexpr int BK = 128;  // dkdv kernel: keys per block
constexpr int BQ = 32;   // dkdv kernel: query rows per tile
constexpr int kRingDq = 3;    // dq kernel: fragment reads in flight ahead of their product
template <int D> constexpr int kRingDkdv = D == 32 ? 4 : 5;  // dkdv kernel: the same (at most a step's products)

struct BwdArgs {
  const void *q, *k, *v, *o, *dout;
  const float* lse;  // natural log, laid out like dsum
  float* dsum;       // D = rowsum(dO * O): element (b, h, token t of b) at b*lse_bs + h*lse_hs + t (+ start)
  void *dq, *dk, *dv;
  const int* cu;  // packed sequences (see pk_attn_varlen_fwd) or NULL
  int total;
  int64_t qs[3], ks[3], vs[3], os[3], gs[3], dqs[3], dks[3], dvs[3];  // (batch, token, head) strides
  int64_t lse_bs, lse_hs;
  int64_t lse_n;  // elements of lse; dsum[lse_n + i] holds lse[i] * log2(e)
  // dk/dv head split: nsplit > 1 blocks per (key tile, kv head), each over
  // group / nsplit of its q heads, leave fp32 partials in part
  // [nsplit][2 (dV, dK)][rows][Hkv][D] (rows: batch * S tokens, or total when
  // packed), summed in split order by dkdv_sum_kernel
  float* part;
  int nsplit;
  int64_t rows;
  int B, S, Hq, Hkv, group;
  float scale;  // signed softmax scale
  float c;      // |scale| * log2(e), at least 1e-30
  uint32_t q_flip;
  // head_dim of the tensors (a multiple of 8, at most the kernels' D) and its
  // 16-byte chunks: rows are laid out at D, reading zeros past head_dim
  int dr, dch;
};

// Buffer offset of a chunk past head_dim: at or past every range the kernels
// build (each below 2^31), and with a tile offset below 2^31 added it cannot
// wrap, so the load returns zeros without a memory access.
constexpr uint32_t kPadOffset = 0x80000000u;

// LDS tile layout: unpadded rows, 16-byte chunk c of row r at c ^ swz(r)
// (head_dim 256 rows span two bank sweeps; chunk c % 16 picks the banks, so
// they take head_dim 128's swizzle)
template <int D> struct Tile {
  static constexpr int ST = D;
  static __device__ __forceinline__ int swz(int row) {
    if constexpr (D == 32 || D == 96)  // 4 or 12 chunks: rows start 64 bytes apart in a bank window, period 4
      return (row >> 2) & 3;
    else if constexpr (D == 192)  // 24 chunks: rows start 128 bytes apart; the swizzle stays in groups of 8 chunks
      return (4 * ((row >> 1) & 1)) | ((row >> 2) & 1) | (2 * ((row >> 3) & 1));
    else if constexpr (D >= 128)
      return 4 * (row & 3) + ((row >> 2) & 3);
    else
      return 4 * ((row >> 1) & 1) + ((row >> 2) & 3);
  }
  // element offset of (row, dim), dim a multiple of 4
  static __device__ __forceinline__ int at(int row, int dim) {
    return row * D + ((((dim >> 3) ^ swz(row)) << 3) | (dim & 7));
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

// head_dim 192 and 256 hold Q, dO and the dQ accumulator in 192 or 256 registers: one wave per SIMD.
// KS: 16-dim steps of the S and dP products, D / 16, or one fewer when the
// row's last 16 dims are all past head_dim (zeros in every operand of that
// step, so skipping it changes no bit)
template <typename T, int D, bool CAUSAL, int KS = D / 16>
__global__ __attribute__((amdgpu_flat_work_group_size(NT, NT), amdgpu_waves_per_eu(D >= 192 ? 1 : 2))) void attn_bwd_dq_kernel(
    BwdArgs a) {
  using Frag = typename Mma<T>::frag;
  using L = Tile<D>;
  constexpr int KCH = D / 8;
  constexpr int TSLOTS = BN * KCH;   // 16-byte slots of a K (or V) tile
  constexpr int TI = (TSLOTS + NT - 1) / NT;  // direct loads per thread per tile of K (and of V): 4, 2 or 1
  // 96-dim rows: a tile is 384 slots, and the second load of waves 2 and 3
  // lies past it; they load nothing (out of range) into `spill`, so every wave
  // issues the same loads and its vmcnt counts hold
  constexpr bool TFULL = TSLOTS % NT == 0;
  constexpr int KK = D / 16;
  constexpr int DT = D / 32;
  constexpr int NSQ = 4;  // K/V tile stages: the two tiles a step reads, one in flight, one landing
  static_assert(KS == KK || KS == KK - 1, "at most the last 16-dim step is skipped");
  __shared__ __attribute__((aligned(16))) T Ks[NSQ][BN * L::ST];
  __shared__ __attribute__((aligned(16))) T Vs[NSQ][BN * L::ST];
  __shared__ __attribute__((aligned(16))) T spill[TFULL ? 8 : 64 * 8];

  // work item: (q tile, batch, kv head, head quad), longest causal rows
  // first; the waves are gp q heads of one kv group (gp = 4, 2 or 1, the
  // largest dividing the group size) x 4/gp row groups of 32, so with a group
  // of 4 every wave covers the same rows and the same keys
  const int G = a.group;
  const int GP = G % 4 == 0 ? 4 : (G % 2 == 0 ? 2 : 1);
  const int rows_per_block = 32 * (4 / GP);
  const int m_tiles = (a.S + rows_per_block - 1) / rows_per_block;
  const int n_quads = G / GP;
  const int per_tile = a.B * a.Hkv * n_quads;
  const int w = blockIdx.x;
  int m_tile, rest;
  if (per_tile % 8 == 0) {  // group-major per XCD, as in the forward
    const int k = w >> 3;
    m_tile = m_tiles - 1 - k % m_tiles;
    rest = (w & 7) + 8 * (k / m_tiles);
  } else {
    m_tile = m_tiles - 1 - w / per_tile;
    rest = w % per_tile;
  }
  const int b = rest / (a.Hkv * n_quads);
  const int hkv = (rest / n_quads) % a.Hkv;
  const int hq = hkv * G + (rest % n_quads) * GP + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) % GP;
  int start, S;
  seq_bounds(a, b, start, S);
  const int m0 = m_tile * rows_per_block;
  if (m0 >= S) return;  // whole block, before any barrier

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r32 = lane & 31;
  const int g = lane >> 5;
  const int wave_first = m0 + (wave / GP) * 32;
  const int q_row = wave_first + r32;
  const bool row_ok = q_row < S;

  const T* qbase = static_cast<const T*>(a.q) + b * a.qs[0] + hq * a.qs[2] + start * a.qs[1];
  const T* obase = static_cast<const T*>(a.o) + b * a.os[0] + hq * a.os[2] + start * a.os[1];
  const T* gbase = static_cast<const T*>(a.dout) + b * a.gs[0] + hq * a.gs[2] + start * a.gs[1];
  const T* kbase = static_cast<const T*>(a.k) + b * a.ks[0] + hkv * a.ks[2] + start * a.ks[1];
  const T* vbase = static_cast<const T*>(a.v) + b * a.vs[0] + hkv * a.vs[2] + start * a.vs[1];
  const int k_bytes = (int)(((int64_t)(S - 1) * a.ks[1] + a.dr) * (int)sizeof(T));
  const int v_bytes = (int)(((int64_t)(S - 1) * a.vs[1] + a.dr) * (int)sizeof(T));
  const __amdgpu_buffer_rsrc_t krsrc = __builtin_amdgcn_make_buffer_rsrc((void*)kbase, (short)0, k_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrsrc = __builtin_amdgcn_make_buffer_rsrc((void*)vbase, (short)0, v_bytes, 0x00020000);
  // Rows of 192 and 256 dims (one wave per SIMD) stage their tiles through the
  // inline-assembly loads, so the step's fragment reads do not first wait for
  // the step's own prefetch; each step then waits for all of its loads before
  // its closing barrier. (Measured slower at the narrower rows.)
  constexpr bool kAsmLoads = D >= 192;
  const rsrc_words kwords = make_rsrc_words(kbase, k_bytes), vwords = make_rsrc_words(vbase, v_bytes);

  // Q^T and dO^T fragments of this lane's row (B operands), and D = rowsum(dO * O)
  Frag qf[KK], gf[KK];
  float dsum = 0.f;
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
    uint4 qr = make_uint4(0, 0, 0, 0), gr = qr, orr = qr;
    if (row_ok && 2 * kk + g < a.dch) {
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
  if (row_ok && g == 0) {
    a.dsum[lidx] = dsum;
    a.dsum[a.lse_n + lidx] = lse2;
  }
  if constexpr (kAsmLoads) {  // the compiler's own loads complete before the first inline-assembly load
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) asm volatile("" ::"v"(qf[kk]), "v"(gf[kk]));
    asm volatile("" ::"v"(lse2), "v"(dsum));
  }

  const int kv_end = CAUSAL ? min(m0 + rows_per_block, S) : S;
  const int n_tiles = (kv_end + BN - 1) / BN;

  // staging straight into LDS: slot i*NT + tid of a tile is row sl / KCH,
  // stored chunk sl % KCH, which holds logical chunk (sl % KCH) ^ swz(row)
  int kgo[TI], vgo[TI];
#pragma unroll
  for (int i = 0; i < TI; ++i) {
    const int sl = i * NT + tid, row = sl / KCH, c = (sl % KCH) ^ L::swz(row);
    const bool in = c < a.dch && sl < TSLOTS;
    kgo[i] = in ? (row * (int)a.ks[1] + c * 8) * (int)sizeof(T) : (int)kPadOffset;
    vgo[i] = in ? (row * (int)a.vs[1] + c * 8) * (int)sizeof(T) : (int)kPadOffset;
  }
  auto issue = [&](int t, int buf) {
#pragma unroll
    for (int i = 0; i < TI; ++i) {
      const bool in = TFULL || i * NT + wave * 64 < TSLOTS;  // wave-uniform
      T* kl = in ? Ks[buf] + (i * NT + wave * 64) * 8 : spill;
      T* vl = in ? Vs[buf] + (i * NT + wave * 64) * 8 : spill;
      const int ko = t * BN * (int)a.ks[1] * (int)sizeof(T), vo = t * BN * (int)a.vs[1] * (int)sizeof(T);
      if constexpr (kAsmLoads) {
        ld_lds16_asm(kwords, kl, kgo[i], ko);
        ld_lds16_asm(vwords, vl, vgo[i], vo);
      } else {
        ld_buf_lds(krsrc, kl, kgo[i], ko);
        ld_buf_lds(vrsrc, vl, vgo[i], vo);
      }
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

  // Software-pipelined steps, as in the dk/dv kernel: step t forms dS of
  // tile u = t - 1 from the S and dP blocks computed in step t - 1, then runs
  // tile u's dQ products interleaved with the S and dP products of tile u + 1.
  // Step t reads tiles t - 1 and t, issues tile t + NSQ - 2 into the stage of
  // tile t - 2 (last read in step t - 1) and ends once tile t + 1 has landed.
  // Tile indices are clamped into the range at the edges, where dS is zero.
  // (Tiles wholly past a wave's rows are masked to zero, not skipped.)
#pragma unroll
  for (int j = 0; j < NSQ - 2; ++j) issue(min(j, n_tiles - 1), j);
  lds_loads_landed();  // all of them: the dsum stores above share the counter
  __syncthreads();
  // product 3h: dQ step h (A = K^T from transposing reads of the tile at ka:
  // 16 keys c = h / DT, dims 32 (h % DT) ..; B = dsf[c]); 3h + 1: S^T step h
  // (A = K fragment h of the tile at kn, B = Q^T); 3h + 2: dP^T step h (A = V
  // fragment h of the tile at vn, B = dO^T). With KS < KK the run ends with
  // the last dQ step alone. Reads run kRingDq products ahead.
  constexpr int RING = kRingDq;
  constexpr int NP = KK + 2 * KS;
  static_assert(RING <= NP, "the ring's first reads stay inside the run");
  // product i: its kind (0 dQ, 1 S^T, 2 dP^T) and step h
  auto kind = [](int i) { return i < 3 * KS ? i % 3 : 0; };
  auto step_of = [](int i) { return i < 3 * KS ? i / 3 : KS + (i - 3 * KS); };
  f32x16 s, dp;  // S^T and dP^T of the wave's next tile
  auto run = [&](const T* ka, const Frag (&dsf)[2], const T* kn, const T* vn) {
    auto fetch = [&](int i) -> Frag {
      const int h = step_of(i);
      if (kind(i) == 1) return *reinterpret_cast<const Frag*>(kn + a_lane[h]);
      if (kind(i) == 2) return *reinterpret_cast<const Frag*>(vn + a_lane[h]);
      const int c = h / DT, dt = h % DT;
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(ka + t_lane[0][dt] + 16 * c * L::ST));
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(ka + t_lane[1][dt] + 16 * c * L::ST));
      return __builtin_bit_cast(Frag, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    };
    Frag ring[RING];
#pragma unroll
    for (int i = 0; i < RING; ++i) ring[i] = fetch(i);
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const Frag f = ring[i % RING];
      if (i + RING < NP) ring[i % RING] = fetch(i + RING);
      const int h = step_of(i);
      if (kind(i) == 0)
        acc[h % DT] = Mma<T>::run(f, dsf[h / DT], acc[h % DT]);
      else if (kind(i) == 1)
        s = Mma<T>::run(f, qf[h], s);
      else
        dp = Mma<T>::run(f, gf[h], dp);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  const int lim = CAUSAL ? min(q_row, S - 1) : S - 1;
  // Tile j sits in stage j % NSQ, so step t >= 1 reads stages (t - 1) % NSQ
  // and t % NSQ and issues into (t + 2) % NSQ. The steps are unrolled over the
  // four stage phases: every LDS fragment address is then a lane register
  // plus an immediate, with no per-step address arithmetic. The last step
  // (t = n_tiles) computes S and dP of stage n_tiles % NSQ, which holds a copy
  // of the last tile (clamped issue), and discards them.
  auto dscores = [&](int u, Frag (&dsf)[2]) {
    // dS = P (dP - D), P = exp2(s c - lse2); keys a row must not see get 0.
    // The test for a mask is wave-uniform, so unmasked tiles branch past it.
    const int kv0 = u * BN;
    const bool need_mask = (CAUSAL && kv0 + BN - 1 > wave_first) || kv0 + BN > S;
    if (need_mask) {
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int r = 8 * c + j;
          const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], a.c, -lse2));
          const float p = kv0 + 8 * (r >> 2) + 4 * g + (r & 3) <= lim ? e : 0.f;
          dsf[c][j] = (T)(p * (dp[r] - dsum));
        }
    } else {
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int r = 8 * c + j;
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], a.c, -lse2));
          dsf[c][j] = (T)(p * (dp[r] - dsum));
        }
    }
  };
  auto finish = [&]() {
    if constexpr (kAsmLoads)
      lds_loads_landed();
    else
      loads_landed_but<(NSQ - 3) * 2 * TI>();
    __syncthreads();
  };
  {
    // step 0: no dS yet (zero factors against the loaded stage 0); S^T, dP^T of tile 0
    issue(min(NSQ - 2, n_tiles - 1), NSQ - 2);
    Frag dsf[2];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) dsf[c][j] = (T)0.f;
    run(Ks[0], dsf, Ks[0], Vs[0]);
    finish();
  }
  auto step = [&](int t, auto phase) {
    constexpr int P = decltype(phase)::value;
    constexpr int PA = (P + NSQ - 1) % NSQ;
    issue(min(t + NSQ - 2, n_tiles - 1), (P + NSQ - 2) % NSQ);
    Frag dsf[2];
    dscores(t - 1, dsf);
    run(Ks[PA], dsf, Ks[P], Vs[P]);  // dQ^T += K^T dS^T; S^T, dP^T of the next tile
    finish();
  };
  static_assert(NSQ == 4, "the step loop is unrolled over four stage phases");
  for (int t = 1;;) {
    step(t, std::integral_constant<int, 1>{});
    if (++t > n_tiles) break;
    step(t, std::integral_constant<int, 2>{});
    if (++t > n_tiles) break;
    step(t, std::integral_constant<int, 3>{});
    if (++t > n_tiles) break;
    step(t, std::integral_constant<int, 0>{});
    if (++t > n_tiles) break;
  }
  lds_loads_landed();  // tiles issued past the end, before the block's LDS is released

  if (row_ok) {
    T* drow = static_cast<T*>(a.dq) + b * a.dqs[0] + hq * a.dqs[2] + (int64_t)(start + q_row) * a.dqs[1];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq)
        if (dt * 32 + 8 * rq + 4 * g < a.dr)
          *reinterpret_cast<uint2*>(drow + dt * 32 + 8 * rq + 4 * g) =
              pack4<T>(acc[dt][4 * rq] * a.scale, acc[dt][4 * rq + 1] * a.scale, acc[dt][4 * rq + 2] * a.scale,
                     acc[dt][4 * rq + 3] * a.scale);
  }
}

// ---------------------------------------------------------------- dkdv kernel

constexpr int NT2 = 512;  // dkdv kernel: 8 waves, two per SIMD

// head_dim 32 and 64 fit 128 registers, so two blocks (or more) share a CU (four waves per SIMD).
// KS: 16-dim steps of the score products (S, dP), as in the dq kernel
template <typename T, int D, bool CAUSAL, int KS = D / 16>
__global__ __attribute__((amdgpu_flat_work_group_size(NT2, NT2), amdgpu_waves_per_eu(D <= 64 ? 4 : 2))) void attn_bwd_dkdv_kernel(
    BwdArgs a) {
  using Frag = typename Mma<T>::frag;
  using L = Tile<D>;
  constexpr int KCH = D / 8;             // 16-byte chunks per row
  constexpr int SLOTS = BQ * KCH;        // 16-byte slots of a Q (or dO) tile: 512 or 256
  constexpr int TI = (2 * SLOTS + NT2 - 1) / NT2;  // direct loads per thread per tile (Q and dO together): 2 or 1
  // 96-dim rows: a stage is 768 slots, and the second load of waves 4-7 lies
  // past it; they load nothing (out of range) into `tspill`, so every wave
  // issues the same loads and its vmcnt counts hold
  constexpr bool TFULL = 2 * SLOTS % NT2 == 0;
  constexpr int NS = 6;                  // query tiles resident or in flight in LDS
  constexpr int PER_ISSUE = TI + 1;      // loads each wave issues per tile (tiles, one row vector)
  constexpr int TILE = BQ * D;
  constexpr int KK = D / 16;
  constexpr int DT = D / 32;
  static_assert(KS == KK || KS == KK - 1, "at most the last 16-dim step is skipped");
  // stage: Q tile then dO tile; row vectors: lse2, then D (64 slots: whole-wave loads)
  __shared__ __attribute__((aligned(16))) T QG[NS][2 * TILE];
  __shared__ __attribute__((aligned(16))) float RV[NS][2][64];
  __shared__ __attribute__((aligned(16))) float spill[64];
  __shared__ __attribute__((aligned(16))) T tspill[TFULL ? 8 : 64 * 8];
  // P of each key slice as fp16 (P <= 1; 11 significant bits, more than the
  // rounded dS it feeds), double-buffered: [buffer][slice][16 values x 64 lanes]
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  __shared__ __attribute__((aligned(16))) _Float16 Pb[2][4][16 * 64];

  const int w = blockIdx.x;
  const int per_tile = a.B * a.Hkv * a.nsplit;
  // first key tiles (the most causal work) first. (Group-major order per XCD,
  // as the forward and dq kernels use, measured 26 % more HBM fetch here: a
  // block streams its group's whole Q/dO from its own key tile on, and the
  // 32 resident blocks of one group start at 32 different places.)
  const int kv_tile = w / per_tile;
  const int gi = w % per_tile;
  const int b = gi / (a.Hkv * a.nsplit);
  const int hkv = (gi / a.nsplit) % a.Hkv;
  const int split = gi % a.nsplit;
  const int heads = a.group / a.nsplit;  // q heads this block walks, from split * heads on
  int start, S;
  seq_bounds(a, b, start, S);
  const int kb0 = kv_tile * BK;
  if (kb0 >= S) return;  // whole block, before any barrier

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // waves w and w + 4 share a SIMD and a key slice: role 0 (waves 0-3) forms
  // P from S = Q K^T and accumulates dV; role 1 (waves 4-7) forms dS from
  // dP = dO V^T and the P role 0 left in LDS, and accumulates dK
  const int role = wave >> 2;
  const int slice = wave & 3;
  const int lane = tid & 63;
  const int r32 = lane & 31;
  const int g = lane >> 5;
  const int kw0 = kb0 + slice * 32;
  const int key = kw0 + r32;
  const bool key_ok = key < S;

  // this lane's key row as the B operand: K (role 0) or V (role 1)
  Frag bf[KK];
  {
    const T* row = role == 0
                       ? static_cast<const T*>(a.k) + b * a.ks[0] + hkv * a.ks[2] + (int64_t)(start + key) * a.ks[1]
                       : static_cast<const T*>(a.v) + b * a.vs[0] + hkv * a.vs[2] + (int64_t)(start + key) * a.vs[1];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      uint4 r = make_uint4(0, 0, 0, 0);
      if (key_ok && 2 * kk + g < a.dch) r = *reinterpret_cast<const uint4*>(row + 16 * kk + 8 * g);
      bf[kk] = __builtin_bit_cast(Frag, r);
    }
  }
  // Q is staged unflipped: a negative scale signs the exponent's coefficient
  // here and dK's final scale
  const float cs = a.q_flip ? -a.c : a.c;

  // query tiles: every q head of the group, rows from the block's first key on (causal)
  const int u0 = CAUSAL ? kb0 / BQ : 0;
  const int n_u = (S + BQ - 1) / BQ - u0;
  const int n_it = heads * n_u;

  // staging: slot sl = i*NT2 + tid of the stage (Q slots, then dO slots) is
  // row (sl % SLOTS) / KCH of that tile, stored chunk sl % KCH, which holds
  // logical chunk (sl % KCH) ^ swz(row); a wave's 64 slots lie in one tile
  int go[TI];
#pragma unroll
  for (int i = 0; i < TI; ++i) {
    const int sl = i * NT2 + tid, op = sl / SLOTS, within = sl % SLOTS;
    const int row = within / KCH, c = (within % KCH) ^ L::swz(row);
    go[i] = c < a.dch && op < 2 ? (row * (int)(op == 0 ? a.qs[1] : a.gs[1]) + c * 8) * (int)sizeof(T)
                                : (int)kPadOffset;
  }
  // Tiles are issued in order: a cursor holds the next tile's q head (within
  // the group) and q tile, and the buffer descriptors of that head, rebuilt
  // only when the head changes; past the end the last tile is issued again.
  // Rows past the end read as zero; their p is masked. Wave 0 also loads the
  // rows' lse2, wave 1 their D, the other waves repeat D into `spill`.
  int cur_h = 0, cur_u = 0, cur_it = 0;
  __amdgpu_buffer_rsrc_t trs[TI], rrs;
  int tstride[TI];  // bytes per row of the tensor each of this wave's tile loads reads
  auto set_head = [&](int h) {
    const int hq = hkv * a.group + split * heads + h;
    const T* qb = static_cast<const T*>(a.q) + b * a.qs[0] + hq * a.qs[2] + start * a.qs[1];
    const T* gb = static_cast<const T*>(a.dout) + b * a.gs[0] + hq * a.gs[2] + start * a.gs[1];
    const float* db = a.dsum + b * a.lse_bs + hq * a.lse_hs + start;
#pragma unroll
    for (int i = 0; i < TI; ++i) {
      const bool isq = i * NT2 + wave * 64 < SLOTS;  // wave-uniform
      tstride[i] = (int)(isq ? a.qs[1] : a.gs[1]) * (int)sizeof(T);
      trs[i] = __builtin_amdgcn_make_buffer_rsrc((void*)(isq ? qb : gb), (short)0,
                                                 (int)(((int64_t)(S - 1) * (isq ? a.qs[1] : a.gs[1]) + a.dr) * (int)sizeof(T)),
                                                 0x00020000);
    }
    rrs = __builtin_amdgcn_make_buffer_rsrc((void*)(wave == 0 ? db + a.lse_n : db), (short)0, S * (int)sizeof(float),
                                            0x00020000);
  };
  set_head(0);
  // the cursor's tile into stage st, then advance the cursor
  auto issue = [&](int st) {
    const int r0 = (u0 + cur_u) * BQ;
#pragma unroll
    for (int i = 0; i < TI; ++i) {
      const bool in = TFULL || i * NT2 + wave * 64 < 2 * SLOTS;  // wave-uniform
      ld_buf_lds(trs[i], in ? QG[st] + (i * NT2 + wave * 64) * 8 : tspill, go[i], r0 * tstride[i]);
    }
    ld_buf_lds4(rrs, wave == 0 ? RV[st][0] : (wave == 1 ? RV[st][1] : spill), lane * (int)sizeof(float),
                r0 * (int)sizeof(float));
    if (cur_it + 1 < n_it) {
      ++cur_it;
      if (++cur_u == n_u) {
        cur_u = 0;
        set_head(++cur_h);
      }
    }
  };

  // Lane offsets of the fragment reads within a stage, with the wave's half of
  // the stage folded in: role 0 accumulates from dO (second half) and scores
  // against Q (first half), role 1 the other way round.
  const int a_half = role == 0 ? 0 : TILE, t_half = role == 0 ? TILE : 0;
  int a_lane[KK], t_lane[2][DT];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) a_lane[kk] = a_half + L::at(r32, 16 * kk + 8 * g);
#pragma unroll
  for (int hi = 0; hi < 2; ++hi)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      t_lane[hi][dt] =
          t_half + L::at(8 * hi + 4 * g + ((lane & 15) >> 2), 32 * dt + 16 * ((lane >> 4) & 1) + 4 * (lane & 3));

  f32x16 acc[DT];  // dV (role 0) or dK (role 1)
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[dt][r] = 0.f;

  // this lane's 16 values of a tile's row vector v (rows 8j + 4g + i, r = 4j + i)
  auto rows16 = [&](const float* v, float (&out)[16]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 x = *reinterpret_cast<const float4*>(v + 8 * j + 4 * g);
      out[4 * j] = x.x;
      out[4 * j + 1] = x.y;
      out[4 * j + 2] = x.z;
      out[4 * j + 3] = x.w;
    }
  };
  // P buffer layout: value r of lane l at (r / 8) * 512 + 8 * l + r % 8 (16-byte lane stride)

  // Software-pipelined steps. In step t a wave works on tile u = t - 1 - role
  // (role 1 trails role 0 by one tile, whose P it reads from LDS): it turns
  // the score block of tile u, computed in the previous step, into the B
  // fragments of its accumulation (role 0: P, also left in Pb[u & 1] as fp16;
  // role 1: dS = P (dP - D)), then runs one interleaved set of products:
  // tile u's accumulation and tile u + 1's score block. The products never
  // wait on each other's results within a step, and the vector work of one
  // wave overlaps the products of the other wave on its SIMD.
  //
  // Step t reads tiles t - 2 .. t (the stage ring holds NS). It issues tile
  // t + NS - 3 into the stage of tile t - 3, last read in step t - 1, and
  // ends once tile t + 1 has landed, leaving NS - 4 tiles in flight. Before
  // the first tile and after the last the wave's tile indices are clamped into
  // the range (those stages hold landed, finite data) and its accumulation
  // factors are zero, so the edge steps run the same products to no effect.
  static_assert(NS >= 5, "the step reads three resident tiles and keeps at least one in flight");
#pragma unroll
  for (int j = 0; j < NS - 3; ++j) issue(j);
  loads_landed_but<(NS - 4) * PER_ISSUE>();
  __syncthreads();
  // The step's products: product 2h is accumulation h (A^T from transposing
  // reads of the tile at abase: 16 keys c = h / DT, dims 32 (h % DT) ..; B =
  // mf[c]), product 2h + 1 is score step h (A from the tile at pbase, B = the
  // lane's key row) into sres; with KS < KK the run ends with the last
  // accumulation step alone. Fragment reads run kRingDkdv products ahead.
  constexpr int NP = KK + KS;
  constexpr int RING = kRingDkdv<D> < NP ? kRingDkdv<D> : NP;
  // product i: a score step or not, and its step h
  auto is_score = [](int i) { return i < 2 * KS && (i & 1); };
  auto step_of = [](int i) { return i < 2 * KS ? i >> 1 : KS + (i - 2 * KS); };
  f32x16 sres;  // score block of the wave's next tile
  auto run = [&](const T* abase, const Frag (&mf)[2], const T* pbase) {
    auto fetch = [&](int i) -> Frag {
      const int h = step_of(i);
      if (is_score(i)) return *reinterpret_cast<const Frag*>(pbase + a_lane[h]);
      const int c = h / DT, dt = h % DT;
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(abase + t_lane[0][dt] + 16 * c * L::ST));
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(abase + t_lane[1][dt] + 16 * c * L::ST));
      return __builtin_bit_cast(Frag, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    };
    Frag ring[RING];
#pragma unroll
    for (int i = 0; i < RING; ++i) ring[i] = fetch(i);
#pragma unroll
    for (int r = 0; r < 16; ++r) sres[r] = 0.f;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const Frag f = ring[i % RING];
      if (i + RING < NP) ring[i % RING] = fetch(i + RING);
      const int h = step_of(i);
      if (is_score(i))
        sres = Mma<T>::run(f, bf[h], sres);
      else
        acc[h % DT] = Mma<T>::run(f, mf[h / DT], acc[h % DT]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Step t of a wave is its local step tau = t - role (role 1 trails by one
  // tile), working on tile u = tau - 1. For tau >= 1 it reads stages
  // (tau - 1) % NS and tau % NS, so the steps are unrolled over the NS stage
  // phases of tau and every fragment address is a lane register plus an
  // immediate. Past the last tile those stages hold landed copies of it (the
  // cursor issues the last tile again), the same data the clamped indices
  // name. The first steps (tau <= 0, before tile 0 is scored) read stage 0.
  auto body = [&](int t, auto a_stage, auto s_stage) {
    constexpr int SA = decltype(a_stage)::value, SS = decltype(s_stage)::value;
    issue((t + NS - 3) % NS);
    const int u = t - 1 - role;
    const bool live = u >= 0 && u < n_it;
    Frag mf[2];
    if (live) {
      const int st = SA;  // u % NS
      float rv[16];  // the tile rows' lse2 (role 0) or D (role 1)
      rows16(RV[st][role], rv);
      if (role == 0) {
        // P = exp2(s c - lse2); keys a row must not see, and rows or keys past
        // the end, get 0. The test for a mask is wave-uniform (the slice's
        // keys, not the lane's), so the unmasked steps branch past it.
        const int q0 = (u0 + u % n_u) * BQ;
        const bool need_mask = (CAUSAL && q0 < kw0 + 32) || kw0 + 32 > S || q0 + BQ > S;
        float p[16];
        if (need_mask) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int qrow = q0 + 8 * (r >> 2) + 4 * g + (r & 3);
            const bool ok = key_ok & (qrow < S) & (!CAUSAL | (key <= qrow));
            const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sres[r], cs, -rv[r]));
            p[r] = ok ? e : 0.f;
          }
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sres[r], cs, -rv[r]));
        }
        _Float16* pw = Pb[SA & 1][slice];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          h8 hv;
#pragma unroll
          for (int i = 0; i < 8; ++i) hv[i] = (_Float16)p[8 * j + i];
          *reinterpret_cast<h8*>(pw + 512 * j + 8 * lane) = hv;
        }
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int j = 0; j < 8; ++j) mf[c][j] = (T)p[8 * c + j];
      } else {
        // dS = P (dP - D), with the P role 0 left for this tile one step ago
        const _Float16* pr = Pb[SA & 1][slice];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const h8 x = *reinterpret_cast<const h8*>(pr + 512 * j + 8 * lane);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int r = 8 * j + i;
            mf[j][i] = (T)((float)x[i] * (sres[r] - rv[r]));
          }
        }
      }
    } else {
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) mf[c][j] = (T)0.f;
    }
    // role 0: dV^T += dO^T P and S = Q K^T of the next tile;
    // role 1: dK^T += Q^T dS and dP = dO V^T of the next tile
    run(QG[SA], mf, QG[SS]);
    loads_landed_but<(NS - 4) * PER_ISSUE>();
    __syncthreads();
  };
  using std::integral_constant;
  int t = 0;
  for (; t <= role; ++t) body(t, integral_constant<int, 0>{}, integral_constant<int, 0>{});  // tau <= 0
  static_assert(NS == 6, "the step loop is unrolled over six stage phases");
  for (;;) {  // tau = t - role >= 1, phase tau % NS = 1, 2, ..., 5, 0
    if (t > n_it + 1) break;
    body(t++, integral_constant<int, 0>{}, integral_constant<int, 1>{});
    if (t > n_it + 1) break;
    body(t++, integral_constant<int, 1>{}, integral_constant<int, 2>{});
    if (t > n_it + 1) break;
    body(t++, integral_constant<int, 2>{}, integral_constant<int, 3>{});
    if (t > n_it + 1) break;
    body(t++, integral_constant<int, 3>{}, integral_constant<int, 4>{});
    if (t > n_it + 1) break;
    body(t++, integral_constant<int, 4>{}, integral_constant<int, 5>{});
    if (t > n_it + 1) break;
    body(t++, integral_constant<int, 5>{}, integral_constant<int, 0>{});
  }
  loads_landed_but<0>();  // tiles issued past the end, before the block's LDS is released

  if (key_ok) {
    const float f = role == 0 ? 1.0f : a.scale;  // dK: signed scale, Q was staged unflipped
    if (a.nsplit > 1) {
      // fp32 partial of this block's heads; dkdv_sum_kernel adds the splits
      const int64_t row = (a.cu != nullptr ? (int64_t)start : (int64_t)b * a.S) + key;
      float* out = a.part + (((int64_t)(split * 2 + role) * a.rows + row) * a.Hkv + hkv) * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq)
          if (dt * 32 + 8 * rq + 4 * g < a.dr)
            *reinterpret_cast<float4*>(out + dt * 32 + 8 * rq + 4 * g) =
              make_float4(acc[dt][4 * rq] * f, acc[dt][4 * rq + 1] * f, acc[dt][4 * rq + 2] * f, acc[dt][4 * rq + 3] * f);
    } else {
      T* out = role == 0
                   ? static_cast<T*>(a.dv) + b * a.dvs[0] + hkv * a.dvs[2] + (int64_t)(start + key) * a.dvs[1]
                   : static_cast<T*>(a.dk) + b * a.dks[0] + hkv * a.dks[2] + (int64_t)(start + key) * a.dks[1];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq)
          if (dt * 32 + 8 * rq + 4 * g < a.dr)
            *reinterpret_cast<uint2*>(out + dt * 32 + 8 * rq + 4 * g) =
                pack4<T>(acc[dt][4 * rq] * f, acc[dt][4 * rq + 1] * f, acc[dt][4 * rq + 2] * f, acc[dt][4 * rq + 3] * f);
    }
  }
}

// dV (role 0) and dK (role 1) of one token row, kv head and 4 dims: the sum of
// the nsplit partials in split order, rounded once. Rows are batch * S tokens
// (dense) or the packed token index.
template <typename T, int D>
__global__ __launch_bounds__(256) void dkdv_sum_kernel(BwdArgs a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // over rows * Hkv * head_dim / 4
  const int q4 = a.dr / 4;
  const int64_t n = a.rows * a.Hkv * q4;
  if (i >= n) return;
  const int d4 = (int)(i % q4) * 4;
  const int hkv = (int)((i / q4) % a.Hkv);
  const int64_t row = i / ((int64_t)q4 * a.Hkv);
  const int64_t b = a.cu != nullptr ? 0 : row / a.S;
  const int64_t t = a.cu != nullptr ? row : row % a.S;
  const int64_t stride = a.rows * a.Hkv * D;  // one (split, role) slab
#pragma unroll
  for (int role = 0; role < 2; ++role) {
    const float* p = a.part + (int64_t)role * stride + (row * a.Hkv + hkv) * D + d4;
    float4 s = *reinterpret_cast<const float4*>(p);
    for (int sp = 1; sp < a.nsplit; ++sp) {
      const float4 x = *reinterpret_cast<const float4*>(p + (int64_t)sp * 2 * stride);
      s.x += x.x;
      s.y += x.y;
      s.z += x.z;
      s.w += x.w;
    }
    T* out = role == 0 ? static_cast<T*>(a.dv) + b * a.dvs[0] + t * a.dvs[1] + hkv * a.dvs[2]
                       : static_cast<T*>(a.dk) + b * a.dks[0] + t * a.dks[1] + hkv * a.dks[2];
    if constexpr (std::is_same<T, float>::value)
      *reinterpret_cast<float4*>(out + d4) = s;
    else
      *reinterpret_cast<uint2*>(out + d4) = pack4<T>(s.x, s.y, s.z, s.w);
  }
}

#include "attn_bwd_f32.h"
#include "attn_bwd_wide.h"

template <typename T, int D, int KS>
int launch_ks(const BwdArgs& a, bool causal, hipStream_t s) {
  const int gp = a.group % 4 == 0 ? 4 : (a.group % 2 == 0 ? 2 : 1);
  const int64_t dq_blocks = (int64_t)((a.S + 32 * (4 / gp) - 1) / (32 * (4 / gp))) * a.B * a.Hq / gp;
  const int64_t kv_blocks = (int64_t)((a.S + BK - 1) / BK) * a.B * a.Hkv * a.nsplit;
  if (causal) {
    hipLaunchKernelGGL((attn_bwd_dq_kernel<T, D, true, KS>), dim3(dq_blocks), dim3(NT), 0, s, a);
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<T, D, true, KS>), dim3(kv_blocks), dim3(NT2), 0, s, a);
  } else {
    hipLaunchKernelGGL((attn_bwd_dq_kernel<T, D, false, KS>), dim3(dq_blocks), dim3(NT), 0, s, a);
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<T, D, false, KS>), dim3(kv_blocks), dim3(NT2), 0, s, a);
  }
  if (a.nsplit > 1) {
    const int64_t n = a.rows * a.Hkv * (a.dr / 4);
    hipLaunchKernelGGL((dkdv_sum_kernel<T, D>), dim3((n + 255) / 256), dim3(256), 0, s, a);
  }
  return launched("pk_attn_bwd");
}

// head_dim 40-48 and 72-80 (Popcorn's 48 and 80) leave the last 16 dims of the
// 64- and 96-dim rows empty: their S and dP steps are skipped. (At 8-16 on the
// 32-dim rows the shorter runs measured slower: 2.53 against 2.44 ms at C5's
// shape, head_dim 16.)
template <typename T, int D>
int launch(const BwdArgs& a, bool causal, hipStream_t s) {
  if constexpr (D == 64 || D == 96)
    if ((a.dr + 15) / 16 < D / 16) return launch_ks<T, D, D / 16 - 1>(a, causal, s);
  return launch_ks<T, D, D / 16>(a, causal, s);
}

// Number of q-head splits of the dk/dv kernel: the smallest divisor of the
// group size that gives at least two blocks per CU, else the group size (one
// q head per block). 1 keeps the direct path with no partials.
int dkdv_splits(int64_t seqs, int64_t seq, int64_t kv_heads, int64_t group) {
  const int64_t blocks = (seq + BK - 1) / BK * seqs * kv_heads;
  const int64_t want = 2 * (int64_t)cu_count();
  for (int64_t d = 1; d <= group; ++d)
    if (group % d == 0 && (blocks * d >= want || d == group)) return (int)d;
  return 1;
}

constexpr int64_t kAlign = 256;
inline int64_t round_up(int64_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

// Workspace bytes: D and lse2 (2 * lse_n floats), then the dk/dv partials when
// the kernel splits the q heads.
// (The partials are laid out at the kernels' row width: 64, 96, 128 or 256 dims; fp32, whose
// kernels have no 96-dim layout, is counted at 128, which covers either.)
int64_t workspace_bytes(int64_t lse_n, int64_t rows, int64_t kv_heads, int64_t head_dim, int nsplit) {
  const int64_t width = head_dim <= 64 ? 64 : (head_dim <= 128 ? 128 : 256);
  const int64_t parts = nsplit > 1 ? (int64_t)nsplit * 2 * rows * kv_heads * width * (int64_t)sizeof(float) : 0;
  return round_up(2 * lse_n * (int64_t)sizeof(float)) + parts;
}

// strides[24] = q, k, v, o, dout, dq, dk, dv (batch, token, head)
int bwd_launch(const char* who, BwdArgs a, void* workspace, int64_t workspace_bytes_given, const int64_t* strides,
               int64_t batch, int64_t seq, int64_t q_heads, int64_t kv_heads, int64_t head_dim, float softmax_scale,
               int causal, int dtype, void* stream) {
  if (batch < 0 || seq < 0 || q_heads < 0 || kv_heads < 0 || head_dim < 0)
    return fail(PK_ERR_INVALID, "%s: negative size", who);
  if (batch == 0 || seq == 0 || q_heads == 0) return PK_OK;
  if (!a.q || !a.k || !a.v || !a.o || !a.dout || !a.lse || !workspace || !a.dq || !a.dk || !a.dv || !strides)
    return fail(PK_ERR_INVALID, "%s: null pointer", who);
  if (kv_heads == 0 || q_heads % kv_heads != 0)
    return fail(PK_ERR_INVALID, "%s: q_heads=%lld is not a multiple of kv_heads=%lld", who, (long long)q_heads,
                (long long)kv_heads);
  a.nsplit = dkdv_splits(batch, seq, kv_heads, q_heads / kv_heads);
  const int64_t need = workspace_bytes(a.lse_n, a.rows, kv_heads, head_dim, a.nsplit);
  if (workspace_bytes_given < need)
    return fail(PK_ERR_INVALID, "%s: workspace of %lld bytes, %lld needed", who, (long long)workspace_bytes_given,
                (long long)need);
  if (!aligned16(workspace)) return fail(PK_ERR_INVALID, "%s: workspace must be 16-byte aligned", who);
  a.dsum = static_cast<float*>(workspace);
  a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + round_up(2 * a.lse_n * (int64_t)sizeof(float)));
  if (dtype != PK_BF16 && dtype != PK_F16 && dtype != PK_F32)
    return fail(PK_ERR_UNSUPPORTED, "%s: dtype code %d (bf16/fp16/fp32 only)", who, dtype);
  const int64_t max_dim = 256;
  if (head_dim <= 0 || head_dim > max_dim || head_dim % 8 != 0)
    return fail(PK_ERR_UNSUPPORTED, "%s: head_dim=%lld (a multiple of 8 up to %lld)", who, (long long)head_dim,
                (long long)max_dim);
  if (!isfinite(softmax_scale)) return fail(PK_ERR_INVALID, "%s: softmax_scale is not finite", who);
  if (seq > (1 << 30) || batch * q_heads > (1 << 20)) return fail(PK_ERR_UNSUPPORTED, "%s: shape too large", who);
  const void* ptrs[] = {a.q, a.k, a.v, a.o, a.dout, a.dq, a.dk, a.dv};
  for (const void* p : ptrs)
    if (!aligned16(p)) return fail(PK_ERR_INVALID, "%s: tensors must be 16-byte aligned", who);
  const int64_t elem = dtype == PK_F32 ? 4 : 2;
  const int64_t unit = 16 / elem;  // strides in whole 16-byte chunks
  for (int i = 0; i < 24; ++i)
    if (strides[i] % unit != 0 || strides[i] < 0)
      return fail(PK_ERR_INVALID, "%s: stride %d = %lld is not a non-negative multiple of %lld", who, i,
                  (long long)strides[i], (long long)unit);
  int64_t* dst[] = {a.qs, a.ks, a.vs, a.os, a.gs, a.dqs, a.dks, a.dvs};
  for (int t = 0; t < 8; ++t)
    for (int i = 0; i < 3; ++i) dst[t][i] = strides[3 * t + i];
  // buffer offsets are 32-bit: rows of one sequence (plus a tile past the end) must fit
  int64_t widest = 0;
  for (int t = 0; t < 5; ++t) widest = dst[t][1] > widest ? dst[t][1] : widest;
  if ((seq + 2 * BK) * widest * elem + head_dim * elem > INT32_MAX)
    return fail(PK_ERR_UNSUPPORTED, "%s: rows span more than 2 GiB per head", who);
  a.B = (int)batch;
  a.S = (int)seq;
  a.Hq = (int)q_heads;
  a.Hkv = (int)kv_heads;
  a.group = (int)(q_heads / kv_heads);
  a.scale = softmax_scale;
  a.c = fmaxf(fabsf(softmax_scale) * 1.4426950408889634f, 1e-30f);
  a.q_flip = softmax_scale < 0.f ? 0x80008000u : 0u;
  a.dr = (int)head_dim;
  a.dch = (int)(head_dim / 8);
  if ((seq + BM - 1) / BM * batch * q_heads > INT32_MAX) return fail(PK_ERR_UNSUPPORTED, "%s: grid too large", who);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // rows are laid out at 32, 96 and 192 (16-bit types), 64, 128 or 256 dims, the chunks past head_dim reading
  // as zeros
  if (dtype == PK_F32)
    return head_dim <= 64 ? launch_f32<64>(a, causal, s)
                          : (head_dim <= 128 ? launch_f32<128>(a, causal, s) : launch_f32<256>(a, causal, s));
  if (head_dim > 192)
    return dtype == PK_BF16 ? launch_wide<bf16, 256>(a, causal, s) : launch_wide<f16, 256>(a, causal, s);
  if (head_dim > 128)
    return dtype == PK_BF16 ? launch_wide<bf16, 192>(a, causal, s) : launch_wide<f16, 192>(a, causal, s);
  if (dtype == PK_BF16)
    return head_dim <= 32   ? launch<bf16, 32>(a, causal, s)
           : head_dim <= 64 ? launch<bf16, 64>(a, causal, s)
           : head_dim <= 96 ? launch<bf16, 96>(a, causal, s)
                            : launch<bf16, 128>(a, causal, s);
  return head_dim <= 32   ? launch<f16, 32>(a, causal, s)
         : head_dim <= 64 ? launch<f16, 64>(a, causal, s)
         : head_dim <= 96 ? launch<f16, 96>(a, causal, s)
                          : launch<f16, 128>(a, causal, s);
}

}  // namespace
}  // namespace pk

extern "C" {

int64_t pk_attn_bwd_workspace(int64_t batch, int64_t seq, int64_t q_heads, int64_t kv_heads, int64_t head_dim) {
  using namespace pk;
  if (batch < 0 || seq < 0 || q_heads < 0 || kv_heads <= 0 || head_dim < 0 || q_heads % kv_heads != 0) return -1;
  const int nsplit = dkdv_splits(batch, seq, kv_heads, q_heads / kv_heads);
  return workspace_bytes(batch * q_heads * seq, batch * seq, kv_heads, head_dim, nsplit);
}

int64_t pk_attn_varlen_bwd_workspace(int64_t num_seqs, int64_t total, int64_t max_seqlen, int64_t q_heads,
                                     int64_t kv_heads, int64_t head_dim) {
  using namespace pk;
  if (num_seqs < 0 || total < 0 || max_seqlen < 0 || q_heads < 0 || kv_heads <= 0 || head_dim < 0 ||
      q_heads % kv_heads != 0)
    return -1;
  const int nsplit = dkdv_splits(num_seqs, max_seqlen, kv_heads, q_heads / kv_heads);
  return workspace_bytes(q_heads * total, total, kv_heads, head_dim, nsplit);
}

int pk_attn_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout, const float* lse,
                void* workspace, int64_t workspace_bytes, void* dq, void* dk, void* dv, const int64_t* strides,
                int64_t batch, int64_t seq, int64_t q_heads, int64_t kv_heads, int64_t head_dim, float softmax_scale,
                int causal, int dtype, void* stream) {
  using namespace pk;
  BwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.dout = dout;
  a.lse = lse;
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  a.cu = nullptr;
  a.lse_bs = q_heads * seq;  // [batch, q_heads, seq]
  a.lse_hs = seq;
  a.lse_n = batch * q_heads * seq;
  a.rows = batch * seq;
  return bwd_launch("pk_attn_bwd", a, workspace, workspace_bytes, strides, batch, seq, q_heads, kv_heads, head_dim,
                    softmax_scale, causal, dtype, stream);
}

int pk_attn_varlen_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout, const float* lse,
                       void* workspace, int64_t workspace_bytes, void* dq, void* dk, void* dv, const int* cu_seqlens,
                       const int64_t* strides, int64_t num_seqs, int64_t total, int64_t max_seqlen, int64_t q_heads,
                       int64_t kv_heads, int64_t head_dim, float softmax_scale, int causal, int dtype, void* stream) {
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
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  a.cu = cu_seqlens;
  a.total = (int)total;
  a.lse_bs = 0;  // [q_heads, total]
  a.lse_hs = total;
  a.lse_n = q_heads * total;
  a.rows = total;
  return bwd_launch(who, a, workspace, workspace_bytes, dense, num_seqs, max_seqlen, q_heads, kv_heads, head_dim,
                    softmax_scale, causal, dtype, stream);
}

}  // extern "C"
