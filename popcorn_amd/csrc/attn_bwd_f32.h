// Attention backward in fp32 on the fp32 matrix cores (v_mfma_f32_32x32x2_f32),
// for Popcorn's float32 attention grid (the 16-bit kernels cover bf16 and
// fp16). Included by attn_bwd.hip inside its namespace, after BwdArgs and
// dkdv_sum_kernel; the two-kernel split, work mapping, workspace (D, lse2 and
// the dk/dv partials) and sign conventions are the 16-bit backward's.
//
// The 32x32x2 product takes one fp32 per lane from each operand: lane (row
// i = lane % 32, half g = lane / 32) gives A[i][g] and B[g][i], and the
// result lane l holds column l % 32, rows 8 (r / 4) + 4 g + r % 4 (register
// r). The contraction order is free as long as both operands follow it, so
// every product below reads its operands in the layout the previous one left:
//
//   score blocks (S^T = K Q^T and dP^T = V dO^T in the dq kernel, S = Q K^T
//   and dP = dO V^T in the dk/dv kernel) contract dims H g + t at product t
//   (H = D / 2): the streamed operand is a 16-byte read of its row from LDS,
//   the stationary one a register;
//   accumulations (dQ += dS K, dV^T += dO^T P, dK^T += Q^T dS) contract, at
//   product t, the row that score register t of the lane holds, so the
//   score-side operand is register t itself. The result's 32 columns (dQ) or
//   rows (dV^T, dK^T) at block dt are dims 128 (dt / W) + W j + dt % W
//   (W = min(D / 32, 4)), so one W-wide read of a row (two at head_dim 256)
//   gives product t's operand for every block, and the blocks of an element
//   line up into W consecutive dims to store.
//
// Tiles of 32 rows x D dims sit in LDS as unpadded rows of 16-byte chunks,
// chunk c of row r at c ^ fswz(r) with fswz(r) = (r % 16) ^ 8 ((r / 4) % 2):
// the 16-byte reads (16 rows, one chunk) hit 16 distinct chunk positions, and
// the DT-wide reads (rows R and R + 4, one row per half-wave, 32 columns)
// put the two halves in opposite halves of the 64 banks. Tiles are filled by
// buffer loads that write LDS directly; rows past the end and dims past
// head_dim read as zero.

#pragma once

constexpr int kF32DqThreads = 256;    // dq kernel: 4 waves of 32 query rows
constexpr int kF32DkdvThreads = 512;  // dk/dv kernel: 4 key slices x 2 roles

__device__ __forceinline__ int fswz(int r) { return (r & 15) ^ (((r >> 2) & 1) << 3); }

// Float offset of (row, dim) in an fp32 tile of D-dim rows
template <int D> __device__ __forceinline__ int fat(int row, int dim) {
  return row * D + (((dim >> 2) ^ fswz(row)) << 2) + (dim & 3);
}

// Accumulation blocks over DO output dims (DO / 32 blocks): block dt's 32
// result columns (dQ) or rows (dV^T, dK^T) are dims 128 (dt / W) + W j + dt % W
// with W = min(DO / 32, 4). One W-wide read of a tile row at column W j (and
// one 128 dims on, for 256 output dims) gives product t's operand for every
// block, and an element's blocks store as W consecutive dims per 128.
template <int DO> struct Cols {
  static constexpr int DT = DO / 32;
  static constexpr int W = DT < 4 ? DT : 4;
  static constexpr int NS = DT / W;  // spans, 128 dims apart
};

// The operands of every block at one product: p is the tile element at column W j of a row (the tile's
// swizzle keeps a chunk's offset within its 128-dim half, so the second span sits 128 floats on)
template <int DO> struct Span {
  using C = Cols<DO>;
  float v[C::DT];
  __device__ __forceinline__ explicit Span(const float* p) {
#pragma unroll
    for (int sp = 0; sp < C::NS; ++sp) {
      if constexpr (C::W == 4) {
        const float4 x = *reinterpret_cast<const float4*>(p + 128 * sp);
        v[4 * sp] = x.x;
        v[4 * sp + 1] = x.y;
        v[4 * sp + 2] = x.z;
        v[4 * sp + 3] = x.w;
      } else {
        const float2 x = *reinterpret_cast<const float2*>(p);
        v[0] = x.x;
        v[1] = x.y;
      }
    }
  }
};

// Element r of every block's accumulator, times f, to the W consecutive dims at p (dim `dim` of the row)
// and, for 256 output dims, 128 dims on; spans from head_dim on are not stored
template <int DO>
__device__ __forceinline__ void store_span(float* p, const f32x16 (&acc)[DO / 32], int r, float f, int dim, int dr) {
  using C = Cols<DO>;
#pragma unroll
  for (int sp = 0; sp < C::NS; ++sp) {
    if (dim + 128 * sp >= dr) continue;
    const int b0 = C::W * sp;
    if constexpr (C::W == 4)
      *reinterpret_cast<float4*>(p + 128 * sp) =
          make_float4(acc[b0][r] * f, acc[b0 + 1][r] * f, acc[b0 + 2][r] * f, acc[b0 + 3][r] * f);
    else
      *reinterpret_cast<float2*>(p) = make_float2(acc[0][r] * f, acc[1][r] * f);
  }
}

// Lane offsets (bytes) of the direct loads that fill a 32-row tile: slot
// sl = i * threads + tid is row sl / CH, stored chunk sl % CH, which holds
// logical chunk (sl % CH) ^ fswz(row); chunks past head_dim get kPadOffset.
template <int D> __device__ __forceinline__ int tile_offset(int sl, int64_t row_stride, int dr) {
  constexpr int CH = D / 4;
  const int row = sl / CH, c = (sl % CH) ^ fswz(row);
  return 4 * c < dr ? (row * (int)row_stride + 4 * c) * (int)sizeof(float) : (int)kPadOffset;
}

// The tiles are staged with the inline-assembly direct loads (ld_lds16_asm):
// the compiler would otherwise wait for a step's prefetch into the other stage
// before the step's first fragment read. Each step still waits for all its
// loads before its closing barrier.
__device__ __forceinline__ rsrc_words rows_rsrc(const float* base, int rows, int64_t row_stride, int dr) {
  return make_rsrc_words(base, (int)(((int64_t)(rows - 1) * row_stride + dr) * (int)sizeof(float)));
}

// dq kernel: one block = 4 waves x 32 query rows over one (sequence, kv head),
// gp of its q heads x 4 / gp row groups, as the 16-bit dq kernel. Each wave
// holds its rows' Q and dO halves in registers and streams K and V tiles of 32
// keys through two LDS buffers. Per tile: S^T = K Q^T and dP^T = V dO^T,
// P = exp2(s c - lse2), dS = P (dP - D), dQ += dS K. The prologue computes
// D = rowsum(dO * O) and lse2 = lse log2(e) for the dk/dv kernel.
template <int D, bool CAUSAL>
__global__ __attribute__((amdgpu_flat_work_group_size(kF32DqThreads, kF32DqThreads), amdgpu_waves_per_eu(D == 64 ? 2 : 1)))
void attn_bwd_f32_dq_kernel(BwdArgs a) {
  constexpr int H = D / 2;
  constexpr int DT = D / 32;
  constexpr int CH = D / 4;
  constexpr int TILE = BN * D;                  // floats of a K (or V) tile
  constexpr int TI = BN * CH / kF32DqThreads;   // direct loads per thread per tile of K (and of V): 4 or 2
  __shared__ __attribute__((aligned(16))) float KV[2][2 * TILE];  // buffer: K tile, then V tile

  // work item: (q tile, batch, kv head, head quad), longest causal rows first
  const int G = a.group;
  const int GP = G % 4 == 0 ? 4 : (G % 2 == 0 ? 2 : 1);
  const int rows_per_block = 32 * (4 / GP);
  const int m_tiles = (a.S + rows_per_block - 1) / rows_per_block;
  const int n_quads = G / GP;
  const int per_tile = a.B * a.Hkv * n_quads;
  const int w = blockIdx.x;
  int m_tile, rest;
  if (per_tile % 8 == 0) {  // group-major per XCD
    const int k = w >> 3;
    m_tile = m_tiles - 1 - k % m_tiles;
    rest = (w & 7) + 8 * (k / m_tiles);
  } else {
    m_tile = m_tiles - 1 - w / per_tile;
    rest = w % per_tile;
  }
  const int b = rest / (a.Hkv * n_quads);
  const int hkv = (rest / n_quads) % a.Hkv;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hq = hkv * G + (rest % n_quads) * GP + wave % GP;
  int start, S;
  seq_bounds(a, b, start, S);
  const int m0 = m_tile * rows_per_block;
  if (m0 >= S) return;  // whole block, before any barrier

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int r32 = lane & 31;
  const int g = lane >> 5;
  const int wave_first = m0 + (wave / GP) * 32;
  const int q_row = wave_first + r32;
  const bool row_ok = q_row < S;

  const float* qbase = static_cast<const float*>(a.q) + b * a.qs[0] + hq * a.qs[2] + start * a.qs[1];
  const float* obase = static_cast<const float*>(a.o) + b * a.os[0] + hq * a.os[2] + start * a.os[1];
  const float* gbase = static_cast<const float*>(a.dout) + b * a.gs[0] + hq * a.gs[2] + start * a.gs[1];
  const float* kbase = static_cast<const float*>(a.k) + b * a.ks[0] + hkv * a.ks[2] + start * a.ks[1];
  const float* vbase = static_cast<const float*>(a.v) + b * a.vs[0] + hkv * a.vs[2] + start * a.vs[1];

  // Q (negated for a negative scale) and dO halves of the lane's row: dims H g .. H g + H - 1
  float qv[H], gv[H];
  float dsum = 0.f;
  const float sg = a.q_flip ? -1.f : 1.f;
#pragma unroll
  for (int u = 0; u < H / 4; ++u) {
    const int d = H * g + 4 * u;
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f), y = x, z = x;
    if (row_ok && d < a.dr) {
      x = *reinterpret_cast<const float4*>(qbase + (int64_t)q_row * a.qs[1] + d);
      y = *reinterpret_cast<const float4*>(gbase + (int64_t)q_row * a.gs[1] + d);
      z = *reinterpret_cast<const float4*>(obase + (int64_t)q_row * a.os[1] + d);
    }
    qv[4 * u] = x.x * sg;
    qv[4 * u + 1] = x.y * sg;
    qv[4 * u + 2] = x.z * sg;
    qv[4 * u + 3] = x.w * sg;
    gv[4 * u] = y.x;
    gv[4 * u + 1] = y.y;
    gv[4 * u + 2] = y.z;
    gv[4 * u + 3] = y.w;
    dsum += y.x * z.x + y.y * z.y + y.z * z.z + y.w * z.w;
  }
  dsum += __shfl_xor(dsum, 32, 64);
  const int64_t lidx = b * a.lse_bs + hq * a.lse_hs + start + q_row;
  // rows past the end: lse2 = +inf makes every p zero
  const float lse2 = row_ok ? a.lse[lidx] * 1.4426950408889634f : INFINITY;
  if (row_ok && g == 0) {
    a.dsum[lidx] = dsum;
    a.dsum[a.lse_n + lidx] = lse2;
  }

  const int kv_end = CAUSAL ? min(m0 + rows_per_block, S) : S;
  const int n_tiles = (kv_end + BN - 1) / BN;
  const rsrc_words krs = rows_rsrc(kbase, S, a.ks[1], a.dr);
  const rsrc_words vrs = rows_rsrc(vbase, S, a.vs[1], a.dr);
  int kgo[TI], vgo[TI];
#pragma unroll
  for (int i = 0; i < TI; ++i) {
    kgo[i] = tile_offset<D>(i * kF32DqThreads + tid, a.ks[1], a.dr);
    vgo[i] = tile_offset<D>(i * kF32DqThreads + tid, a.vs[1], a.dr);
  }
  auto issue = [&](int t, int buf) {
#pragma unroll
    for (int i = 0; i < TI; ++i) {
      const int at = (i * kF32DqThreads + wave * 64) * 4;
      ld_lds16_asm(krs, &KV[buf][at], kgo[i], t * BN * (int)a.ks[1] * (int)sizeof(float));
      ld_lds16_asm(vrs, &KV[buf][TILE + at], vgo[i], t * BN * (int)a.vs[1] * (int)sizeof(float));
    }
  };

  f32x16 dq[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[dt][r] = 0.f;
  const float c = a.c;

  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), seen by the compiler: its own loads are done
  issue(0, 0);
  lds_loads_landed();
  __syncthreads();
  for (int t = 0; t < n_tiles; ++t) {
    const int buf = t & 1;
    // the next tile into the other buffer, which every wave finished reading in the last step
    if (t + 1 < n_tiles) issue(t + 1, buf ^ 1);
    const float* Kt = KV[buf];
    const float* Vt = KV[buf] + TILE;

    // S^T = K Q^T and dP^T = V dO^T: register r holds key 8 (r / 4) + 4 g + r % 4 of the tile for the lane's row
    f32x16 s, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = 0.f;
      dp[r] = 0.f;
    }
#pragma unroll
    for (int u = 0; u < H / 4; ++u) {
      const float4 kf = *reinterpret_cast<const float4*>(Kt + fat<D>(r32, H * g + 4 * u));
      const float4 vf = *reinterpret_cast<const float4*>(Vt + fat<D>(r32, H * g + 4 * u));
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.x, qv[4 * u], s, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x2f32(vf.x, gv[4 * u], dp, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.y, qv[4 * u + 1], s, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x2f32(vf.y, gv[4 * u + 1], dp, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.z, qv[4 * u + 2], s, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x2f32(vf.z, gv[4 * u + 2], dp, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.w, qv[4 * u + 3], s, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x2f32(vf.w, gv[4 * u + 3], dp, 0, 0, 0);
      // at 256 dims Q and dO fill the VGPRs: keep the scheduler from hoisting every read ahead
      if constexpr (D == 256) __builtin_amdgcn_sched_barrier(0);
    }

    // dS = P (dP - D) over the keys the row may see
    const int lim = CAUSAL ? min(q_row, S - 1) : S - 1;
    float ds[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = t * BN + 8 * (r >> 2) + 4 * g + (r & 3);
      const float p = exp2f(fmaf(s[r], c, -lse2));
      ds[r] = key > lim ? 0.f : p * (dp[r] - dsum);
    }

    // dQ += dS K: product u takes the key of register u; block dt's column j is dim 128 (dt / W) + W j + dt % W
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const Span<D> kd(Kt + fat<D>(8 * (u >> 2) + 4 * g + (u & 3), Cols<D>::W * r32));
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) dq[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(ds[u], kd.v[dt], dq[dt], 0, 0, 0);
      if constexpr (D == 256) __builtin_amdgcn_sched_barrier(0);
    }

    lds_loads_landed();  // this wave's part of the next tile
    __syncthreads();
  }

  // dQ = scale dS K: register r of block dt is row 8 (r / 4) + 4 g + r % 4 of the wave, dim DT r32 + dt
  {
    const int col = Cols<D>::W * r32;
    float* dqb = static_cast<float*>(a.dq) + b * a.dqs[0] + hq * a.dqs[2] + start * a.dqs[1] + col;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = wave_first + 8 * (r >> 2) + 4 * g + (r & 3);
      if (row < S) store_span<D>(dqb + (int64_t)row * a.dqs[1], dq, r, a.scale, col, a.dr);
    }
  }
}

// dk/dv kernel: one block = 128 keys of one (sequence, kv head) in four 32-key
// slices, two waves per slice (waves s and s + 4 share a SIMD). Role 0 holds
// the slice's K half rows, computes S = Q K^T, P = exp2(s c - lse2), leaves P
// in LDS and accumulates dV^T += dO^T P; role 1 holds V, computes dP = dO V^T
// one step later, reads that P, forms dS = P (dP - D) and accumulates
// dK^T += Q^T dS. Query tiles of 32 rows (Q then dO, with their lse2 and D
// rows), over the q heads of the group the block covers, arrive through three
// LDS stages: the two a step reads and the one landing.
template <int D, bool CAUSAL>
__global__ __attribute__((amdgpu_flat_work_group_size(kF32DkdvThreads, kF32DkdvThreads), amdgpu_waves_per_eu(2)))
void attn_bwd_f32_dkdv_kernel(BwdArgs a) {
  constexpr int H = D / 2;
  constexpr int DT = D / 32;
  constexpr int CH = D / 4;
  constexpr int TILE = BQ * D;                     // floats of a Q (or dO) tile
  constexpr int SLOTS = BQ * CH;                   // 16-byte slots of a tile
  constexpr int TI = 2 * SLOTS / kF32DkdvThreads;  // direct loads per thread per stage: 4 or 2 (Q, then dO)
  static_assert(TI % 2 == 0, "a thread's loads split evenly between the Q and dO tiles");
  __shared__ __attribute__((aligned(16))) float QG[3][2 * TILE];  // stage: Q tile, then dO tile
  __shared__ __attribute__((aligned(16))) float RV[3][2][64];     // stage: lse2 rows, D rows (32 used)
  __shared__ __attribute__((aligned(16))) float4 Pb[2][4][4 * 64];  // P per slice: [buffer][slice][r / 4][lane]

  const int w = blockIdx.x;
  const int per_tile = a.B * a.Hkv * a.nsplit;
  const int kv_tile = w / per_tile;  // first key tiles (the most causal work) first
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
  const int role = wave >> 2;
  const int slice = wave & 3;
  const int lane = tid & 63;
  const int r32 = lane & 31;
  const int g = lane >> 5;
  const int key = kb0 + slice * 32 + r32;
  const bool key_ok = key < S;

  // the lane's key half row (dims H g + t): K (role 0) or V (role 1)
  float kv[H];
  {
    const float* row = role == 0
                           ? static_cast<const float*>(a.k) + b * a.ks[0] + hkv * a.ks[2] + (int64_t)(start + key) * a.ks[1]
                           : static_cast<const float*>(a.v) + b * a.vs[0] + hkv * a.vs[2] + (int64_t)(start + key) * a.vs[1];
#pragma unroll
    for (int u = 0; u < H / 4; ++u) {
      const int d = H * g + 4 * u;
      float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
      if (key_ok && d < a.dr) x = *reinterpret_cast<const float4*>(row + d);
      kv[4 * u] = x.x;
      kv[4 * u + 1] = x.y;
      kv[4 * u + 2] = x.z;
      kv[4 * u + 3] = x.w;
    }
  }
  // Q is staged unflipped: a negative scale signs the exponent's coefficient here and dK's final scale
  const float cs = a.q_flip ? -a.c : a.c;

  // query tiles: every q head of the block's share of the group, rows from the block's first key on (causal)
  const int u0 = CAUSAL ? kb0 / BQ : 0;
  const int n_u = (S + BQ - 1) / BQ - u0;
  const int n_it = heads * n_u;

  int go[TI];
#pragma unroll
  for (int i = 0; i < TI; ++i)
    go[i] = tile_offset<D>((i * kF32DkdvThreads + tid) % SLOTS, i < TI / 2 ? a.qs[1] : a.gs[1], a.dr);
  // tile it (q head it / n_u of the block's, q tile u0 + it % n_u) into stage st; waves 0 and 1 also load
  // its rows' lse2 and D (rows past the end read as zero)
  auto issue = [&](int it, int st) {
    const int hq = hkv * a.group + split * heads + it / n_u;
    const int r0 = (u0 + it % n_u) * BQ;
    const float* qb = static_cast<const float*>(a.q) + b * a.qs[0] + hq * a.qs[2] + start * a.qs[1];
    const float* gb = static_cast<const float*>(a.dout) + b * a.gs[0] + hq * a.gs[2] + start * a.gs[1];
    const rsrc_words qrs = rows_rsrc(qb, S, a.qs[1], a.dr);
    const rsrc_words grs = rows_rsrc(gb, S, a.gs[1], a.dr);
#pragma unroll
    for (int i = 0; i < TI; ++i)
      ld_lds16_asm(i < TI / 2 ? qrs : grs, &QG[st][(i * kF32DkdvThreads + wave * 64) * 4], go[i],
                 r0 * (int)(i < TI / 2 ? a.qs[1] : a.gs[1]) * (int)sizeof(float));
    if (wave < 2) {
      const float* rb = a.dsum + b * a.lse_bs + hq * a.lse_hs + start + (wave == 0 ? a.lse_n : 0);
      const rsrc_words rrs = make_rsrc_words(rb, S * (int)sizeof(float));
      ld_lds4_asm(rrs, RV[st][wave], lane * (int)sizeof(float), r0 * (int)sizeof(float));
    }
  };

  f32x16 acc[DT];  // dV^T (role 0) or dK^T (role 1): block dt's row i is dim DT i + dt, the column the lane's key
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[dt][r] = 0.f;

  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), seen by the compiler: its own loads are done
  issue(0, 0);
  lds_loads_landed();
  __syncthreads();
  // step t: role 0 works on tile t, role 1 on tile t - 1 (whose P role 0 left in Pb[(t - 1) & 1])
  for (int t = 0; t <= n_it; ++t) {
    if (t + 1 < n_it) issue(t + 1, (t + 1) % 3);
    const int it = role == 0 ? t : t - 1;
    if (it >= 0 && it < n_it) {
      const int st = it % 3;
      const int r0 = (u0 + it % n_u) * BQ;
      const float* Qt = QG[st];
      const float* Gt = QG[st] + TILE;
      // score block: S = Q K^T (role 0) or dP = dO V^T (role 1); register r holds query row
      // r0 + 8 (r / 4) + 4 g + r % 4 of the lane's key
      const float* At = role == 0 ? Qt : Gt;
      f32x16 s;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
      for (int u = 0; u < H / 4; ++u) {
        const float4 af = *reinterpret_cast<const float4*>(At + fat<D>(r32, H * g + 4 * u));
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(af.x, kv[4 * u], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(af.y, kv[4 * u + 1], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(af.z, kv[4 * u + 2], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(af.w, kv[4 * u + 3], s, 0, 0, 0);
      }
      // the lane's 16 values of the tile's lse2 (role 0) or D (role 1) rows
      float rv[16];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 x = *reinterpret_cast<const float4*>(&RV[st][role][8 * j + 4 * g]);
        rv[4 * j] = x.x;
        rv[4 * j + 1] = x.y;
        rv[4 * j + 2] = x.z;
        rv[4 * j + 3] = x.w;
      }
      float f[16];  // P (role 0) or dS (role 1)
      float4* pb = &Pb[it & 1][slice][lane];
      if (role == 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qr = r0 + 8 * (r >> 2) + 4 * g + (r & 3);
          const bool masked = qr >= S || (CAUSAL && qr < key);
          f[r] = masked ? 0.f : exp2f(fmaf(s[r], cs, -rv[r]));
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) pb[64 * j] = make_float4(f[4 * j], f[4 * j + 1], f[4 * j + 2], f[4 * j + 3]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float4 p = pb[64 * j];
          const float pj[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = 4 * j + i;
            const int qr = r0 + 8 * j + 4 * g + i;
            const bool masked = qr >= S || (CAUSAL && qr < key);
            f[r] = masked ? 0.f : pj[i] * (s[r] - rv[r]);
          }
        }
      }
      // dV^T += dO^T P (role 0) or dK^T += Q^T dS (role 1): product u takes the query row of register u
      const float* Ct = role == 0 ? Gt : Qt;
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const Span<D> cd(Ct + fat<D>(8 * (u >> 2) + 4 * g + (u & 3), Cols<D>::W * r32));
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(cd.v[dt], f[u], acc[dt], 0, 0, 0);
      }
    }
    lds_loads_landed();  // this wave's part of the next tile
    __syncthreads();
  }

  if (key_ok) {
    const float fs = role == 0 ? 1.0f : a.scale;  // dK: signed scale, Q was staged unflipped
    float* out;
    if (a.nsplit > 1) {  // fp32 partial of this block's heads; dkdv_sum_kernel adds the splits
      const int64_t row = (a.cu != nullptr ? (int64_t)start : (int64_t)b * a.S) + key;
      out = a.part + (((int64_t)(split * 2 + role) * a.rows + row) * a.Hkv + hkv) * D;
    } else {
      out = role == 0 ? static_cast<float*>(a.dv) + b * a.dvs[0] + hkv * a.dvs[2] + (int64_t)(start + key) * a.dvs[1]
                      : static_cast<float*>(a.dk) + b * a.dks[0] + hkv * a.dks[2] + (int64_t)(start + key) * a.dks[1];
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = 8 * (r >> 2) + 4 * g + (r & 3);
      store_span<D>(out + Cols<D>::W * i, acc, r, fs, Cols<D>::W * i, a.dr);
    }
  }
}

// dk/dv kernel at head_dim 256 (and 136-248, laid out at 256). A 32-key slice's
// K and V half rows alone take 256 registers here and its dK and dV another
// 256, so one wave per slice does both roles (as the 16-bit kernel at this
// width) for half of the output dims: block pair (2 w, 2 w + 1) covers the
// same keys, dims 0-127 and 128-255 of dK and dV, each computing S and dP over
// all 256 dims (the scores cost twice; the accumulations are split). Per query
// tile: S = Q K^T and dP = dO V^T interleaved, P and dS in registers, then
// dV^T += dO^T P and dK^T += Q^T dS over the block's 128 dims. Q/dO tiles are
// double-buffered.
template <bool CAUSAL>
__global__ __attribute__((amdgpu_flat_work_group_size(kF32DqThreads, kF32DqThreads), amdgpu_waves_per_eu(1)))
void attn_bwd_f32_dkdv_wide_kernel(BwdArgs a) {
  constexpr int D = 256;
  constexpr int DO = 128;  // output dims per block
  constexpr int H = D / 2;
  constexpr int DT = DO / 32;
  constexpr int CH = D / 4;
  constexpr int TILE = BQ * D;
  constexpr int SLOTS = BQ * CH;
  constexpr int TI = 2 * SLOTS / kF32DqThreads;  // direct loads per thread per stage: 16 (Q, then dO)
  static_assert(TI % 2 == 0 && (TI / 2) * kF32DqThreads == SLOTS, "a thread's loads split evenly over Q and dO");
  __shared__ __attribute__((aligned(16))) float QG[2][2 * TILE];  // buffer: Q tile, then dO tile
  __shared__ __attribute__((aligned(16))) float RV[2][2][64];     // buffer: lse2 rows, D rows (32 used)

  const int half = blockIdx.x & 1;  // output dims 128 half .. 128 half + 127
  const int w = blockIdx.x >> 1;
  const int per_tile = a.B * a.Hkv * a.nsplit;
  const int kv_tile = w / per_tile;  // first key tiles (the most causal work) first
  const int gi = w % per_tile;
  const int b = gi / (a.Hkv * a.nsplit);
  const int hkv = (gi / a.nsplit) % a.Hkv;
  const int split = gi % a.nsplit;
  const int heads = a.group / a.nsplit;
  int start, S;
  seq_bounds(a, b, start, S);
  const int kb0 = kv_tile * BK;
  if (kb0 >= S || 128 * half >= a.dr) return;  // whole block, before any barrier

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r32 = lane & 31;
  const int g = lane >> 5;
  const int kw0 = kb0 + wave * 32;
  const int key = kw0 + r32;
  const bool key_ok = key < S;

  // the lane's K and V half rows (dims H g + t)
  float kv[H], vv[H];
  {
    const float* krow = static_cast<const float*>(a.k) + b * a.ks[0] + hkv * a.ks[2] + (int64_t)(start + key) * a.ks[1];
    const float* vrow = static_cast<const float*>(a.v) + b * a.vs[0] + hkv * a.vs[2] + (int64_t)(start + key) * a.vs[1];
#pragma unroll
    for (int u = 0; u < H / 4; ++u) {
      const int d = H * g + 4 * u;
      float4 x = make_float4(0.f, 0.f, 0.f, 0.f), y = x;
      if (key_ok && d < a.dr) {
        x = *reinterpret_cast<const float4*>(krow + d);
        y = *reinterpret_cast<const float4*>(vrow + d);
      }
      kv[4 * u] = x.x;
      kv[4 * u + 1] = x.y;
      kv[4 * u + 2] = x.z;
      kv[4 * u + 3] = x.w;
      vv[4 * u] = y.x;
      vv[4 * u + 1] = y.y;
      vv[4 * u + 2] = y.z;
      vv[4 * u + 3] = y.w;
    }
  }
  const float cs = a.q_flip ? -a.c : a.c;  // Q is staged unflipped

  const int u0 = CAUSAL ? kb0 / BQ : 0;
  const int n_u = (S + BQ - 1) / BQ - u0;
  const int n_it = heads * n_u;

  int go[TI];
#pragma unroll
  for (int i = 0; i < TI; ++i)
    go[i] = tile_offset<D>((i * kF32DqThreads + tid) % SLOTS, i < TI / 2 ? a.qs[1] : a.gs[1], a.dr);
  auto issue = [&](int it, int st) {
    const int hq = hkv * a.group + split * heads + it / n_u;
    const int r0 = (u0 + it % n_u) * BQ;
    const float* qb = static_cast<const float*>(a.q) + b * a.qs[0] + hq * a.qs[2] + start * a.qs[1];
    const float* gb = static_cast<const float*>(a.dout) + b * a.gs[0] + hq * a.gs[2] + start * a.gs[1];
    const rsrc_words qrs = rows_rsrc(qb, S, a.qs[1], a.dr);
    const rsrc_words grs = rows_rsrc(gb, S, a.gs[1], a.dr);
#pragma unroll
    for (int i = 0; i < TI; ++i)
      ld_lds16_asm(i < TI / 2 ? qrs : grs, &QG[st][(i * kF32DqThreads + wave * 64) * 4], go[i],
                 r0 * (int)(i < TI / 2 ? a.qs[1] : a.gs[1]) * (int)sizeof(float));
    if (wave < 2) {
      const float* rb = a.dsum + b * a.lse_bs + hq * a.lse_hs + start + (wave == 0 ? a.lse_n : 0);
      const rsrc_words rrs = make_rsrc_words(rb, S * (int)sizeof(float));
      ld_lds4_asm(rrs, RV[st][wave], lane * (int)sizeof(float), r0 * (int)sizeof(float));
    }
  };

  f32x16 acc_v[DT], acc_k[DT];  // dV^T and dK^T over the block's dims: block dt's row i is dim 128 half + 4 i + dt
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_v[dt][r] = acc_k[dt][r] = 0.f;

  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), seen by the compiler: its own loads are done
  issue(0, 0);
  lds_loads_landed();
  __syncthreads();
  for (int t = 0; t < n_it; ++t) {
    const int st = t & 1;
    if (t + 1 < n_it) issue(t + 1, st ^ 1);
    const float* Qt = QG[st];
    const float* Gt = QG[st] + TILE;
    const int r0 = (u0 + t % n_u) * BQ;

    // S = Q K^T and dP = dO V^T over all 256 dims: register r holds query row r0 + 8 (r / 4) + 4 g + r % 4
    f32x16 s, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
#pragma unroll
    for (int u = 0; u < H / 4; ++u) {
      const float4 qf = *reinterpret_cast<const float4*>(Qt + fat<D>(r32, H * g + 4 * u));
      const float4 gf = *reinterpret_cast<const float4*>(Gt + fat<D>(r32, H * g + 4 * u));
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(qf.x, kv[4 * u], s, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x2f32(gf.x, vv[4 * u], dp, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(qf.y, kv[4 * u + 1], s, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x2f32(gf.y, vv[4 * u + 1], dp, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(qf.z, kv[4 * u + 2], s, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x2f32(gf.z, vv[4 * u + 2], dp, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(qf.w, kv[4 * u + 3], s, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x2f32(gf.w, vv[4 * u + 3], dp, 0, 0, 0);
    }

    // P = exp2(s c - lse2), dS = P (dP - D); masked rows and keys get 0
    float p[16], ds[16];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 l4 = *reinterpret_cast<const float4*>(&RV[st][0][8 * j + 4 * g]);
      const float4 d4 = *reinterpret_cast<const float4*>(&RV[st][1][8 * j + 4 * g]);
      const float lv[4] = {l4.x, l4.y, l4.z, l4.w}, dv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * j + i;
        const int qr = r0 + 8 * j + 4 * g + i;
        const bool masked = qr >= S || (CAUSAL && qr < key);
        p[r] = masked ? 0.f : exp2f(fmaf(s[r], cs, -lv[i]));
        ds[r] = masked ? 0.f : p[r] * (dp[r] - dv[i]);
      }
    }

    // dV^T += dO^T P and dK^T += Q^T dS over dims 128 half + 4 i + dt: product u takes the query row of register u
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int row = 8 * (u >> 2) + 4 * g + (u & 3);
      const Span<DO> gd(Gt + fat<D>(row, 128 * half + 4 * r32));
      const Span<DO> qd(Qt + fat<D>(row, 128 * half + 4 * r32));
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        acc_v[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(gd.v[dt], p[u], acc_v[dt], 0, 0, 0);
        acc_k[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(qd.v[dt], ds[u], acc_k[dt], 0, 0, 0);
      }
    }

    lds_loads_landed();  // this wave's part of the next tile
    __syncthreads();
  }

  if (key_ok) {
    float *dv_out, *dk_out;
    if (a.nsplit > 1) {  // fp32 partials of this block's heads; dkdv_sum_kernel adds the splits
      const int64_t row = (a.cu != nullptr ? (int64_t)start : (int64_t)b * a.S) + key;
      dv_out = a.part + (((int64_t)(split * 2 + 0) * a.rows + row) * a.Hkv + hkv) * D;
      dk_out = a.part + (((int64_t)(split * 2 + 1) * a.rows + row) * a.Hkv + hkv) * D;
    } else {
      dv_out = static_cast<float*>(a.dv) + b * a.dvs[0] + hkv * a.dvs[2] + (int64_t)(start + key) * a.dvs[1];
      dk_out = static_cast<float*>(a.dk) + b * a.dks[0] + hkv * a.dks[2] + (int64_t)(start + key) * a.dks[1];
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = 128 * half + 4 * (8 * (r >> 2) + 4 * g + (r & 3));
      store_span<DO>(dv_out + d, acc_v, r, 1.0f, d, a.dr);
      store_span<DO>(dk_out + d, acc_k, r, a.scale, d, a.dr);  // signed scale: Q was staged unflipped
    }
  }
}

template <int D> int launch_f32(const BwdArgs& a, bool causal, hipStream_t s) {
  const int gp = a.group % 4 == 0 ? 4 : (a.group % 2 == 0 ? 2 : 1);
  const int64_t dq_blocks = (int64_t)((a.S + 32 * (4 / gp) - 1) / (32 * (4 / gp))) * a.B * a.Hq / gp;
  const int64_t kv_blocks = (int64_t)((a.S + BK - 1) / BK) * a.B * a.Hkv * a.nsplit;
  if (causal)
    hipLaunchKernelGGL((attn_bwd_f32_dq_kernel<D, true>), dim3(dq_blocks), dim3(kF32DqThreads), 0, s, a);
  else
    hipLaunchKernelGGL((attn_bwd_f32_dq_kernel<D, false>), dim3(dq_blocks), dim3(kF32DqThreads), 0, s, a);
  if constexpr (D == 256) {  // two blocks per 128 keys, one per half of the output dims
    if (causal)
      hipLaunchKernelGGL((attn_bwd_f32_dkdv_wide_kernel<true>), dim3(2 * kv_blocks), dim3(kF32DqThreads), 0, s, a);
    else
      hipLaunchKernelGGL((attn_bwd_f32_dkdv_wide_kernel<false>), dim3(2 * kv_blocks), dim3(kF32DqThreads), 0, s, a);
  } else if (causal) {
    hipLaunchKernelGGL((attn_bwd_f32_dkdv_kernel<D, true>), dim3(kv_blocks), dim3(kF32DkdvThreads), 0, s, a);
  } else {
    hipLaunchKernelGGL((attn_bwd_f32_dkdv_kernel<D, false>), dim3(kv_blocks), dim3(kF32DkdvThreads), 0, s, a);
  }
  if (a.nsplit > 1) {
    const int64_t n = a.rows * a.Hkv * (a.dr / 4);
    hipLaunchKernelGGL((dkdv_sum_kernel<float, D>), dim3((n + 255) / 256), dim3(256), 0, s, a);
  }
  return launched("pk_attn_bwd");
}
