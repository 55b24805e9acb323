// Attention dK/dV at head_dim 192 and 256 (136-184 laid out at 192, 200-248
// at 256) for the 16-bit dtypes. Included by attn_bwd.hip inside its namespace, after
// dkdv_sum_kernel. The work mapping (128 keys of one (sequence, kv head) per
// block, q-head splits with fp32 partials), the workspace, the LDS swizzle and
// the fragment layouts are the head_dim 64/128 dk/dv kernel's; what changes is
// the split of the work between waves. At 256 dims a 32-row Q or dO tile is
// 16 KB, so that kernel's six stages would not fit in LDS, and one key slice's
// K or V fragments (64 registers) plus its dV or dK accumulator (128) leave no
// room for a second role's wave on the SIMD anyway. Here one wave per 32-key
// slice does both roles, one wave per SIMD (K, V, dK and dV in 384 of its 512
// registers): per query tile S = Q K^T and dP = dO V^T interleaved, then
// P = exp2(s c - lse2) and dS = P (dP - D) in registers (no P hand-off through
// LDS), then dV^T += dO^T P and dK^T += Q^T dS interleaved. Q/dO tiles are
// double-buffered: the next tile's direct loads (inline assembly, so that the
// compiler does not wait for them before reading the other buffer) fly during
// the current step.

#pragma once

constexpr int kWideThreads = 256;  // four 32-key slices, one wave each

template <typename T, int D, bool CAUSAL>
__global__ __attribute__((amdgpu_flat_work_group_size(kWideThreads, kWideThreads), amdgpu_waves_per_eu(1)))
void attn_bwd_dkdv_wide_kernel(BwdArgs a) {
  static_assert(D == 128 || D == 192 || D == 256, "rows of 128, 192 or 256 dims");
  using Frag = typename Mma<T>::frag;
  using L = Tile<D>;
  constexpr int KCH = D / 8;                    // 16-byte chunks per row
  constexpr int SLOTS = BQ * KCH;               // 16-byte slots of a Q (or dO) tile
  constexpr int TILE = BQ * D;                  // elements of a tile
  constexpr int TI = 2 * SLOTS / kWideThreads;  // direct loads per thread per stage: Q, then dO
  constexpr int KK = D / 16;
  constexpr int DT = D / 32;
  __shared__ __attribute__((aligned(16))) T QG[2][2 * TILE];   // buffer: Q tile, then dO tile
  __shared__ __attribute__((aligned(16))) float RV[2][2][64];  // buffer: lse2 rows, D rows (32 used)

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
  const int lane = tid & 63;
  const int r32 = lane & 31;
  const int g = lane >> 5;
  const int kw0 = kb0 + wave * 32;
  const int key = kw0 + r32;
  const bool key_ok = key < S;

  // the lane's K and V rows as B operands: fragment h holds dims 16 h + 8 g .. + 7
  Frag kf[KK], vf[KK];
  {
    const T* krow = static_cast<const T*>(a.k) + b * a.ks[0] + hkv * a.ks[2] + (int64_t)(start + key) * a.ks[1];
    const T* vrow = static_cast<const T*>(a.v) + b * a.vs[0] + hkv * a.vs[2] + (int64_t)(start + key) * a.vs[1];
#pragma unroll
    for (int h = 0; h < KK; ++h) {
      uint4 x = make_uint4(0, 0, 0, 0), y = x;
      if (key_ok && 2 * h + g < a.dch) {
        x = *reinterpret_cast<const uint4*>(krow + 16 * h + 8 * g);
        y = *reinterpret_cast<const uint4*>(vrow + 16 * h + 8 * g);
      }
      kf[h] = __builtin_bit_cast(Frag, x);
      vf[h] = __builtin_bit_cast(Frag, y);
    }
    // these loads complete before the first inline-assembly load
#pragma unroll
    for (int h = 0; h < KK; ++h) asm volatile("" ::"v"(kf[h]), "v"(vf[h]));
  }
  // Q is staged unflipped: a negative scale signs the exponent's coefficient here and dK's final scale
  const float cs = a.q_flip ? -a.c : a.c;

  // query tiles: every q head of the block's share of the group, rows from the block's first key on (causal)
  const int u0 = CAUSAL ? kb0 / BQ : 0;
  const int n_u = (S + BQ - 1) / BQ - u0;
  const int n_it = heads * n_u;

  // staging: slot sl = i * threads + tid of a stage (Q slots, then dO slots) is row (sl % SLOTS) / KCH of
  // its tile, stored chunk sl % KCH, which holds logical chunk (sl % KCH) ^ swz(row)
  static_assert(TI % 2 == 0 && (TI / 2) * kWideThreads == SLOTS, "a thread's loads split evenly over Q and dO");
  int go[TI];
#pragma unroll
  for (int i = 0; i < TI; ++i) {
    const int within = (i * kWideThreads + tid) % SLOTS;
    const int row = within / KCH, c = (within % KCH) ^ L::swz(row);
    go[i] = c < a.dch ? (row * (int)(i < TI / 2 ? a.qs[1] : a.gs[1]) + c * 8) * (int)sizeof(T) : (int)kPadOffset;
  }
  // tile it (q head it / n_u of the block's, q tile u0 + it % n_u) into buffer st; waves 0 and 1 also load its
  // rows' lse2 and D. Rows past the end read as zero (their p is masked).
  auto issue = [&](int it, int st) {
    const int hq = hkv * a.group + split * heads + it / n_u;
    const int r0 = (u0 + it % n_u) * BQ;
    const T* qb = static_cast<const T*>(a.q) + b * a.qs[0] + hq * a.qs[2] + start * a.qs[1];
    const T* gb = static_cast<const T*>(a.dout) + b * a.gs[0] + hq * a.gs[2] + start * a.gs[1];
    const rsrc_words qrs = make_rsrc_words(qb, (int)(((int64_t)(S - 1) * a.qs[1] + a.dr) * (int)sizeof(T)));
    const rsrc_words grs = make_rsrc_words(gb, (int)(((int64_t)(S - 1) * a.gs[1] + a.dr) * (int)sizeof(T)));
#pragma unroll
    for (int i = 0; i < TI; ++i)
      ld_lds16_asm(i < TI / 2 ? qrs : grs, QG[st] + (i * kWideThreads + wave * 64) * 8, go[i],
                 r0 * (int)(i < TI / 2 ? a.qs[1] : a.gs[1]) * (int)sizeof(T));
    if (wave < 2) {
      const float* rb = a.dsum + b * a.lse_bs + hq * a.lse_hs + start + (wave == 0 ? a.lse_n : 0);
      const rsrc_words rrs = make_rsrc_words(rb, S * (int)sizeof(float));
      ld_lds4_asm(rrs, RV[st][wave], lane * (int)sizeof(float), r0 * (int)sizeof(float));
    }
  };

  // Lane offsets of the fragment reads. The tile swizzle repeats every PERIOD
  // elements of a row (128 at 128 and 256 dims, 64 at 192), so fragment h
  // (or block dt) of a later period is the first period's offset plus whole
  // periods.
  constexpr int PERIOD = D == 192 ? 64 : 128;
  constexpr int KH = PERIOD / 16, DH = PERIOD / 32;
  int a_lane[KH], t_lane[2][DH];
#pragma unroll
  for (int h = 0; h < KH; ++h) a_lane[h] = L::at(r32, 16 * h + 8 * g);
#pragma unroll
  for (int hi = 0; hi < 2; ++hi)
#pragma unroll
    for (int dt = 0; dt < DH; ++dt)
      t_lane[hi][dt] = L::at(8 * hi + 4 * g + ((lane & 15) >> 2), 32 * dt + 16 * ((lane >> 4) & 1) + 4 * (lane & 3));
  // row fragment h of a tile (A operand of a score product: its 32 rows, dims 16 h + 8 g ..)
  auto row_frag = [&](const T* tile, int h) -> Frag {
    return *reinterpret_cast<const Frag*>(tile + a_lane[h % KH] + (h / KH) * PERIOD);
  };
  // transposed fragment of a tile (A operand of an accumulation: dims 32 dt + row l % 32, rows of chunk c)
  auto col_frag = [&](const T* tile, int c, int dt) -> Frag {
    const int off = 16 * c * L::ST + (dt / DH) * PERIOD;
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(tile + t_lane[0][dt % DH] + off));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(tile + t_lane[1][dt % DH] + off));
    return __builtin_bit_cast(Frag, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  // 32 products in order, each A fragment read kRing products ahead of it; the scheduling barrier after
  // each product keeps the compiler from hoisting every read (and its registers) to the front
  constexpr int kRing = 4, NP = 2 * KK;
  static_assert(NP == 4 * DT && kRing <= NP, "32 score products and 32 accumulation products per step");
  auto run = [&](auto fetch, auto product) {
    Frag ring[kRing];
#pragma unroll
    for (int i = 0; i < kRing; ++i) ring[i] = fetch(i);
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const Frag f = ring[i % kRing];
      if (i + kRing < NP) ring[i % kRing] = fetch(i + kRing);
      product(i, f);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  f32x16 acc_v[DT], acc_k[DT];  // dV^T and dK^T: block dt's row i is dim 32 dt + i, the column the lane's key
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_v[dt][r] = acc_k[dt][r] = 0.f;

  issue(0, 0);
  lds_loads_landed();
  __syncthreads();
  for (int t = 0; t < n_it; ++t) {
    const int st = t & 1;
    // the next tile into the other buffer, which every wave finished reading in the last step
    if (t + 1 < n_it) issue(t + 1, st ^ 1);
    const T* Qt = QG[st];
    const T* Gt = QG[st] + TILE;

    // S = Q K^T and dP = dO V^T: register r holds query row r0 + 8 (r / 4) + 4 g + r % 4 of the lane's key.
    // Product 2h scores fragment h of Q against K, 2h + 1 that of dO against V.
    f32x16 s, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
    run(
        [&](int i) { return row_frag(i & 1 ? Gt : Qt, i >> 1); },
        [&](int i, const Frag& f) {
          if (i & 1)
            dp = Mma<T>::run(f, vf[i >> 1], dp);
          else
            s = Mma<T>::run(f, kf[i >> 1], s);
        });

    // P = exp2(s c - lse2) and dS = P (dP - D); keys a row must not see, and rows or keys past the end, get 0.
    // The test for a mask is wave-uniform (the slice's keys), so unmasked steps branch past it.
    const int r0 = (u0 + t % n_u) * BQ;
    const bool need_mask = (CAUSAL && r0 < kw0 + 32) || kw0 + 32 > S || r0 + BQ > S;
    Frag pf[2], sf[2];  // B operands: register 8 c + j of the score block is element j of fragment c
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 l4 = *reinterpret_cast<const float4*>(&RV[st][0][8 * j + 4 * g]);
      const float4 d4 = *reinterpret_cast<const float4*>(&RV[st][1][8 * j + 4 * g]);
      const float lv[4] = {l4.x, l4.y, l4.z, l4.w}, dv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * j + i;
        const int qrow = r0 + 8 * j + 4 * g + i;
        float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], cs, -lv[i]));
        if (need_mask) p = (key_ok & (qrow < S) & (!CAUSAL | (key <= qrow))) ? p : 0.f;
        pf[r >> 3][r & 7] = (T)p;
        sf[r >> 3][r & 7] = (T)(p * (dp[r] - dv[i]));
      }
    }

    // dV^T += dO^T P and dK^T += Q^T dS: product 2h (h = DT c + dt) accumulates block dt of dV^T over the 16
    // query rows of fragment c, 2h + 1 the same block of dK^T
    run(
        [&](int i) { return col_frag(i & 1 ? Qt : Gt, (i >> 1) / DT, (i >> 1) % DT); },
        [&](int i, const Frag& f) {
          const int dt = (i >> 1) % DT, c = (i >> 1) / DT;
          if (i & 1)
            acc_k[dt] = Mma<T>::run(f, sf[c], acc_k[dt]);
          else
            acc_v[dt] = Mma<T>::run(f, pf[c], acc_v[dt]);
        });

    lds_loads_landed();  // this wave's part of the next tile
    __syncthreads();
  }

  if (key_ok) {
    if (a.nsplit > 1) {
      // fp32 partials of this block's heads; dkdv_sum_kernel adds the splits
      const int64_t row = (a.cu != nullptr ? (int64_t)start : (int64_t)b * a.S) + key;
      float* dv_out = a.part + (((int64_t)(split * 2 + 0) * a.rows + row) * a.Hkv + hkv) * D;
      float* dk_out = a.part + (((int64_t)(split * 2 + 1) * a.rows + row) * a.Hkv + hkv) * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const int d = dt * 32 + 8 * rq + 4 * g;
          if (d < a.dr) {
            *reinterpret_cast<float4*>(dv_out + d) =
                make_float4(acc_v[dt][4 * rq], acc_v[dt][4 * rq + 1], acc_v[dt][4 * rq + 2], acc_v[dt][4 * rq + 3]);
            *reinterpret_cast<float4*>(dk_out + d) =
                make_float4(acc_k[dt][4 * rq] * a.scale, acc_k[dt][4 * rq + 1] * a.scale,
                            acc_k[dt][4 * rq + 2] * a.scale, acc_k[dt][4 * rq + 3] * a.scale);
          }
        }
    } else {
      T* dv_out = static_cast<T*>(a.dv) + b * a.dvs[0] + hkv * a.dvs[2] + (int64_t)(start + key) * a.dvs[1];
      T* dk_out = static_cast<T*>(a.dk) + b * a.dks[0] + hkv * a.dks[2] + (int64_t)(start + key) * a.dks[1];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const int d = dt * 32 + 8 * rq + 4 * g;
          if (d < a.dr) {
            *reinterpret_cast<uint2*>(dv_out + d) =
                pack4<T>(acc_v[dt][4 * rq], acc_v[dt][4 * rq + 1], acc_v[dt][4 * rq + 2], acc_v[dt][4 * rq + 3]);
            *reinterpret_cast<uint2*>(dk_out + d) =
                pack4<T>(acc_k[dt][4 * rq] * a.scale, acc_k[dt][4 * rq + 1] * a.scale,
                         acc_k[dt][4 * rq + 2] * a.scale, acc_k[dt][4 * rq + 3] * a.scale);
          }
        }
    }
  }
}

// head_dim 136-256 in bf16 or fp16 (rows of D = 192 or 256): the dq kernel at D and the single-role dk/dv kernel
template <typename T, int D> int launch_wide(const BwdArgs& a, bool causal, hipStream_t s) {
  const int gp = a.group % 4 == 0 ? 4 : (a.group % 2 == 0 ? 2 : 1);
  const int64_t dq_blocks = (int64_t)((a.S + 32 * (4 / gp) - 1) / (32 * (4 / gp))) * a.B * a.Hq / gp;
  const int64_t kv_blocks = (int64_t)((a.S + BK - 1) / BK) * a.B * a.Hkv * a.nsplit;
  if (causal) {
    hipLaunchKernelGGL((attn_bwd_dq_kernel<T, D, true>), dim3(dq_blocks), dim3(NT), 0, s, a);
    hipLaunchKernelGGL((attn_bwd_dkdv_wide_kernel<T, D, true>), dim3(kv_blocks), dim3(kWideThreads), 0, s, a);
  } else {
    hipLaunchKernelGGL((attn_bwd_dq_kernel<T, D, false>), dim3(dq_blocks), dim3(NT), 0, s, a);
    hipLaunchKernelGGL((attn_bwd_dkdv_wide_kernel<T, D, false>), dim3(kv_blocks), dim3(kWideThreads), 0, s, a);
  }
  if (a.nsplit > 1) {
    const int64_t n = a.rows * a.Hkv * (a.dr / 4);
    hipLaunchKernelGGL((dkdv_sum_kernel<T, D>), dim3((n + 255) / 256), dim3(256), 0, s, a);
  }
  return launched("pk_attn_bwd");
}
