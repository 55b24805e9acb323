// Attention forward in fp32 on the fp32 matrix cores (v_mfma_f32_32x32x2_f32),
// for Popcorn's float32 attention grid (the 16-bit kernels cover bf16 and
// fp16). Included by attn_fwd.hip inside its namespace, after AttnArgs and
// before the entry points; the work mapping, GQA head packing, causal range
// and packed sequences are the 16-bit forward's.
//
// Each wave holds 32 query rows of one q head and walks the keys in tiles of
// 32. The 32x32x2 product takes one fp32 per lane from each operand: lane
// (row i = lane % 32, half g = lane / 32) gives A[i][g] and B[g][i]. The
// contraction order is free as long as both operands follow it, so:
//   * S^T = K Q^T contracts dims H*g + t at product t (H = D / 2): a lane reads
//     its key's half row of K from LDS in 16-byte pieces and holds its query
//     row's half of Q in registers;
//   * O^T += V^T P^T contracts, at product t, the key that score register t of
//     the lane holds (8 (t / 4) + 4 g + t % 4, the 32x32 accumulator layout),
//     so P^T's operand is the softmax output register t itself and V^T's is a
//     16-byte read from a transposed V tile.
// Scores get an online softmax in the exp2 domain (running max m, sum l, O
// rescaled by exp2(m_old - m_new) when the max grows), the exact algorithm,
// since at fp32 there is no rounding headroom to spend on a fixed reference
// max. K and V tiles are staged through registers into two LDS buffers: the
// next tile's global loads are in flight while the current tile's 2 D
// products run.

#pragma once

constexpr int kF32Threads = 256;

// head_dim 256 holds Q's half row and the O^T accumulator in 256 registers: one wave per SIMD
template <int D, bool CAUSAL>
__global__ __attribute__((amdgpu_flat_work_group_size(kF32Threads, kF32Threads), amdgpu_waves_per_eu(D == 256 ? 1 : 2)))
void attn_fwd_f32_kernel(AttnArgs a) {
  constexpr int H = D / 2;                    // dims per half-wave in the score contraction
  constexpr int DT = D / 32;                  // 32-dim blocks of O^T
  constexpr int KST = D + 4;                  // K row stride in LDS (floats): 16-byte aligned rows
  constexpr int VST = BN + 4;                 // V^T row stride in LDS (floats)
  constexpr int CH = D / 4;                   // 16-byte chunks per row
  constexpr int PER = BN * CH / kF32Threads;  // chunks of a K (or V) tile per thread
  static_assert(PER * kF32Threads == BN * CH, "a tile is a whole number of chunks per thread");
  __shared__ __attribute__((aligned(16))) float Ks[2][BN * KST];
  __shared__ __attribute__((aligned(16))) float Vt[2][D * VST];

  // ---- work item, as the 16-bit forward: (q tile, batch, kv head, head quad)
  const int G = a.group, GP = a.gp;
  const int n_quads = G / GP;
  const int per_tile = a.B * a.Hkv * n_quads;
  const int w = blockIdx.x;
  int m_tile, rest;
  if (per_tile % 8 == 0) {
    const int k = w >> 3;
    m_tile = a.m_tiles - 1 - k % a.m_tiles;
    rest = (w & 7) + 8 * (k / a.m_tiles);
  } else {
    m_tile = a.m_tiles - 1 - w / per_tile;
    rest = w % per_tile;
  }
  const int b = rest / (a.Hkv * n_quads);
  const int hkv = (rest / n_quads) % a.Hkv;
  const int quad = rest % n_quads;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hq = hkv * G + quad * GP + wave % GP;
  const int rows_per_block = 32 * (4 / GP);

  int S = a.S, start = 0;
  if (a.cu != nullptr) {
    start = min(max(a.cu[b], 0), a.total);
    S = min(min(max(a.cu[b + 1], start), a.total) - start, a.S);
  }
  const int m0 = m_tile * rows_per_block;
  if (m0 >= S) return;  // whole block: before any barrier

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int r32 = lane & 31;
  const int g = lane >> 5;
  const int q_row = m0 + (wave / GP) * 32 + r32;

  const float* qbase = static_cast<const float*>(a.q) + b * a.qsb + hq * a.qsh + start * a.qss;
  const float* kbase = static_cast<const float*>(a.k) + b * a.ksb + hkv * a.ksh + start * a.kss;
  const float* vbase = static_cast<const float*>(a.v) + b * a.vsb + hkv * a.vsh + start * a.vss;

  // ---- Q: the lane's query row, dims H*g .. H*g + H - 1 (zeros past head_dim), negated for a negative scale
  float qv[H];
#pragma unroll
  for (int u = 0; u < H / 4; ++u) {
    const int d = H * g + 4 * u;
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (q_row < S && d < a.dr) x = *reinterpret_cast<const float4*>(qbase + (int64_t)q_row * a.qss + d);
    const float sg = a.q_flip ? -1.f : 1.f;
    qv[4 * u] = x.x * sg;
    qv[4 * u + 1] = x.y * sg;
    qv[4 * u + 2] = x.z * sg;
    qv[4 * u + 3] = x.w * sg;
  }

  const int kv_end = CAUSAL ? min(m0 + rows_per_block, S) : S;
  const int n_tiles = (kv_end + BN - 1) / BN;

  // ---- staging: chunk i = j * 256 + tid of a tile is key i / CH, dims 4 (i % CH) .. + 3. At 256 dims a
  // tile goes through the registers in two parts (one staged after the scores, one after the step), so
  // the staging holds 32 registers instead of 64.
  constexpr int PARTS = D == 256 ? 2 : 1;
  constexpr int PP = PER / PARTS;  // chunks per thread per part
  float4 kreg[PP], vreg[PP];
  auto fetch = [&](int tile, int part) {
#pragma unroll
    for (int j = 0; j < PP; ++j) {
      const int i = (part * PP + j) * kF32Threads + tid, key = tile * BN + i / CH, d = 4 * (i % CH);
      const bool ok = key < S && d < a.dr;
      kreg[j] = ok ? *reinterpret_cast<const float4*>(kbase + (int64_t)key * a.kss + d) : make_float4(0.f, 0.f, 0.f, 0.f);
      vreg[j] = ok ? *reinterpret_cast<const float4*>(vbase + (int64_t)key * a.vss + d) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  auto stage = [&](int buf, int part) {
#pragma unroll
    for (int j = 0; j < PP; ++j) {
      const int i = (part * PP + j) * kF32Threads + tid, key = i / CH, d = 4 * (i % CH);
      *reinterpret_cast<float4*>(&Ks[buf][key * KST + d]) = kreg[j];
      Vt[buf][(d + 0) * VST + key] = vreg[j].x;
      Vt[buf][(d + 1) * VST + key] = vreg[j].y;
      Vt[buf][(d + 2) * VST + key] = vreg[j].z;
      Vt[buf][(d + 3) * VST + key] = vreg[j].w;
    }
  };

  f32x16 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;
  float m = -INFINITY, l = 0.f;  // the row's running max (exp2 domain) and sum; both halves of the wave hold them
  const float c = a.c;

#pragma unroll
  for (int part = 0; part < PARTS; ++part) {
    fetch(0, part);
    stage(0, part);
  }
  __syncthreads();
  for (int t = 0; t < n_tiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < n_tiles) fetch(t + 1, 0);

    // S^T = K Q^T: score register r holds key 8 (r / 4) + 4 g + r % 4 of this tile for the lane's row
    f32x16 s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
    const float* krow = &Ks[buf][r32 * KST + H * g];
#pragma unroll
    for (int u = 0; u < H / 4; ++u) {
      const float4 kf = *reinterpret_cast<const float4*>(krow + 4 * u);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.x, qv[4 * u], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.y, qv[4 * u + 1], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.z, qv[4 * u + 2], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.w, qv[4 * u + 3], s, 0, 0, 0);
    }

    // two-part staging: the first part of the next tile into the other buffer (nothing reads it this
    // step), then the second part's loads, in flight over the rest of the step
    if constexpr (PARTS == 2) {
      if (t + 1 < n_tiles) {
        stage(buf ^ 1, 0);
        fetch(t + 1, 1);
      }
    }

    // online softmax over the tile's keys a row may see
    const int lim = CAUSAL ? min(q_row, S - 1) : S - 1;
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = t * BN + 8 * (r >> 2) + 4 * g + (r & 3);
      if (key > lim) s[r] = -INFINITY;
      mx = fmaxf(mx, s[r]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m, mx * c);  // finite from the first tile on: every row sees key 0
    const float alpha = exp2f(m - m_new);
    float ps = 0.f;
    float p[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      p[r] = exp2f(fmaf(s[r], c, -m_new));
      ps += p[r];
    }
    ps += __shfl_xor(ps, 32, 64);
    l = l * alpha + ps;
    m = m_new;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;

    // O^T += V^T P^T: product t takes the key of score register t
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const float* vrow = &Vt[buf][(dt * 32 + r32) * VST + 4 * g];
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const float4 vf = *reinterpret_cast<const float4*>(vrow + 8 * q4);
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf.x, p[4 * q4], o[dt], 0, 0, 0);
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf.y, p[4 * q4 + 1], o[dt], 0, 0, 0);
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf.z, p[4 * q4 + 2], o[dt], 0, 0, 0);
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf.w, p[4 * q4 + 3], o[dt], 0, 0, 0);
      }
    }

    // the next tile into the other buffer, which every wave finished reading in the last step
    if (t + 1 < n_tiles) stage(buf ^ 1, PARTS - 1);
    __syncthreads();
  }

  // ---- O = O^T / l: register r of block dt is dim dt * 32 + 8 (r / 4) + 4 g + r % 4 of the lane's row
  if (q_row < S) {
    const float inv = 1.0f / l;
    float* orow = static_cast<float*>(a.o) + b * a.osb + hq * a.osh + (int64_t)(start + q_row) * a.oss;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = dt * 32 + 8 * q4 + 4 * g;
        if (d < a.dr)
          *reinterpret_cast<float4*>(orow + d) = make_float4(o[dt][4 * q4] * inv, o[dt][4 * q4 + 1] * inv,
                                                             o[dt][4 * q4 + 2] * inv, o[dt][4 * q4 + 3] * inv);
      }
    if (a.lse != nullptr && g == 0)
      a.lse[b * a.lse_bs + hq * a.lse_hs + start + q_row] = (m + log2f(l)) * 0.69314718055994530942f;
  }
}

template <int D> int launch_f32(const AttnArgs& a, int causal, hipStream_t s) {
  const int blocks = a.m_tiles * a.B * a.Hq / a.gp;
  if (causal)
    hipLaunchKernelGGL((attn_fwd_f32_kernel<D, true>), dim3(blocks), dim3(kF32Threads), 0, s, a);
  else
    hipLaunchKernelGGL((attn_fwd_f32_kernel<D, false>), dim3(blocks), dim3(kF32Threads), 0, s, a);
  return launched("pk_attn_fwd");
}
