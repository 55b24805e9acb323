// Attention forward (flash-style, grouped-query, optional causal mask) on
// gfx950 matrix cores.
//
// Block = 4 wavefronts of 32 query rows each, over one (batch, kv head):
// gp q heads of that kv head's group (4, 2 or 1, the largest dividing the
// group size) x 4/gp consecutive row groups. With 4 q heads per kv head every
// wave holds the same 32 rows of its own head, so the block's K/V tiles serve
// all four and every wave sees the same causal range. Three blocks share a CU
// (three waves per SIMD). Keys stream through LDS in tiles of BN = 32.
//
// Per tile each wave computes
//   S^T (32 keys x 32 queries)  = K_tile . Q^T   (v_mfma_f32_32x32x16, K from
//                                                 LDS, Q^T held in registers)
//   O^T (head_dim x 32 queries) += V^T . P^T
// Working on transposes puts one query per lane column: the MFMA result
// layout gives lane l the 16 entries of query l%32 in key rows
// 8*(r/4) + 4*(l/32) + r%4, so the softmax sums are in-lane except for one
// exchange with lane l^32. P leaves the accumulator registers directly as the
// B operand of the second product: the key order inside each 16-key MFMA
// step is permuted identically in P^T and in the V^T fragments, which the
// contraction does not see.
//
// Per step (per wave): step t masks S(t) and exponentiates it into P(t),
// then issues one run of matrix products, O += V(t)^T P(t)^T followed by
// S(t+1) = K(t+1) Q^T written over S(t), whose LDS fragment reads run kRing
// products ahead of their use. One S array (not two) leaves the registers
// for that read-ahead, and the three waves that share a SIMD overlap one
// wave's softmax with another's products. Staging runs ahead of that: the
// step starts by issuing K(t+2) and V(t+1) as buffer loads that write LDS
// directly (no staging registers, no LDS stores), into buffers every wave
// has finished with, and ends once they have landed; one barrier per step.
// The head_dim-128 kernel fits three waves per SIMD (three blocks per CU).
//
// Softmax with a fixed reference max: m is the row max of s * c over the
// first key tile (key 0 is visible to every row) and stays put, so no step
// computes a row max or rescales O; p = exp2(s * c - m) is one FMA plus one
// exp, with c = |scale| * log2(e) (a negative scale negates Q on load, which
// is exact). Later scores may exceed m: o = acc / l and lse = m + log(l) are
// unchanged by the choice of m as long as P and the sums stay in range, which
// holds while l stays below 2^32 (2^15 for fp16, whose P must fit in fp16:
// every p is at most l). A block where some row's l leaves that range, or is
// not finite, sweeps its keys again with the exact online max (rescaling O
// when the max grows by more than 2^8), so the result never depends on the
// data being benign. The log-sum-exp output is converted back to natural log.
//
// LDS layouts (a tile is contiguous 16-byte slots; a wave's direct load fills
// 64 consecutive slots, each lane fetching the chunk its slot holds, and a
// lane whose K slot is padding reads past the buffer's range, which returns
// zeros without a memory access):
//   K [BN][D + 8]: 16-byte fragment reads of 16 consecutive rows start 272,
//       208 or 144 bytes apart and so cover all 64 banks once.
//   V [BN][D], unpadded, with chunk c of row r at slot c ^ vswz(r). V^T
//       fragments come from ds_read_b64_tr_b16: within a 16-lane group, lane
//       s reads keys base + s/4, dims d0 + 4*(s%4) .. +3, and lane i receives
//       dims d0 + i of keys base .. base + 3 -- half of one MFMA A fragment.
//       The two 16-lane groups served together read 4 rows x 4 chunks, which
//       the swizzle places in 16 distinct slots of a 256-byte bank window.
//       96-dim rows (192 bytes) need no swizzle: 4 consecutive rows start 0,
//       192, 128 and 64 bytes into that window.
//
// K and V are read through buffer resources based at the (batch, kv head):
// a tile is one scalar offset, and rows at or past S read as zero, so no load
// is predicated; such keys are masked like causal ones. Work order: each XCD
// (dispatch is round-robin over the 8 XCDs) runs its (batch, kv head) groups
// one after another, longest causal rows first within a group, so the blocks
// resident on an XCD read the same K/V prefix.
#include <math.h>

#include <type_traits>

#include "api.h"
#include "attn_common.h"

namespace pk {
namespace {

using namespace attn;

constexpr int BN = 32;
constexpr int NT = 256;
// fragment reads in flight ahead of the product that uses them (head_dim 256,
// whose Q^T fragments and O^T accumulators take 192 registers, keeps fewer)
template <int D> constexpr int kRing = D >= 192 ? 3 : (D == 32 ? 4 : 6);  // at most the step's 2 * D / 16 products
// Buffer offset of a padding slot: at or past every range the kernel builds
// (each below 2^31), and with a tile offset below 2^31 added it cannot wrap.
constexpr uint32_t kPadOffset = 0x80000000u;

// Slot of chunk c of V row r is c ^ vswz(r): the two 16-lane groups of a
// transposing read cover 4 rows x 4 chunks, which this spreads over 16
// distinct slots of a 256-byte bank window (rows of head_dim 64 are 128 bytes;
// 96-dim rows, 192 bytes, already start 64 bytes apart modulo the window, and
// 192-dim rows, 384 bytes, 128 bytes apart, which the swizzle halves).
template <int D> __device__ __forceinline__ int vswz(int r) {
  if constexpr (D == 32 || D == 96) return 0;  // 64-byte rows: four of them fill the window
  else if constexpr (D == 192) return 4 * ((r >> 1) & 1);
  else return D >= 128 ? 4 * (r & 3) : 4 * ((r >> 1) & 1);
}

// Largest row sum the fixed-max sweep accepts (see the header).
template <typename T> constexpr float kFastLimit = 4294967296.0f;
template <> constexpr float kFastLimit<f16> = 32768.0f;

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  // Packed sequences: sequence b holds tokens [cu[b], cu[b+1]) of `total`,
  // batch strides are 0 and S is the longest sequence. NULL: a dense batch.
  const int* cu;
  int total;
  int64_t qsb, qss, qsh, ksb, kss, ksh, vsb, vss, vsh, osb, oss, osh;
  int64_t lse_bs, lse_hs;  // lse element (b, h, token t of b) at b*lse_bs + h*lse_hs + t (+ cu[b] when packed)
  int B, S, Hq, Hkv, group, m_tiles;
  int gp;  // q heads of one kv group per block (4, 2 or 1); the block's 4 waves are gp heads x 4/gp row groups
  float c;          // |scale| * log2(e), at least 1e-30
  uint32_t q_flip;  // 0x80008000 when scale < 0 (negates both halves of a packed pair), else 0
  // head_dim of the tensors (a multiple of 8, at most the kernel's D) and its
  // 16-byte chunks: the kernel lays rows out at D and reads zeros past them
  int dr, dch;
};

// KS: 16-dim steps of the score products, D / 16, or one fewer when the row's
// last 16 dims are all past head_dim (zeros in Q and K, so the step adds exact
// zeros and skipping it changes no bit)
template <typename T, int D, bool CAUSAL, int KS>
__global__ __attribute__((amdgpu_flat_work_group_size(NT, NT), amdgpu_waves_per_eu(2))) void attn_fwd_kernel(
    AttnArgs a) {
  using Frag = typename Mma<T>::frag;
  constexpr int KST = D + 8;   // K row stride in LDS, elements
  constexpr int KCH = D / 8;   // 16-byte chunks per K/V row
  constexpr int KK = D / 16;
  constexpr int DT = D / 32;
  static_assert(KS == KK || KS == KK - 1, "at most the last 16-dim step is skipped");
  __shared__ __attribute__((aligned(16))) T Ks[2][BN * KST];
  __shared__ __attribute__((aligned(16))) T Vs[2][BN * D];

  // ---- work item: (q tile, batch, kv head, head quad) -- a group is one
  // (batch, kv head, quad). A block's waves are gp q heads of one kv group x
  // 4/gp row groups of 32, so its K/V tiles serve every head it holds.
  const int G = a.group, GP = a.gp;
  const int n_quads = G / GP;
  const int per_tile = a.B * a.Hkv * n_quads;
  const int w = blockIdx.x;
  // With a multiple of 8 groups, XCD x (block w runs on XCD w % 8) takes
  // groups x, x + 8, ... one after another, each group's q tiles longest
  // first: the ~96 blocks resident on an XCD then share one group's K/V
  // prefix in its L2 (4.4x less HBM fetch at C5 than interleaving four
  // groups per XCD). Otherwise q tiles run longest first over all groups.
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
  const int wave_id = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hq = hkv * G + quad * GP + wave_id % GP;
  const int rows_per_block = 32 * (4 / GP);

  // this block's sequence: all of it for a dense batch; tokens [cu[b], cu[b+1])
  // of a packed one (clamped, so a malformed table cannot address past `total`)
  int S = a.S, start = 0;
  if (a.cu != nullptr) {
    start = min(max(a.cu[b], 0), a.total);
    S = min(min(max(a.cu[b + 1], start), a.total) - start, a.S);
  }
  const int m0 = m_tile * rows_per_block;
  if (m0 >= S) return;  // whole block: before any barrier

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r32 = lane & 31;
  const int g = lane >> 5;
  const int wave_first = m0 + (wave / GP) * 32;
  const int q_row = wave_first + r32;

  const T* qbase = static_cast<const T*>(a.q) + b * a.qsb + hq * a.qsh + start * a.qss;
  const T* kbase = static_cast<const T*>(a.k) + b * a.ksb + hkv * a.ksh + start * a.kss;
  const T* vbase = static_cast<const T*>(a.v) + b * a.vsb + hkv * a.vsh + start * a.vss;
  // K/V of this (sequence, kv head) through buffer resources: rows at or past
  // S read as zero (range-checked), and a tile's base is one scalar offset.
  const int k_bytes = (int)(((int64_t)(S - 1) * a.kss + a.dr) * (int)sizeof(T));
  const int v_bytes = (int)(((int64_t)(S - 1) * a.vss + a.dr) * (int)sizeof(T));
  const __amdgpu_buffer_rsrc_t krsrc = __builtin_amdgcn_make_buffer_rsrc((void*)kbase, (short)0, k_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrsrc = __builtin_amdgcn_make_buffer_rsrc((void*)vbase, (short)0, v_bytes, 0x00020000);
  // 32-, 96-, 192- and 256-dim rows stage their tiles through the
  // inline-assembly loads, so the step's fragment reads do not first wait for
  // the step's own prefetch (each step waits for all its loads before its
  // closing barrier). Measured slower at 128 dims and no faster at 64.
  constexpr bool kAsmLoads = D != 64 && D != 128;
  const rsrc_words kwords = make_rsrc_words(kbase, k_bytes), vwords = make_rsrc_words(vbase, v_bytes);

  // ---- Q^T fragments: qf[kk] = Q[q_row][16kk + 8g .. +8], sign-flipped for a negative scale
  Frag qf[KS];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    uint4 raw = make_uint4(0, 0, 0, 0);
    if (q_row < S && 2 * kk + g < a.dch)
      raw = *reinterpret_cast<const uint4*>(qbase + (int64_t)q_row * a.qss + 16 * kk + 8 * g);
    raw.x ^= a.q_flip;
    raw.y ^= a.q_flip;
    raw.z ^= a.q_flip;
    raw.w ^= a.q_flip;
    qf[kk] = __builtin_bit_cast(Frag, raw);
  }
  // the compiler's own loads complete (a wait it sees: vmcnt(0)) before the first inline-assembly load
  if constexpr (kAsmLoads) __builtin_amdgcn_s_waitcnt(0x0F70);

  const int kv_end = CAUSAL ? min(m0 + rows_per_block, S) : S;
  const int n_tiles = (kv_end + BN - 1) / BN;

  // ---- tile staging straight into LDS: a padded K tile is KSLOTS 16-byte
  // slots, slot s of a wave instruction landing at its base + 16*lane; the
  // lane fetches the global chunk its slot holds, and pad slots read out of
  // range (zeros, no memory traffic; nobody reads them)
  constexpr int KSPR = KST / 8;  // slots per padded K row
  constexpr int KSLOTS = BN * KSPR;
  constexpr int KI = (KSLOTS + NT - 1) / NT;
  int kgo[KI];
#pragma unroll
  for (int i = 0; i < KI; ++i) {
    const int sl = i * NT + tid, row = sl / KSPR, col = sl % KSPR;
    kgo[i] = col < a.dch ? (row * (int)a.kss + col * 8) * (int)sizeof(T) : (int)kPadOffset;
  }
  // V rows are unpadded, chunk c of row r at slot c ^ vswz(r). Where a row
  // has a power-of-two count of chunks, the rows of one instruction's slots
  // differ from the next's by NT / KCH (a multiple of 4), so every instruction
  // shares the lane's chunk and only the row base moves; 32-, 96- and 192-dim
  // rows (4, 12 and 24 chunks) take an offset per instruction (for 32 and 96
  // dims the last one covers the tile's remaining 128 slots).
  constexpr int VSLOTS = BN * KCH;
  constexpr bool VWHOLE = NT % KCH == 0 && VSLOTS % NT == 0;
  constexpr int VI = (VSLOTS + NT - 1) / NT;
  static_assert(VWHOLE ? (NT / KCH) % 4 == 0 : ((D == 32 || D == 96 || D == 192) && VSLOTS % 64 == 0),
                "V staging covers whole rows, or whole waves of slots");
  int vgo[VWHOLE ? 1 : VI];
  if constexpr (VWHOLE) {
    const int row = tid / KCH, pos = tid % KCH, chunk = pos ^ vswz<D>(row);
    vgo[0] = chunk < a.dch ? (row * (int)a.vss + chunk * 8) * (int)sizeof(T) : (int)kPadOffset;
  } else {
#pragma unroll
    for (int i = 0; i < VI; ++i) {
      const int sl = i * NT + tid, row = sl / KCH, chunk = (sl % KCH) ^ vswz<D>(row);
      vgo[i] = chunk < a.dch ? (row * (int)a.vss + chunk * 8) * (int)sizeof(T) : (int)kPadOffset;
    }
  }
  // this lane's element offsets: K fragment kk at k_lane + 16 kk (row r32,
  // dims 16kk + 8g ..), and the transposing V reads (see pv)
  const int k_lane = r32 * KST + 8 * g;
  // V^T reads: the lane reads key row kr (+ 16c + 8h), dims 32 dt +
  // 16 ((lane >> 4) & 1) + 4 (lane & 3) .. +3, i.e. chunk 4 dt + vq; with the
  // swizzle that chunk sits at 4 (dt ^ vs) + vq, one offset per dt
  int v_dt[DT];
  {
    const int kr = 4 * g + ((lane & 15) >> 2);
    const int vq = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
    const int vs = vswz<D>(kr) / 4;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) v_dt[dt] = kr * D + (4 * (dt ^ vs) + vq) * 8 + 4 * (lane & 1);
  }

  // tile t of K into Ks[buf] / of V into Vs[buf], asynchronously (vmcnt)
  auto dma_k = [&](int t, int buf) {
    const int tile = t * BN * (int)a.kss * (int)sizeof(T);
#pragma unroll
    for (int i = 0; i < KI; ++i)
      if (KSLOTS % NT == 0 || i * NT + tid < KSLOTS)
      {
        if constexpr (kAsmLoads)
          ld_lds16_asm(kwords, Ks[buf] + (i * NT + wave * 64) * 8, kgo[i], tile);
        else
          ld_buf_lds(krsrc, Ks[buf] + (i * NT + wave * 64) * 8, kgo[i], tile);
      }
  };
  auto dma_v = [&](int t, int buf) {
    const int tile = t * BN * (int)a.vss * (int)sizeof(T);
#pragma unroll
    for (int i = 0; i < VI; ++i) {
      if constexpr (VWHOLE)
      {
        if constexpr (kAsmLoads)
          ld_lds16_asm(vwords, Vs[buf] + (i * NT + wave * 64) * 8, vgo[0],
                       tile + i * (NT / KCH) * (int)a.vss * (int)sizeof(T));
        else
          ld_buf_lds(vrsrc, Vs[buf] + (i * NT + wave * 64) * 8, vgo[0],
                     tile + i * (NT / KCH) * (int)a.vss * (int)sizeof(T));
      }
      else if (VSLOTS % NT == 0 || i * NT + wave * 64 < VSLOTS)  // wave-uniform
      {
        if constexpr (kAsmLoads)
          ld_lds16_asm(vwords, Vs[buf] + (i * NT + wave * 64) * 8, vgo[i], tile);
        else
          ld_buf_lds(vrsrc, Vs[buf] + (i * NT + wave * 64) * 8, vgo[i], tile);
      }
    }
  };
  auto landed = [&]() { lds_loads_landed(); };
  // S^T of the K tile in buffer buf
  auto scores = [&](int buf) {
    const T* ks = Ks[buf];
    f32x16 s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) s = Mma<T>::run(*reinterpret_cast<const Frag*>(ks + k_lane + 16 * kk), qf[kk], s);
    return s;
  };
  // whether tile t holds keys some row of this wave must not see
  auto need_mask = [&](int t) { return (CAUSAL && t * BN + BN - 1 > wave_first) || t * BN + BN > S; };
  auto apply_mask = [&](int t, f32x16& s) {
    // last visible key of this lane's query; rows past the end (zero loads) are masked too
    const int lim = CAUSAL ? min(q_row, S - 1) : S - 1;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = t * BN + 8 * (r >> 2) + 4 * g + (r & 3);
      s[r] = key <= lim ? s[r] : -INFINITY;
    }
  };
  f32x16 acc[DT];
  // O^T += V^T P^T over the tile's two 16-key steps. V^T fragments come from
  // transposing reads of row-major V: within each 16-lane group, lane s reads
  // keys (base + s/4), dims (d0 + 4*(s%4)) .. +3, and lane i receives dims
  // d0 + i of keys base .. base + 3.
  auto vfrag = [&](const T* vb, int c, int dt) -> Frag {
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(vb + v_dt[dt] + 16 * c * D));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(vb + v_dt[dt] + (16 * c + 8) * D));
    return __builtin_bit_cast(Frag, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };
  auto pv = [&](int buf, const Frag (&pf)[2]) {
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[dt] = Mma<T>::run(vfrag(Vs[buf], c, dt), pf[c], acc[dt]);
  };
  float m_i;  // reference max of s * c for query q_row
  float l_i;  // this lane's half of the denominator
  // P = exp2(s * c - m) as the B fragments of the two 16-key steps; l += row sum
  auto softmax = [&](const f32x16& s, float m_use, Frag (&pf)[2]) {
    float rs;  // starts at the first p, not at 0 (0 + p is an instruction)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[8 * c + j], a.c, -m_use));
        rs = c == 0 && j == 0 ? p : rs + p;
        pf[c][j] = (T)p;
      }
    l_i += rs;
  };
  auto clear = [&]() {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[dt][r] = 0.f;
    l_i = 0.f;
  };

  // ---- fast sweep: fixed max; each step exponentiates S(t), then runs the
  // products of O += V(t)^T P(t)^T and S(t+1) over the same S registers
  clear();
  dma_k(0, 0);
  dma_v(0, 0);
  dma_k(1, 1);  // past the end this reads zeros or keys nobody uses
  landed();
  __syncthreads();
  f32x16 sc = scores(0);
  if (need_mask(0)) apply_mask(0, sc);
  {
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[r]);
    m_i = fmaxf(mx, __shfl_xor(mx, 32, 64)) * a.c;
  }
  __syncthreads();  // K(0) is read; the first step overwrites its buffer
  Frag pf[2];
  // Step t. Buffers: V(t) in Vs[t&1] and K(t+1) in Ks[(t+1)&1] are read;
  // K(t+2) goes to Ks[t&1] and V(t+1) to Vs[(t+1)&1], whose previous tiles
  // were last read in step t-1. Product i < KK is V^T P^T step i (16 keys c =
  // i / DT, head dims 32 * (i % DT) ..); product KK + kk is S^T step kk.
  // Fragment i + kRing is read as product i issues, and sched_barrier keeps
  // that order (the compiler would otherwise bunch the reads).
  // The step is unrolled over the two buffer parities (P = t & 1), so every
  // LDS fragment address is a lane register plus an immediate.
  auto step = [&](int t, auto parity) {
    constexpr int P = decltype(parity)::value;
    dma_k(min(t + 2, n_tiles), P);
    dma_v(min(t + 1, n_tiles - 1), P ^ 1);
    if (need_mask(t)) apply_mask(t, sc);
    softmax(sc, m_i, pf);
    const T* ks = Ks[P ^ 1] + k_lane;
    auto fetch = [&](int i) -> Frag {
      if (i < KK) return vfrag(Vs[P], i / DT, i % DT);
      return *reinterpret_cast<const Frag*>(ks + 16 * (i - KK));
    };
    constexpr int N = KK + KS;  // 2 * DT == KK products of V^T P^T, KS of S^T
    constexpr int R = kRing<D> < N ? kRing<D> : N;
    Frag ring[R];
#pragma unroll
    for (int i = 0; i < R; ++i) ring[i] = fetch(i);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const Frag f = ring[i % R];
      if (i + R < N) ring[i % R] = fetch(i + R);
      if (i < KK) {
        acc[i % DT] = Mma<T>::run(f, pf[i / DT], acc[i % DT]);
      } else {
        if (i == KK) {
#pragma unroll
          for (int r = 0; r < 16; ++r) sc[r] = 0.f;
        }
        sc = Mma<T>::run(f, qf[i - KK], sc);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    landed();
    __syncthreads();
  };
  for (int t = 0;;) {
    step(t, std::integral_constant<int, 0>{});
    if (++t >= n_tiles) break;
    step(t, std::integral_constant<int, 1>{});
    if (++t >= n_tiles) break;
  }

  {
    const float l_tot = l_i + __shfl_xor(l_i, 32, 64);
    const bool bad = !(l_tot <= kFastLimit<T>) || !(fabsf(m_i) < INFINITY);
    if (__syncthreads_or(bad)) {
      // ---- exact sweep: online max; O and l are rescaled only when the max
      // grows by more than 2^8 (exponents stay <= 8, and o = acc / l uses the
      // same max in both)
      clear();
      m_i = -INFINITY;
      dma_k(0, 0);
      dma_v(0, 0);
      landed();
      __syncthreads();
      for (int u = 0; u < n_tiles; ++u) {
        dma_k(min(u + 1, n_tiles - 1), (u + 1) & 1);
        dma_v(min(u + 1, n_tiles - 1), (u + 1) & 1);
        f32x16 s = scores(u & 1);
        if (need_mask(u)) apply_mask(u, s);
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[r]);
        const float m_cand = fmaxf(mx, __shfl_xor(mx, 32, 64)) * a.c;
        if (!__all(m_cand <= m_i + 8.0f)) {
          const float m_new = fmaxf(m_i, m_cand);
          const float alpha = __builtin_amdgcn_exp2f(m_i - m_new);  // 0 when m_i = -inf
          l_i *= alpha;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[dt][r] *= alpha;
          m_i = m_new;
        }
        softmax(s, m_i == -INFINITY ? 0.f : m_i, pf);
        pv(u & 1, pf);
        landed();
        __syncthreads();
      }
    }
  }

  // ---- epilogue
  const float l_tot = l_i + __shfl_xor(l_i, 32, 64);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  if (q_row < S) {
    T* orow = static_cast<T*>(a.o) + b * a.osb + hq * a.osh + (int64_t)(start + q_row) * a.oss;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int d0 = dt * 32 + 8 * rq + 4 * g;
        if (d0 >= a.dr) continue;
        const uint32_t lo = (uint32_t)__builtin_bit_cast(uint16_t, from_f32<T>(acc[dt][4 * rq] * inv)) |
                            ((uint32_t)__builtin_bit_cast(uint16_t, from_f32<T>(acc[dt][4 * rq + 1] * inv)) << 16);
        const uint32_t hi = (uint32_t)__builtin_bit_cast(uint16_t, from_f32<T>(acc[dt][4 * rq + 2] * inv)) |
                            ((uint32_t)__builtin_bit_cast(uint16_t, from_f32<T>(acc[dt][4 * rq + 3] * inv)) << 16);
        *reinterpret_cast<uint2*>(orow + d0) = make_uint2(lo, hi);
      }
    if (a.lse != nullptr && g == 0)
      a.lse[b * a.lse_bs + hq * a.lse_hs + start + q_row] = (m_i + log2f(l_tot)) * 0.69314718055994530942f;
  }
}

template <typename T, int D, int KS>
int launch_ks(const AttnArgs& a, bool causal, hipStream_t s) {
  const int64_t blocks = (int64_t)a.m_tiles * a.B * a.Hq / a.gp;
  if (causal)
    hipLaunchKernelGGL((attn_fwd_kernel<T, D, true, KS>), dim3(blocks), dim3(NT), 0, s, a);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<T, D, false, KS>), dim3(blocks), dim3(NT), 0, s, a);
  return launched("pk_attn_fwd");
}

// head_dim 8-16, 40-48 and 72-80 (Popcorn's 16, 48 and 80) leave the last 16
// dims of the 32-, 64- and 96-dim rows empty: their score step is skipped
template <typename T, int D>
int launch(const AttnArgs& a, bool causal, hipStream_t s) {
  if constexpr (D <= 96)
    if ((a.dr + 15) / 16 < D / 16) return launch_ks<T, D, D / 16 - 1>(a, causal, s);
  return launch_ks<T, D, D / 16>(a, causal, s);
}

}  // namespace
}  // namespace pk

namespace pk {
namespace {

// Checks shared by the dense and the packed entry point, then the launch.
// strides: q, k, v, o (batch, token, head) in elements; `seq` is the longest
// sequence, `batch` the number of sequences.
#include "attn_fwd_f32.h"

int attn_launch(const char* who, AttnArgs a, const int64_t* strides, int64_t batch, int64_t seq, int64_t q_heads,
                int64_t kv_heads, int64_t head_dim, float softmax_scale, int causal, int dtype, void* stream) {
  if (batch < 0 || seq < 0 || q_heads < 0 || kv_heads < 0 || head_dim < 0)
    return fail(PK_ERR_INVALID, "%s: negative size", who);
  if (batch == 0 || seq == 0 || q_heads == 0) return PK_OK;
  if (!a.q || !a.k || !a.v || !a.o || !strides) return fail(PK_ERR_INVALID, "%s: null pointer", who);
  if (kv_heads == 0 || q_heads % kv_heads != 0)
    return fail(PK_ERR_INVALID, "%s: q_heads=%lld is not a multiple of kv_heads=%lld", who, (long long)q_heads,
                (long long)kv_heads);
  if (dtype != PK_BF16 && dtype != PK_F16 && dtype != PK_F32)
    return fail(PK_ERR_UNSUPPORTED, "%s: dtype code %d (bf16/fp16/fp32 only)", who, dtype);
  const int max_dim = 256;
  if (head_dim <= 0 || head_dim > max_dim || head_dim % 8 != 0)
    return fail(PK_ERR_UNSUPPORTED, "%s: head_dim=%lld (a multiple of 8 up to %d for this dtype)", who,
                (long long)head_dim, max_dim);
  if (!isfinite(softmax_scale)) return fail(PK_ERR_INVALID, "%s: softmax_scale is not finite", who);
  if (seq > (1 << 30) || batch * q_heads > (1 << 20)) return fail(PK_ERR_UNSUPPORTED, "%s: shape too large", who);
  if (!aligned16(a.q) || !aligned16(a.k) || !aligned16(a.v) || !aligned16(a.o))
    return fail(PK_ERR_INVALID, "%s: q/k/v/o must be 16-byte aligned", who);
  const int unit = dtype == PK_F32 ? 4 : 8;  // elements per 16 bytes
  for (int i = 0; i < 12; ++i)
    if (strides[i] % unit != 0 || strides[i] < 0)
      return fail(PK_ERR_INVALID, "%s: stride %d = %lld is not a non-negative multiple of %d", who, i,
                  (long long)strides[i], unit);
  a.qsb = strides[0];
  a.qss = strides[1];
  a.qsh = strides[2];
  a.ksb = strides[3];
  a.kss = strides[4];
  a.ksh = strides[5];
  a.vsb = strides[6];
  a.vss = strides[7];
  a.vsh = strides[8];
  a.osb = strides[9];
  a.oss = strides[10];
  a.osh = strides[11];
  a.B = (int)batch;
  a.S = (int)seq;
  a.Hq = (int)q_heads;
  a.Hkv = (int)kv_heads;
  a.group = (int)(q_heads / kv_heads);
  a.gp = a.group % 4 == 0 ? 4 : (a.group % 2 == 0 ? 2 : 1);
  a.m_tiles = (int)((seq + 32 * (4 / a.gp) - 1) / (32 * (4 / a.gp)));
  // Buffer offsets are 32-bit: within one sequence the tile loads reach up to
  // two tiles past its last row (reading zeros there), and every such offset
  // must fit.
  // (the fp32 kernel addresses with 64-bit pointers)
  const int64_t reach = (seq + 3 * BN) * (strides[4] > strides[7] ? strides[4] : strides[7]) * 2 + head_dim * 2;
  if (dtype != PK_F32 && reach > INT32_MAX)
    return fail(PK_ERR_UNSUPPORTED, "%s: K/V rows span more than 2 GiB per head", who);
  a.c = fmaxf(fabsf(softmax_scale) * 1.4426950408889634f, 1e-30f);
  a.q_flip = softmax_scale < 0.f ? 0x80008000u : 0u;
  a.dr = (int)head_dim;
  a.dch = (int)(head_dim / 8);
  if ((int64_t)a.m_tiles * batch * q_heads / a.gp > INT32_MAX) return fail(PK_ERR_UNSUPPORTED, "%s: grid too large", who);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // rows are laid out at 32, 96 and 192 (16-bit types), 64, 128 or 256 dims, the chunks past
  // head_dim reading as zeros
  if (dtype == PK_F32)
    return head_dim <= 64 ? launch_f32<64>(a, causal, s)
                          : (head_dim <= 128 ? launch_f32<128>(a, causal, s) : launch_f32<256>(a, causal, s));
  if (dtype == PK_BF16)
    return head_dim <= 32    ? launch<bf16, 32>(a, causal, s)
           : head_dim <= 64  ? launch<bf16, 64>(a, causal, s)
           : head_dim <= 96  ? launch<bf16, 96>(a, causal, s)
           : head_dim <= 128 ? launch<bf16, 128>(a, causal, s)
           : head_dim <= 192 ? launch<bf16, 192>(a, causal, s)
                             : launch<bf16, 256>(a, causal, s);
  return head_dim <= 32    ? launch<f16, 32>(a, causal, s)
         : head_dim <= 64  ? launch<f16, 64>(a, causal, s)
         : head_dim <= 96  ? launch<f16, 96>(a, causal, s)
         : head_dim <= 128 ? launch<f16, 128>(a, causal, s)
         : head_dim <= 192 ? launch<f16, 192>(a, causal, s)
                           : launch<f16, 256>(a, causal, s);
}

}  // namespace
}  // namespace pk

extern "C" {

int pk_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse, const int64_t* strides,
                int64_t batch, int64_t seq, int64_t q_heads, int64_t kv_heads, int64_t head_dim, float softmax_scale,
                int causal, int dtype, void* stream) {
  using namespace pk;
  AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.lse = lse;
  a.cu = nullptr;
  a.lse_bs = q_heads * seq;  // [batch, q_heads, seq]
  a.lse_hs = seq;
  return attn_launch("pk_attn_fwd", a, strides, batch, seq, q_heads, kv_heads, head_dim, softmax_scale, causal, dtype,
                     stream);
}

int pk_attn_varlen_fwd(const void* q, const void* k, const void* v, void* o, float* lse, const int* cu_seqlens,
                       const int64_t* strides, int64_t num_seqs, int64_t total, int64_t max_seqlen, int64_t q_heads,
                       int64_t kv_heads, int64_t head_dim, float softmax_scale, int causal, int dtype, void* stream) {
  using namespace pk;
  const char* who = "pk_attn_varlen_fwd";
  if (num_seqs < 0 || total < 0 || max_seqlen < 0) return fail(PK_ERR_INVALID, "%s: negative size", who);
  if (num_seqs == 0 || total == 0 || max_seqlen == 0) return PK_OK;
  if (!cu_seqlens || !strides) return fail(PK_ERR_INVALID, "%s: null pointer", who);
  if (total > INT32_MAX || max_seqlen > total) return fail(PK_ERR_INVALID, "%s: max_seqlen %lld exceeds total %lld", who,
                                                        (long long)max_seqlen, (long long)total);
  // packed tensors have no batch dimension: strides are (token, head) of q, k, v, o
  const int64_t dense[12] = {0, strides[0], strides[1], 0, strides[2], strides[3],
                             0, strides[4], strides[5], 0, strides[6], strides[7]};
  AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.lse = lse;
  a.cu = cu_seqlens;
  a.total = (int)total;
  a.lse_bs = 0;  // [q_heads, total]
  a.lse_hs = total;
  return attn_launch(who, a, dense, num_seqs, max_seqlen, q_heads, kv_heads, head_dim, softmax_scale, causal, dtype,
                     stream);
}

}  // extern "C"
