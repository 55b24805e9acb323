// Attention forward (flash-style, grouped-query, optional causal mask) on
// gfx950 matrix cores.
//
// Block = 4 wavefronts x 32 query rows (BM = 128) of one (batch, q head);
// keys stream through LDS in tiles of BN = 64, double-buffered: K and V of
// tile t+1 are fetched into registers (buffer loads) while tile t is
// multiplied, then stored to the idle LDS buffer.
//
// Per tile each wave computes
//   S^T (32 keys x 32 queries)  = K_tile . Q^T   (v_mfma_f32_32x32x16, K from
//                                                 LDS, Q^T held in registers)
//   O^T (head_dim x 32 queries) += V^T . P^T
// Working on transposes puts one query per lane column: the MFMA result
// layout gives lane l the 16 entries of query l%32 in key rows
// 8*(r/4) + 4*(l/32) + r%4, so the online-softmax row max / sum are in-lane
// except for one exchange with lane l^32, and the rescale of O^T by that
// query's alpha is lane-uniform. P leaves the accumulator registers directly
// as the B operand of the second product: the key order inside each
// 16-key MFMA step is permuted identically in P^T and in the V^T fragments,
// which the contraction does not see.
//
// LDS layouts:
//   K [BN][D]: 16-byte chunk c of row r sits at chunk position c ^ (r % (D/8)),
//       so the 16-byte fragment reads of consecutive rows hit distinct banks.
//   V [BN][D + 16]: row-major. V^T fragments come from ds_read_b64_tr_b16:
//       within a 16-lane group, lane s reads keys base + s/4, dims
//       d0 + 4*(s%4) .. +3, and lane i receives dims d0 + i of keys
//       base .. base + 3 -- half of one MFMA A fragment; the padding puts the
//       four rows of one read on different banks.
//
// K and V are read through buffer resources based at the (batch, kv head):
// a tile is one scalar offset, and rows at or past S read as zero, so no load
// is predicated; such keys are masked like causal ones.
//
// Softmax runs in base 2: raw scores s are reduced to a row max first and
// exp2(s * c - m) is one FMA plus one exp with c = |scale| * log2(e) (a
// negative scale negates Q on load, which is exact). The running max m only
// moves when some query's candidate exceeds it by more than 8: exponents stay
// <= 8, and o = acc / l uses the same m in both, so the result is unchanged
// while most tiles skip the O rescale. The log-sum-exp output is converted
// back to natural log. Causal blocks only visit key tiles up to their last
// query and a wave skips the MFMAs of a tile wholly above its diagonal. Work
// order: longest causal rows first, and the q heads sharing a kv head land on
// the same XCD (dispatch is round-robin over the 8 XCDs), so their K/V tiles
// are shared through that XCD's L2.
#include <math.h>

#include "api.h"
#include "common.h"

namespace pk {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128;
constexpr int BN = 64;
constexpr int NT = 256;

template <typename T> struct Mma;
template <> struct Mma<bf16> {
  typedef bf16x8 frag;
  static __device__ __forceinline__ f32x16 run(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mma<f16> {
  typedef f16x8 frag;
  static __device__ __forceinline__ f32x16 run(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  int64_t qsb, qss, qsh, ksb, kss, ksh, vsb, vss, vsh, osb, oss, osh;
  int B, S, Hq, Hkv, group, m_tiles;
  int k_bytes, v_bytes;  // bytes from a (batch, kv head) base to the end of its last row
  float c;          // |scale| * log2(e), at least 1e-30
  uint32_t q_flip;  // 0x80008000 when scale < 0 (negates both halves of a packed pair), else 0
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s4;

__device__ __forceinline__ uint4 ld_buf(__amdgpu_buffer_rsrc_t r, int voffset, int soffset) {
  typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, voffset, soffset, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

template <typename T, int D, bool CAUSAL>
__global__ __attribute__((amdgpu_flat_work_group_size(NT, NT), amdgpu_waves_per_eu(2))) void attn_fwd_kernel(
    AttnArgs a) {
  using Frag = typename Mma<T>::frag;
  constexpr int KST = D;       // K row stride in LDS, elements (16-byte chunks XOR-swizzled by row)
  constexpr int VST = D + 16;  // V row stride in LDS, elements (row-major; read transposed)
  constexpr int KCH = D / 8;   // 16-byte chunks per K/V row
  constexpr int K_ROWS = NT / KCH;
  constexpr int K_PASSES = BN / K_ROWS;
  constexpr int V_RPT = BN * KCH / NT;  // consecutive V rows per thread
  __shared__ __attribute__((aligned(16))) T Ks[2][BN * KST];
  __shared__ __attribute__((aligned(16))) T Vs[2][BN * VST];

  // ---- work item: (batch, kv head, q tile) groups, q heads of a group adjacent on one XCD
  const int G = a.group;
  const int w = blockIdx.x;
  int gidx, hig;
  if (gridDim.x % (8 * G) == 0) {
    const int wp = w >> 3;
    gidx = (wp / G) * 8 + (w & 7);
    hig = wp % G;
  } else {
    gidx = w / G;
    hig = w % G;
  }
  const int per_tile = a.B * a.Hkv;
  const int m_tile = a.m_tiles - 1 - gidx / per_tile;
  const int rest = gidx % per_tile;
  const int b = rest / a.Hkv;
  const int hkv = rest % a.Hkv;
  const int hq = hkv * G + hig;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int r32 = lane & 31;
  const int g = lane >> 5;
  const int m0 = m_tile * BM;
  const int q_row = m0 + wave * 32 + r32;

  const T* qbase = static_cast<const T*>(a.q) + b * a.qsb + hq * a.qsh;
  const T* kbase = static_cast<const T*>(a.k) + b * a.ksb + hkv * a.ksh;
  const T* vbase = static_cast<const T*>(a.v) + b * a.vsb + hkv * a.vsh;
  // K/V of this (batch, kv head) through buffer resources: rows at or past S
  // read as zero (range-checked), and a tile's base is one scalar offset.
  const __amdgpu_buffer_rsrc_t krsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)kbase, (short)0, a.k_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)vbase, (short)0, a.v_bytes, 0x00020000);

  // ---- Q^T fragments: qf[kk] = Q[q_row][16kk + 8g .. +8], sign-flipped for a negative scale
  Frag qf[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
    uint4 raw = make_uint4(0, 0, 0, 0);
    if (q_row < a.S) raw = *reinterpret_cast<const uint4*>(qbase + (int64_t)q_row * a.qss + 16 * kk + 8 * g);
    raw.x ^= a.q_flip;
    raw.y ^= a.q_flip;
    raw.z ^= a.q_flip;
    raw.w ^= a.q_flip;
    qf[kk] = *reinterpret_cast<const Frag*>(&raw);
  }

  const int kv_end = CAUSAL ? (m0 + BM < a.S ? m0 + BM : a.S) : a.S;
  const int n_tiles = (kv_end + BN - 1) / BN;

  // ---- tile staging: K rows by 16-byte chunk, V rows V_RPT at a time
  const int kc = tid % KCH, kr = tid / KCH;
  const int vr = (tid / KCH) * V_RPT;
  const int koff = (kr * (int)a.kss + kc * 8) * (int)sizeof(T);  // byte offset of this lane's first K chunk
  const int voff = (vr * (int)a.vss + kc * 8) * (int)sizeof(T);
  uint4 kreg[K_PASSES], vreg[V_RPT];
  // this lane's element offsets of its K fragments (row r32, chunk 2kk + g, swizzled)
  int k_lane[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) k_lane[kk] = r32 * KST + (((2 * kk + g) ^ (r32 & (KCH - 1))) * 8);
  // this lane's element offset for the transposing V reads (see the PV loop)
  const int v_lane = (4 * g + ((lane & 15) >> 2)) * VST + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  f32x16 acc[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[dt][r] = 0.f;
  float m_i = -INFINITY;  // running max of s * c for query q_row
  float l_i = 0.f;        // this lane's half of the running denominator

#define PK_LOAD_TILE(t)                                                                                        \
  do {                                                                                                         \
    const int ktile_ = (t)*BN * (int)a.kss * (int)sizeof(T);                                                   \
    const int vtile_ = (t)*BN * (int)a.vss * (int)sizeof(T);                                                   \
    _Pragma("unroll") for (int p = 0; p < K_PASSES; ++p)                                                       \
      kreg[p] = ld_buf(krsrc, koff + p * K_ROWS * (int)a.kss * (int)sizeof(T), ktile_);                       \
    _Pragma("unroll") for (int i = 0; i < V_RPT; ++i)                                                          \
      vreg[i] = ld_buf(vrsrc, voff + i * (int)a.vss * (int)sizeof(T), vtile_);                                \
  } while (0)

#define PK_STORE_TILE(buf)                                                                                     \
  do {                                                                                                         \
    T* ks_ = Ks[buf];                                                                                          \
    _Pragma("unroll") for (int p = 0; p < K_PASSES; ++p)                                                       \
        *reinterpret_cast<uint4*>(ks_ + (kr + p * K_ROWS) * KST + (kc ^ ((kr + p * K_ROWS) & (KCH - 1))) * 8) = kreg[p]; \
    T* vs_ = Vs[buf];                                                                                          \
    _Pragma("unroll") for (int i = 0; i < V_RPT; ++i)                                                          \
        *reinterpret_cast<uint4*>(vs_ + (vr + i) * VST + kc * 8) = vreg[i];                                   \
  } while (0)

  PK_LOAD_TILE(0);
  PK_STORE_TILE(0);
  __syncthreads();

  const int wave_first = m0 + wave * 32;
  for (int t = 0; t < n_tiles; ++t) {
    const int buf = t & 1;
    // The last iteration re-reads its own tile into the idle buffer: the
    // staging registers never sit behind a branch, which keeps them in VGPRs.
    PK_LOAD_TILE(min(t + 1, n_tiles - 1));
    const int kv0 = t * BN;
    if (!(CAUSAL && kv0 > wave_first + 31)) {
      const T* ks = Ks[buf];
      f32x16 s[2];
#pragma unroll
      for (int st = 0; st < 2; ++st) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s[st][r] = 0.f;
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
          const Frag kf = *reinterpret_cast<const Frag*>(ks + st * 32 * KST + k_lane[kk]);
          s[st] = Mma<T>::run(kf, qf[kk], s[st]);
        }
      }
      // mask, row max of the raw scores
      const bool need_mask = (CAUSAL && kv0 + BN - 1 > wave_first) || kv0 + BN > a.S;
      if (need_mask) {
        // last visible key of this lane's query; rows past the end (clamped loads) are masked too
        const int lim = CAUSAL ? min(q_row, a.S - 1) : a.S - 1;
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kv0 + st * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
            s[st][r] = key <= lim ? s[st][r] : -INFINITY;
          }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[st][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      // The running max only moves when some query's max grew by more than
      // 2^8: exponents then stay <= 8 (p <= 256, exact in bf16 range) and the
      // final o = acc / l uses the same stale max in both, so the result is
      // unchanged while most tiles skip the O rescale entirely.
      const float m_cand = mx * a.c;
      if (!__all(m_cand <= m_i + 8.0f)) {
        const float m_new = fmaxf(m_i, m_cand);
        const float alpha = __builtin_amdgcn_exp2f(m_i - m_new);  // 0 when m_i = -inf
        l_i *= alpha;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[dt][r] *= alpha;
        m_i = m_new;
      }
      const float m_use = m_i == -INFINITY ? 0.f : m_i;
      float rs = 0.f;
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[st][r], a.c, -m_use));
          s[st][r] = p;
          rs += p;
        }
      l_i += rs;

      // O^T += V^T P^T, four 16-key steps
      // V^T fragments by transposing reads of row-major V: within each 16-lane
      // group, lane s reads keys (base + s/4), dims (d0 + 4*(s%4)) .. +3, and
      // lane i receives dims d0 + i of keys base .. base + 3.
      lds_s4* vt = (lds_s4*)(Vs[buf] + v_lane);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        Frag pf;
#pragma unroll
        for (int j = 0; j < 8; ++j) pf[j] = (T)s[c >> 1][8 * (c & 1) + j];
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(vt + ((16 * c) * VST + dt * 32) / 4);
          const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(vt + ((16 * c + 8) * VST + dt * 32) / 4);
          const s16x8 both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
          acc[dt] = Mma<T>::run(__builtin_bit_cast(Frag, both), pf, acc[dt]);
        }
      }
    }
    PK_STORE_TILE(buf ^ 1);
    __syncthreads();
  }
#undef PK_LOAD_TILE
#undef PK_STORE_TILE

  // ---- epilogue
  const float l_tot = l_i + __shfl_xor(l_i, 32, 64);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  if (q_row < a.S) {
    T* orow = static_cast<T*>(a.o) + b * a.osb + hq * a.osh + (int64_t)q_row * a.oss;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int d0 = dt * 32 + 8 * rq + 4 * g;
        const uint32_t lo = (uint32_t)__builtin_bit_cast(uint16_t, from_f32<T>(acc[dt][4 * rq] * inv)) |
                            ((uint32_t)__builtin_bit_cast(uint16_t, from_f32<T>(acc[dt][4 * rq + 1] * inv)) << 16);
        const uint32_t hi = (uint32_t)__builtin_bit_cast(uint16_t, from_f32<T>(acc[dt][4 * rq + 2] * inv)) |
                            ((uint32_t)__builtin_bit_cast(uint16_t, from_f32<T>(acc[dt][4 * rq + 3] * inv)) << 16);
        *reinterpret_cast<uint2*>(orow + d0) = make_uint2(lo, hi);
      }
    if (a.lse != nullptr && g == 0)
      a.lse[((int64_t)b * a.Hq + hq) * a.S + q_row] = (m_i + log2f(l_tot)) * 0.69314718055994530942f;
  }
}

template <typename T, int D>
int launch(const AttnArgs& a, bool causal, hipStream_t s) {
  const int64_t blocks = (int64_t)a.m_tiles * a.B * a.Hq;
  if (causal)
    hipLaunchKernelGGL((attn_fwd_kernel<T, D, true>), dim3(blocks), dim3(NT), 0, s, a);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<T, D, false>), dim3(blocks), dim3(NT), 0, s, a);
  return launched("pk_attn_fwd");
}

}  // namespace
}  // namespace pk

extern "C" {

int pk_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse, const int64_t* strides,
                int64_t batch, int64_t seq, int64_t q_heads, int64_t kv_heads, int64_t head_dim, float softmax_scale,
                int causal, int dtype, void* stream) {
  using namespace pk;
  if (batch < 0 || seq < 0 || q_heads < 0 || kv_heads < 0 || head_dim < 0)
    return fail(PK_ERR_INVALID, "pk_attn_fwd: negative size");
  if (batch == 0 || seq == 0 || q_heads == 0) return PK_OK;
  if (!q || !k || !v || !o || !strides) return fail(PK_ERR_INVALID, "pk_attn_fwd: null pointer");
  if (kv_heads == 0 || q_heads % kv_heads != 0)
    return fail(PK_ERR_INVALID, "pk_attn_fwd: q_heads=%lld is not a multiple of kv_heads=%lld", (long long)q_heads,
                (long long)kv_heads);
  if (dtype != PK_BF16 && dtype != PK_F16)
    return fail(PK_ERR_UNSUPPORTED, "pk_attn_fwd: dtype code %d (bf16/fp16 only)", dtype);
  if (head_dim != 64 && head_dim != 128)
    return fail(PK_ERR_UNSUPPORTED, "pk_attn_fwd: head_dim=%lld (64 or 128 only)", (long long)head_dim);
  if (!isfinite(softmax_scale)) return fail(PK_ERR_INVALID, "pk_attn_fwd: softmax_scale is not finite");
  if (seq > (1 << 30) || batch * q_heads > (1 << 20))
    return fail(PK_ERR_UNSUPPORTED, "pk_attn_fwd: shape too large");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return fail(PK_ERR_INVALID, "pk_attn_fwd: q/k/v/o must be 16-byte aligned");
  for (int i = 0; i < 12; ++i)
    if (strides[i] % 8 != 0 || strides[i] < 0)
      return fail(PK_ERR_INVALID, "pk_attn_fwd: stride %d = %lld is not a non-negative multiple of 8", i,
                  (long long)strides[i]);
  AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.lse = lse;
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
  a.m_tiles = (int)((seq + BM - 1) / BM);
  // buffer offsets are 32-bit: every row offset inside one (batch, kv head) must fit
  const int64_t k_span = ((seq - 1) * strides[4] + head_dim) * 2, v_span = ((seq - 1) * strides[7] + head_dim) * 2;
  if (k_span > INT32_MAX - 4096 || v_span > INT32_MAX - 4096)
    return fail(PK_ERR_UNSUPPORTED, "pk_attn_fwd: K/V rows span more than 2 GiB per head");
  a.k_bytes = (int)k_span;
  a.v_bytes = (int)v_span;
  a.c = fmaxf(fabsf(softmax_scale) * 1.4426950408889634f, 1e-30f);
  a.q_flip = softmax_scale < 0.f ? 0x80008000u : 0u;
  if ((int64_t)a.m_tiles * batch * q_heads > INT32_MAX) return fail(PK_ERR_UNSUPPORTED, "pk_attn_fwd: grid too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == PK_BF16) return head_dim == 64 ? launch<bf16, 64>(a, causal, s) : launch<bf16, 128>(a, causal, s);
  return head_dim == 64 ? launch<f16, 64>(a, causal, s) : launch<f16, 128>(a, causal, s);
}

}  // extern "C"
