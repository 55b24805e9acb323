// Attention forward (flash-style, grouped-query, optional causal mask) on
// gfx950 matrix cores.
//
// Block = 4 wavefronts x 32 query rows (BM = 128) of one (batch, q head);
// keys stream through LDS in tiles of BN = 64, double-buffered: the global
// loads of tile t+1 are in flight while tile t is multiplied.
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
// 16-key MFMA step is permuted identically in P^T and in the V^T fragments
// read from LDS, which the contraction does not see. V is transposed once per
// tile on its way into LDS (V^T rows padded to 68 keys -> 34-dword stride,
// conflict-free 8-byte reads for 32 lanes); K rows are padded to D + 8.
//
// Softmax runs in base 2 on s * scale * log2(e); the log-sum-exp output is
// converted back to natural log. Causal blocks only visit key tiles up to
// their last query and a wave skips the MFMAs of a tile wholly above its
// diagonal. Work order: longest causal rows first, and the q heads sharing a
// kv head land on the same XCD (dispatch is round-robin over the 8 XCDs), so
// their K/V tiles are shared through that XCD's L2.
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
  float scale_log2;
};

template <typename T, int D, bool CAUSAL>
__global__ __attribute__((amdgpu_flat_work_group_size(NT, NT), amdgpu_waves_per_eu(2))) void attn_fwd_kernel(
    AttnArgs a) {
  using Frag = typename Mma<T>::frag;
  constexpr int KST = D + 8;   // K row stride in LDS, elements
  constexpr int VST = BN + 4;  // V^T row stride in LDS, elements
  constexpr int KCH = D / 8;   // 16-byte chunks per K/V row
  constexpr int K_ROWS = NT / KCH;
  constexpr int K_PASSES = BN / K_ROWS;
  constexpr int V_RPT = BN * KCH / NT;  // consecutive V rows per thread
  static_assert(V_RPT == 2 || V_RPT == 4, "V transpose packs 2 or 4 keys");
  __shared__ __attribute__((aligned(16))) T Ks[2][BN * KST];
  __shared__ __attribute__((aligned(16))) T Vt[2][D * VST];

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

  // ---- Q^T fragments: qf[kk] = Q[q_row][16kk + 8g .. +8]
  Frag qf[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
    if (q_row < a.S) {
      qf[kk] = *reinterpret_cast<const Frag*>(qbase + (int64_t)q_row * a.qss + 16 * kk + 8 * g);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) qf[kk][j] = (T)0.f;
    }
  }

  const int kv_end = CAUSAL ? (m0 + BM < a.S ? m0 + BM : a.S) : a.S;
  const int n_tiles = (kv_end + BN - 1) / BN;

  // ---- tile staging
  const int kc = tid % KCH, kr = tid / KCH;
  const int vr = (tid / KCH) * V_RPT;
  uint4 kreg[K_PASSES], vreg[V_RPT];
  const uint4 zero4 = make_uint4(0, 0, 0, 0);
  auto load_tile = [&](int t) {
    const int kv0 = t * BN;
#pragma unroll
    for (int p = 0; p < K_PASSES; ++p) {
      const int row = kv0 + kr + p * K_ROWS;
      kreg[p] = row < a.S ? *reinterpret_cast<const uint4*>(kbase + (int64_t)row * a.kss + kc * 8) : zero4;
    }
#pragma unroll
    for (int i = 0; i < V_RPT; ++i) {
      const int row = kv0 + vr + i;
      vreg[i] = row < a.S ? *reinterpret_cast<const uint4*>(vbase + (int64_t)row * a.vss + kc * 8) : zero4;
    }
  };
  auto store_tile = [&](int buf) {
    T* ks = Ks[buf];
#pragma unroll
    for (int p = 0; p < K_PASSES; ++p) *reinterpret_cast<uint4*>(ks + (kr + p * K_ROWS) * KST + kc * 8) = kreg[p];
    T* vt = Vt[buf];
    const unsigned short* h[V_RPT];
#pragma unroll
    for (int i = 0; i < V_RPT; ++i) h[i] = reinterpret_cast<const unsigned short*>(&vreg[i]);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      T* dst = vt + (kc * 8 + e) * VST + vr;
      if constexpr (V_RPT == 4) {
        *reinterpret_cast<uint2*>(dst) =
            make_uint2((unsigned)h[0][e] | ((unsigned)h[1][e] << 16), (unsigned)h[2][e] | ((unsigned)h[3][e] << 16));
      } else {
        *reinterpret_cast<unsigned*>(dst) = (unsigned)h[0][e] | ((unsigned)h[1][e] << 16);
      }
    }
  };

  float m_i = -INFINITY;  // running max of s*scale*log2e for query q_row
  float l_i = 0.f;        // this lane's half of the running denominator
  f32x16 acc[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[dt][r] = 0.f;

  load_tile(0);
  store_tile(0);
  __syncthreads();

  const int wave_first = m0 + wave * 32;
  for (int t = 0; t < n_tiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < n_tiles) load_tile(t + 1);
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
          const Frag kf = *reinterpret_cast<const Frag*>(ks + (st * 32 + r32) * KST + 16 * kk + 8 * g);
          s[st] = Mma<T>::run(kf, qf[kk], s[st]);
        }
      }
      // scale, mask, row max
      const bool need_mask = (CAUSAL && kv0 + BN - 1 > wave_first) || kv0 + BN > a.S;
      float mx = -INFINITY;
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float x = s[st][r] * a.scale_log2;
          if (need_mask) {
            const int key = kv0 + st * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
            if ((CAUSAL && key > q_row) || key >= a.S) x = -INFINITY;
          }
          s[st][r] = x;
          mx = fmaxf(mx, x);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_i, mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_i - m_use);
      float rs = 0.f;
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = __builtin_amdgcn_exp2f(s[st][r] - m_use);
          s[st][r] = p;
          rs += p;
        }
      l_i = l_i * alpha + rs;
      m_i = m_new;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[dt][r] *= alpha;

      // O^T += V^T P^T, four 16-key steps
      const T* vt = Vt[buf];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        Frag pf;
#pragma unroll
        for (int j = 0; j < 8; ++j) pf[j] = (T)s[c >> 1][8 * (c & 1) + j];
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
          const T* row = vt + (dt * 32 + r32) * VST + 16 * c + 4 * g;
          const uint2 lo = *reinterpret_cast<const uint2*>(row);
          const uint2 hi = *reinterpret_cast<const uint2*>(row + 8);
          Frag vf;
          uint4 packed = make_uint4(lo.x, lo.y, hi.x, hi.y);
          vf = *reinterpret_cast<const Frag*>(&packed);
          acc[dt] = Mma<T>::run(vf, pf, acc[dt]);
        }
      }
    }
    if (t + 1 < n_tiles) store_tile(buf ^ 1);
    __syncthreads();
  }

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
        T o4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o4[i] = from_f32<T>(acc[dt][4 * rq + i] * inv);
        *reinterpret_cast<uint2*>(orow + d0) = *reinterpret_cast<const uint2*>(o4);
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
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  if ((int64_t)a.m_tiles * batch * q_heads > INT32_MAX) return fail(PK_ERR_UNSUPPORTED, "pk_attn_fwd: grid too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == PK_BF16) return head_dim == 64 ? launch<bf16, 64>(a, causal, s) : launch<bf16, 128>(a, causal, s);
  return head_dim == 64 ? launch<f16, 64>(a, causal, s) : launch<f16, 128>(a, causal, s);
}

}  // extern "C"
