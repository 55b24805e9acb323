// Rotary position embedding over x [batch, seq, heads, head_dim].
//
// Work item = (batch, seq, head, chunk): a chunk is VEC pairs for NeoX halves
// (two 16-byte loads, at j and j + half) or VEC/2 pairs for GPT-J interleaved
// pairs (one 16-byte load), plus passthrough chunks that copy channels
// 2*half.. when y is not x. A block covers whole (batch, seq) positions when
// heads*chunks <= 256, so one block reads each cos/sin row once from L2 and
// reuses it across all heads. Arithmetic is fp32 without contraction and one
// final rounding, which is the reference's op sequence (products rounded, then
// the sum).
#include "api.h"
#include "common.h"

namespace pk {
namespace {

constexpr int kThreads = 256;

struct RotArgs {
  int64_t xsb, xss, xsh, ysb, yss, ysh;  // strides, elements
  int seq, heads, head_dim, half;
  int chunks;      // rotation chunks per head
  int tail;        // passthrough chunks per head (0 when in place)
  int per_head;    // chunks + tail
  int per_pos;     // heads * per_head
  int pos_per_block;
  int64_t positions;  // batch * seq
};

template <typename C, int N> __device__ __forceinline__ void load_table(const C* p, float (&out)[N]) {
#pragma unroll
  for (int j = 0; j < N; ++j) out[j] = to_f32(p[j]);
}

template <int N> __device__ __forceinline__ void load_table(const float* p, float (&out)[N]) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int j = 0; j < N; j += 4) {
      const float4 v = *reinterpret_cast<const float4*>(p + j);
      out[j] = v.x;
      out[j + 1] = v.y;
      out[j + 2] = v.z;
      out[j + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) out[j] = p[j];
  }
}

// Loads/stores VEC consecutive elements of T: one 16-byte non-temporal access
// when VEC fills it (x and y are touched once; the cos/sin rows, reused by
// every head of a position, stay cacheable), element accesses otherwise.
template <typename T, int VEC> struct Chunk {
  T v[VEC];
  __device__ __forceinline__ void load(const T* p) {
    if constexpr (VEC * sizeof(T) == 16) {
      *reinterpret_cast<u32x4*>(v) = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) v[j] = p[j];
    }
  }
  __device__ __forceinline__ void store(T* p) const {
    if constexpr (VEC * sizeof(T) == 16) {
      __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(v), reinterpret_cast<u32x4*>(p));
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) p[j] = v[j];
    }
  }
};

template <typename T, typename C, int VEC, int TAILV, bool INTERLEAVED, bool CONJ>
__global__ __launch_bounds__(kThreads) void rotary_kernel(const T* __restrict__ x, const C* __restrict__ cosp,
                                                          const C* __restrict__ sinp, T* y, RotArgs a) {
  // Work inside one block: pos_per_block positions x per_pos items, strided
  // by the block size when one position has more items than threads.
  const int64_t pos0 = (int64_t)blockIdx.x * a.pos_per_block;
  const int items = a.pos_per_block * a.per_pos;
  for (int it = threadIdx.x; it < items; it += kThreads) {
    const int pl = it / a.per_pos;
    const int rem = it - pl * a.per_pos;
    const int64_t pos = pos0 + pl;
    if (pos >= a.positions) break;
    const int h = rem / a.per_head;
    const int c = rem - h * a.per_head;
    const int64_t b = pos / a.seq;
    const int s = (int)(pos - b * a.seq);
    const T* xr = x + b * a.xsb + s * a.xss + h * a.xsh;
    T* yr = y + b * a.ysb + s * a.yss + h * a.ysh;

    if (c >= a.chunks) {  // passthrough channels
      const int off = 2 * a.half + (c - a.chunks) * TAILV;
      Chunk<T, TAILV> t;
      t.load(xr + off);
      t.store(yr + off);
      continue;
    }
    if constexpr (!INTERLEAVED) {
      const int j = c * VEC;
      Chunk<T, VEC> x1, x2;
      x1.load(xr + j);
      x2.load(xr + a.half + j);
      float cs[VEC], sn[VEC];
      load_table(cosp + (int64_t)s * a.half + j, cs);
      load_table(sinp + (int64_t)s * a.half + j, sn);
      Chunk<T, VEC> y1, y2;
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        const float u = to_f32(x1.v[k]), v = to_f32(x2.v[k]);
        const float sk = CONJ ? -sn[k] : sn[k];
        y1.v[k] = from_f32<T>(u * cs[k] - v * sk);
        y2.v[k] = from_f32<T>(u * sk + v * cs[k]);
      }
      y1.store(yr + j);
      y2.store(yr + a.half + j);
    } else {
      constexpr int PAIRS = VEC / 2;
      const int e = c * VEC;  // first element; pair index e / 2
      Chunk<T, VEC> xv;
      xv.load(xr + e);
      float cs[PAIRS], sn[PAIRS];
      load_table(cosp + (int64_t)s * a.half + e / 2, cs);
      load_table(sinp + (int64_t)s * a.half + e / 2, sn);
      Chunk<T, VEC> yv;
#pragma unroll
      for (int k = 0; k < PAIRS; ++k) {
        const float u = to_f32(xv.v[2 * k]), v = to_f32(xv.v[2 * k + 1]);
        const float sk = CONJ ? -sn[k] : sn[k];
        yv.v[2 * k] = from_f32<T>(u * cs[k] - v * sk);
        yv.v[2 * k + 1] = from_f32<T>(u * sk + v * cs[k]);
      }
      yv.store(yr + e);
    }
  }
}

template <typename T, typename C, int VEC, int TAILV, bool IL, bool CONJ>
void launch(const void* x, const void* cs, const void* sn, void* y, const RotArgs& a, hipStream_t s) {
  const int64_t blocks = (a.positions + a.pos_per_block - 1) / a.pos_per_block;
  hipLaunchKernelGGL((rotary_kernel<T, C, VEC, TAILV, IL, CONJ>), dim3(blocks), dim3(kThreads), 0, s,
                     static_cast<const T*>(x), static_cast<const C*>(cs), static_cast<const C*>(sn),
                     static_cast<T*>(y), a);
}

template <typename T, typename C, int VEC, int TAILV, bool IL>
void pick_conj(int conj, const void* x, const void* cs, const void* sn, void* y, const RotArgs& a, hipStream_t s) {
  if (conj) launch<T, C, VEC, TAILV, IL, true>(x, cs, sn, y, a, s);
  else launch<T, C, VEC, TAILV, IL, false>(x, cs, sn, y, a, s);
}

// vec: every chunk is one 16-byte pack (V elements). Otherwise NeoX chunks are
// single pairs and GPT-J chunks single (2-element) pairs; passthrough moves
// one element at a time.
template <typename T, typename C>
int run(bool vec, int il, int conj, const void* x, const void* cs, const void* sn, void* y, RotArgs a,
        hipStream_t s) {
  constexpr int V = 16 / sizeof(T);
  const int unit = vec ? V : (il ? 2 : 1);
  const int tail_unit = vec ? V : 1;
  a.chunks = il ? (2 * a.half) / unit : a.half / unit;
  a.tail = x == y ? 0 : (a.head_dim - 2 * a.half) / tail_unit;
  a.per_head = a.chunks + a.tail;
  a.per_pos = a.heads * a.per_head;
  if (a.per_pos == 0) return PK_OK;
  a.pos_per_block = a.per_pos >= kThreads ? 1 : kThreads / a.per_pos;
  if (vec) {
    if (il) pick_conj<T, C, V, V, true>(conj, x, cs, sn, y, a, s);
    else pick_conj<T, C, V, V, false>(conj, x, cs, sn, y, a, s);
  } else {
    if (il) pick_conj<T, C, 2, 1, true>(conj, x, cs, sn, y, a, s);
    else pick_conj<T, C, 1, 1, false>(conj, x, cs, sn, y, a, s);
  }
  return launched("pk_rotary");
}

}  // namespace
}  // namespace pk

extern "C" {

int pk_rotary(const void* x, const void* cos, const void* sin, void* y, const int64_t* strides, int64_t batch,
              int64_t seq, int64_t heads, int64_t head_dim, int64_t half, int x_dtype, int cs_dtype, int interleaved,
              int conjugate, void* stream) {
  using namespace pk;
  if (batch < 0 || seq < 0 || heads < 0 || head_dim < 0 || half < 0)
    return fail(PK_ERR_INVALID, "pk_rotary: negative size");
  if (2 * half > head_dim)
    return fail(PK_ERR_INVALID, "pk_rotary: half=%lld exceeds head_dim/2 (head_dim=%lld)", (long long)half,
                (long long)head_dim);
  if (batch == 0 || seq == 0 || heads == 0 || head_dim == 0) return PK_OK;
  if (!x || !y || !strides || (half > 0 && (!cos || !sin))) return fail(PK_ERR_INVALID, "pk_rotary: null pointer");
  if (!known_dtype(x_dtype) || !known_dtype(cs_dtype))
    return fail(PK_ERR_UNSUPPORTED, "pk_rotary: dtype codes %d/%d", x_dtype, cs_dtype);
  if (seq > INT32_MAX || heads > INT32_MAX || head_dim > INT32_MAX || batch * seq > ((int64_t)1 << 40))
    return fail(PK_ERR_UNSUPPORTED, "pk_rotary: shape too large");
  if (x == y) {
    for (int i = 0; i < 3; ++i)
      if (strides[i] != strides[3 + i]) return fail(PK_ERR_INVALID, "pk_rotary: in place with differing strides");
  }
  RotArgs a{};
  a.xsb = strides[0];
  a.xss = strides[1];
  a.xsh = strides[2];
  a.ysb = strides[3];
  a.yss = strides[4];
  a.ysh = strides[5];
  a.seq = (int)seq;
  a.heads = (int)heads;
  a.head_dim = (int)head_dim;
  a.half = (int)half;
  a.positions = batch * seq;

  // 16-byte chunks need every chunk start aligned: base pointers, strides,
  // the rotated width and the passthrough width in whole packs. fp32 tables
  // are read as float4 when a chunk spans 4 or more pairs.
  const int V = 16 / elem_size(x_dtype);
  bool vec = aligned16(x) && aligned16(y);
  for (int i = 0; i < 6; ++i) vec = vec && strides[i] % V == 0;
  vec = vec && (interleaved ? 2 * half : half) % V == 0 && (head_dim - 2 * half) % V == 0;
  if (vec && half > 0 && cs_dtype == PK_F32) vec = half % 4 == 0 && aligned16(cos) && aligned16(sin);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (x_dtype) {
    case PK_F32:
      switch (cs_dtype) {
        case PK_F32: return run<float, float>(vec, interleaved, conjugate, x, cos, sin, y, a, s);
        case PK_BF16: return run<float, bf16>(vec, interleaved, conjugate, x, cos, sin, y, a, s);
        default: return run<float, f16>(vec, interleaved, conjugate, x, cos, sin, y, a, s);
      }
    case PK_BF16:
      switch (cs_dtype) {
        case PK_F32: return run<bf16, float>(vec, interleaved, conjugate, x, cos, sin, y, a, s);
        case PK_BF16: return run<bf16, bf16>(vec, interleaved, conjugate, x, cos, sin, y, a, s);
        default: return run<bf16, f16>(vec, interleaved, conjugate, x, cos, sin, y, a, s);
      }
    default:
      switch (cs_dtype) {
        case PK_F32: return run<f16, float>(vec, interleaved, conjugate, x, cos, sin, y, a, s);
        case PK_BF16: return run<f16, bf16>(vec, interleaved, conjugate, x, cos, sin, y, a, s);
        default: return run<f16, f16>(vec, interleaved, conjugate, x, cos, sin, y, a, s);
      }
  }
}

}  // extern "C"
