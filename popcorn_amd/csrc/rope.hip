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

template <typename T, int VEC> struct Pack {
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

template <typename T, typename C, int VEC, int U, bool TRANSPOSE>
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
      Pack<T, VEC> x1[U], x2[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int g = hh + u;
        if (g >= h_end) break;
        const int t = g >= a.heads[0];
        const int h = t ? g - a.heads[0] : g;
        const T* xr = static_cast<const T*>(a.x[t]) + xo[t] + h * a.xs[t][1];
        x1[u].load(xr);
        x2[u].load(xr + a.half);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int g = hh + u;
        if (g >= h_end) break;
        const int t = g >= a.heads[0];
        const int h = t ? g - a.heads[0] : g;
        Pack<T, VEC> y1, y2;
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
          const float p = to_f32(x1[u].v[k]), q = to_f32(x2[u].v[k]);
          if constexpr (!TRANSPOSE) {
            y1.v[k] = from_f32<T>(p * c1[k] - q * s1[k]);
            y2.v[k] = from_f32<T>(q * c2[k] + p * s2[k]);
          } else {
            y1.v[k] = from_f32<T>(p * c1[k] + q * s2[k]);
            y2.v[k] = from_f32<T>(q * c2[k] - p * s1[k]);
          }
        }
        T* yr = static_cast<T*>(a.y[t]) + yo[t] + h * a.ys[t][1];
        y1.store(yr);
        y2.store(yr + a.half);
      }
    }
  }
}

template <typename T, typename C, int VEC>
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
    hipLaunchKernelGGL((rope_kernel<T, C, VEC, U, true>), dim3((unsigned)blocks), dim3(kThreads), 0, s,
                       static_cast<const C*>(cs), static_cast<const C*>(sn), a);
  else
    hipLaunchKernelGGL((rope_kernel<T, C, VEC, U, false>), dim3((unsigned)blocks), dim3(kThreads), 0, s,
                       static_cast<const C*>(cs), static_cast<const C*>(sn), a);
  return launched("pk_rope");
}

template <typename T, typename C> int run(bool vec, const void* cs, const void* sn, const RopeArgs& a, int tr,
                                          hipStream_t s) {
  constexpr int V = 16 / sizeof(T);
  return vec ? launch<T, C, V>(cs, sn, a, tr, s) : launch<T, C, 1>(cs, sn, a, tr, s);
}

template <typename T> int run_cs(int cs_dtype, bool vec, const void* cs, const void* sn, const RopeArgs& a, int tr,
                                 hipStream_t s) {
  switch (cs_dtype) {
    case PK_F32: return run<T, float>(vec, cs, sn, a, tr, s);
    case PK_BF16: return run<T, bf16>(vec, cs, sn, a, tr, s);
    default: return run<T, f16>(vec, cs, sn, a, tr, s);
  }
}

}  // namespace
}  // namespace pk

extern "C" {

int pk_rope(const void* q, const void* k, const void* cos, const void* sin, void* yq, void* yk,
            const int64_t* strides, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq, int64_t head_dim,
            int64_t cos_batch, int x_dtype, int cs_dtype, int transpose, void* stream) {
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
  if (!known_dtype(x_dtype) || !known_dtype(cs_dtype))
    return fail(PK_ERR_UNSUPPORTED, "pk_rope: dtype codes %d/%d", x_dtype, cs_dtype);
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
  // 16-byte packs of x when every row start and both halves are 16-byte
  // aligned (half a multiple of V and strides multiples of V); a pack's table
  // entries are then 16-byte loads too whenever they fill whole 16 bytes,
  // which needs only the table bases aligned.
  const int64_t V = 16 / elem_size(x_dtype);
  bool vec = a.half % V == 0;
  const void* ptrs[] = {q, k, yq, yk};
  for (const void* p : ptrs) vec = vec && (p == nullptr || aligned16(p));
  for (int i = 0; i < 12; ++i) vec = vec && strides[i] % V == 0;
  if ((V * elem_size(cs_dtype)) % 16 == 0) vec = vec && aligned16(cos) && aligned16(sin);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (x_dtype) {
    case PK_F32: return run_cs<float>(cs_dtype, vec, cos, sin, a, transpose, s);
    case PK_BF16: return run_cs<bf16>(cs_dtype, vec, cos, sin, a, transpose, s);
    default: return run_cs<f16>(cs_dtype, vec, cos, sin, a, transpose, s);
  }
}

}  // extern "C"
