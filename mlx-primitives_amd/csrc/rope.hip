// Rotary position embedding (RoPE) for gfx950, half-split ("NeoX") form.
//
// Restates mlx_primitives/kernels/rope.py:451-497 (rope) over the cos/sin
// cache of rope.py:223-255 (precompute_rope_cache): for a row at position p
// and i < D/2, with c = cos[p, i], s = sin[p, i]:
//   out[i]       = x[i] * c - x[i + D/2] * s
//   out[i + D/2] = x[i] * s + x[i + D/2] * c
// computed in float32 and rounded once to the element type. This is the
// rotation fused_rope_attention applies to Q and K before attention
// (kernels/fused_rope_attention.py:711-714). Memory bound: one thread per 8
// dimension pairs, 16-byte loads and stores for 16-bit types. The caches are
// contiguous (n_pos, D/2) arrays of any of the three element types.
#include "mpx_common.h"

#include <algorithm>

namespace mpx {

struct RopeParams {
  const void* x;
  void* out;
  const void* cos;
  const void* sin;
  int64_t x_sb, x_ss, x_sh;  // element strides of x (batch, seq, head)
  int64_t o_sb, o_ss, o_sh;  // element strides of out
  int B, S, H, D;
  int offset;   // position of sequence index 0
  int n_pos;    // rows of the cos / sin caches
  int64_t rows; // B * S * H
  const int32_t* pos;  // per-batch position of sequence index 0 (replaces offset), or null
  int32_t* err;        // with pos: err[0] = 1 for a row whose position is outside the cache
};

template <int DT>
struct Elem;
template <>
struct Elem<MPX_F32> {
  typedef float T;
};
template <>
struct Elem<MPX_F16> {
  typedef _Float16 T;
};
template <>
struct Elem<MPX_BF16> {
  typedef __bf16 T;
};

template <typename T>
__device__ __forceinline__ float to_f(T v) {
  return (float)v;
}
template <typename T>
__device__ __forceinline__ T from_f(float v) {
  return (T)v;
}

// Eight consecutive elements (one 16-byte load for 16-bit types, two for f32).
template <typename T>
struct V8 {
  T v[8];
};

template <typename T>
__device__ __forceinline__ V8<T> load8(const T* p) {
  V8<T> r;
  if constexpr (sizeof(T) == 2) {
    *(u32x4*)r.v = *(const u32x4*)p;
  } else {
    *(u32x4*)r.v = *(const u32x4*)p;
    *(u32x4*)(r.v + 4) = *(const u32x4*)(p + 4);
  }
  return r;
}

template <typename T>
__device__ __forceinline__ void store8(T* p, const V8<T>& r) {
  if constexpr (sizeof(T) == 2) {
    *(u32x4*)p = *(const u32x4*)r.v;
  } else {
    *(u32x4*)p = *(const u32x4*)r.v;
    *(u32x4*)(p + 4) = *(const u32x4*)(r.v + 4);
  }
}

template <int XT, int CT>
__global__ __launch_bounds__(256) void rope_kernel(RopeParams p) {
  typedef typename Elem<XT>::T T;
  typedef typename Elem<CT>::T C;
  const int half = p.D / 2, cpr = half / 8;  // 8-pair chunks per row
  const int64_t n = p.rows * cpr;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / cpr;
    const int d = (int)(i - row * cpr) * 8;
    const int h = (int)(row % p.H);
    const int64_t bs = row / p.H;
    const int s = (int)(bs % p.S);
    const int b = (int)(bs / p.S);
    const T* x = (const T*)p.x + b * p.x_sb + s * p.x_ss + h * p.x_sh;
    T* o = (T*)p.out + b * p.o_sb + s * p.o_ss + h * p.o_sh;
    int position = p.offset + s;
    if (p.pos) {
      position = p.pos[b] + s;
      if (position < 0 || position >= p.n_pos) {
        p.err[0] = 1;
        continue;
      }
    }
    const int64_t cbase = (int64_t)position * half + d;
    const V8<T> x1 = load8(x + d), x2 = load8(x + half + d);
    const V8<C> cs = load8((const C*)p.cos + cbase), sn = load8((const C*)p.sin + cbase);
    V8<T> y1, y2;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float r1, r2;
      rope_pair(to_f(x1.v[e]), to_f(x2.v[e]), to_f(cs.v[e]), to_f(sn.v[e]), r1, r2);
      y1.v[e] = from_f<T>(r1);
      y2.v[e] = from_f<T>(r2);
    }
    store8(o + d, y1);
    store8(o + half + d, y2);
  }
}

template <int XT>
hipError_t launch_rope(const RopeParams& p, int cache_dtype, int blocks, hipStream_t st) {
  switch (cache_dtype) {
    case MPX_F32:
      hipLaunchKernelGGL((rope_kernel<XT, MPX_F32>), dim3(blocks), dim3(256), 0, st, p);
      break;
    case MPX_F16:
      hipLaunchKernelGGL((rope_kernel<XT, MPX_F16>), dim3(blocks), dim3(256), 0, st, p);
      break;
    default:
      hipLaunchKernelGGL((rope_kernel<XT, MPX_BF16>), dim3(blocks), dim3(256), 0, st, p);
      break;
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// KV-cache append with K rotated on the way in (mpx_kv_append_rope): token t
// of sequence b, at position pos = start[b] + t, goes to page
// block_tables[b, pos / bs], slot pos % bs of the pools (num_blocks, bs, H, D)
// as in mpx_kv_append (kv_cache.hip), its K row rotated to pos. One thread per
// (token, head, 8-pair chunk): K dims [8j, 8j + 8) and [D/2 + 8j, D/2 + 8j + 8)
// rotated, the same V dims copied. A token that cannot be placed is skipped
// and reported in err: [0] negative position, [1] block index past the
// table, [2] page id outside the pool, [3] position at or past n_pos.
struct AppendRopeParams {
  const void* k;
  const void* v;
  void* kpool;
  void* vpool;
  const void* cos;
  const void* sin;
  const int32_t* bt;
  const int32_t* start;
  const int32_t* ntok;
  int32_t* err;
  int64_t k_sb, k_st, k_sh, v_sb, v_st, v_sh;  // source strides in elements
  int B, T, H, D, num_blocks, bs, max_blocks, n_pos;
};

template <int XT, int CT>
__global__ __launch_bounds__(256) void kv_append_rope_kernel(AppendRopeParams p) {
  typedef typename Elem<XT>::T T;
  typedef typename Elem<CT>::T C;
  const int half = p.D / 2, cpr = half / 8;  // 8-pair chunks per row
  const int64_t n = (int64_t)p.B * p.T * p.H * cpr;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / cpr;  // (b * T + t) * H + h
    const int d = (int)(i - row * cpr) * 8;
    const int h = (int)(row % p.H);
    const int64_t tok = row / p.H;
    const int t = (int)(tok % p.T);
    const int b = (int)(tok / p.T);
    if (t >= p.ntok[b]) continue;
    const int pos = p.start[b] + t;
    if (pos < 0) {
      p.err[0] = 1;
      continue;
    }
    const int bi = pos / p.bs;
    if (bi >= p.max_blocks) {
      p.err[1] = 1;
      continue;
    }
    const int page = p.bt[(int64_t)b * p.max_blocks + bi];
    if (page < 0 || page >= p.num_blocks) {
      p.err[2] = 1;
      continue;
    }
    if (pos >= p.n_pos) {
      p.err[3] = 1;
      continue;
    }
    const int64_t slot = ((int64_t)page * p.bs + (pos - bi * p.bs)) * p.H + h;
    T* kd = (T*)p.kpool + slot * p.D;
    T* vd = (T*)p.vpool + slot * p.D;
    const T* ks = (const T*)p.k + b * p.k_sb + t * p.k_st + h * p.k_sh;
    const T* vs = (const T*)p.v + b * p.v_sb + t * p.v_st + h * p.v_sh;
    const int64_t cbase = (int64_t)pos * half + d;
    const V8<T> x1 = load8(ks + d), x2 = load8(ks + half + d);
    const V8<C> cs = load8((const C*)p.cos + cbase), sn = load8((const C*)p.sin + cbase);
    V8<T> y1, y2;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float r1, r2;
      rope_pair(to_f(x1.v[e]), to_f(x2.v[e]), to_f(cs.v[e]), to_f(sn.v[e]), r1, r2);
      y1.v[e] = from_f<T>(r1);
      y2.v[e] = from_f<T>(r2);
    }
    store8(kd + d, y1);
    store8(kd + half + d, y2);
    store8(vd + d, load8(vs + d));
    store8(vd + half + d, load8(vs + half + d));
  }
}

template <int XT>
hipError_t launch_append_rope(const AppendRopeParams& p, int cache_dtype, int blocks,
                              hipStream_t st) {
  switch (cache_dtype) {
    case MPX_F32:
      hipLaunchKernelGGL((kv_append_rope_kernel<XT, MPX_F32>), dim3(blocks), dim3(256), 0, st, p);
      break;
    case MPX_F16:
      hipLaunchKernelGGL((kv_append_rope_kernel<XT, MPX_F16>), dim3(blocks), dim3(256), 0, st, p);
      break;
    default:
      hipLaunchKernelGGL((kv_append_rope_kernel<XT, MPX_BF16>), dim3(blocks), dim3(256), 0, st,
                         p);
      break;
  }
  return hipGetLastError();
}

// Shared argument checks of the entry points that rotate (x: (B, S, H, D)).
int check_rope_args(const char* fn, int dtype, int cache_dtype, int D, const void* cos_cache,
                    const void* sin_cache) {
  MPX_CHECK_ARG(dtype == MPX_F32 || dtype == MPX_F16 || dtype == MPX_BF16,
                "%s: unknown dtype code %d", fn, dtype);
  MPX_CHECK_ARG(cache_dtype == MPX_F32 || cache_dtype == MPX_F16 || cache_dtype == MPX_BF16,
                "%s: unknown cache dtype code %d", fn, cache_dtype);
  MPX_CHECK_ARG(D > 0 && D % 16 == 0, "%s: head_dim must be a positive multiple of 16", fn);
  MPX_CHECK_ARG(cos_cache && sin_cache, "%s: null cos / sin table", fn);
  MPX_CHECK_ARG(((uintptr_t)cos_cache & 15u) == 0 && ((uintptr_t)sin_cache & 15u) == 0,
                "%s: cos / sin tables must be 16-byte aligned", fn);
  return MPX_OK;
}

}  // namespace mpx

using namespace mpx;

extern "C" int mpx_rope(const void* x, void* out, const void* cos_cache, const void* sin_cache,
                        const int64_t* x_strides, const int64_t* out_strides, int B, int S, int H,
                        int D, int offset, int n_pos, int dtype, int cache_dtype, void* stream) {
  clear_error();
  MPX_CHECK_ARG(dtype == MPX_F32 || dtype == MPX_F16 || dtype == MPX_BF16,
                "mpx_rope: unknown dtype code %d", dtype);
  MPX_CHECK_ARG(cache_dtype == MPX_F32 || cache_dtype == MPX_F16 || cache_dtype == MPX_BF16,
                "mpx_rope: unknown cache dtype code %d", cache_dtype);
  MPX_CHECK_ARG(B >= 0 && S >= 0 && H >= 0 && n_pos >= 0, "mpx_rope: negative size");
  MPX_CHECK_ARG(D > 0 && D % 16 == 0, "mpx_rope: head_dim must be a positive multiple of 16");
  MPX_CHECK_ARG(offset >= 0, "mpx_rope: negative position offset");
  if ((long)B * S * H == 0) return MPX_OK;
  MPX_CHECK_ARG((long)offset + S <= n_pos,
                "mpx_rope: positions %d..%d exceed the cache's %d rows", offset, offset + S - 1,
                n_pos);
  MPX_CHECK_ARG(x && out && cos_cache && sin_cache && x_strides && out_strides,
                "mpx_rope: null pointer argument");
  const int es = dtype == MPX_F32 ? 4 : 2;
  MPX_CHECK_ARG(((uintptr_t)x & 15u) == 0 && ((uintptr_t)out & 15u) == 0 &&
                    ((uintptr_t)cos_cache & 15u) == 0 && ((uintptr_t)sin_cache & 15u) == 0,
                "mpx_rope: tensors must be 16-byte aligned");
  for (int i = 0; i < 3; ++i)
    MPX_CHECK_ARG(x_strides[i] >= 0 && (x_strides[i] * es) % 16 == 0 && out_strides[i] >= 0 &&
                      (out_strides[i] * es) % 16 == 0,
                  "mpx_rope: strides must be non-negative multiples of 16 bytes");
  RopeParams p;
  p.x = x; p.out = out; p.cos = cos_cache; p.sin = sin_cache;
  p.x_sb = x_strides[0]; p.x_ss = x_strides[1]; p.x_sh = x_strides[2];
  p.o_sb = out_strides[0]; p.o_ss = out_strides[1]; p.o_sh = out_strides[2];
  p.B = B; p.S = S; p.H = H; p.D = D; p.offset = offset; p.n_pos = n_pos;
  p.rows = (int64_t)B * S * H;
  p.pos = nullptr; p.err = nullptr;
  const int64_t n = p.rows * (D / 16);
  const int blocks = (int)std::min<int64_t>((n + 255) / 256, 65536);
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (dtype == MPX_F32)
    e = launch_rope<MPX_F32>(p, cache_dtype, blocks, st);
  else if (dtype == MPX_F16)
    e = launch_rope<MPX_F16>(p, cache_dtype, blocks, st);
  else
    e = launch_rope<MPX_BF16>(p, cache_dtype, blocks, st);
  MPX_CHECK_HIP(e);
  return MPX_OK;
}

extern "C" int mpx_rope_at(const void* x, void* out, const void* cos_cache, const void* sin_cache,
                           const int64_t* x_strides, const int64_t* out_strides, int B, int S,
                           int H, int D, const int32_t* positions, int n_pos, int dtype,
                           int cache_dtype, int32_t* errors, void* stream) {
  clear_error();
  int rc = check_rope_args("mpx_rope_at", dtype, cache_dtype, D, cos_cache, sin_cache);
  if (rc != MPX_OK) return rc;
  MPX_CHECK_ARG(B >= 0 && S >= 0 && H >= 0 && n_pos >= 0, "mpx_rope_at: negative size");
  if ((long)B * S * H == 0) return MPX_OK;
  MPX_CHECK_ARG(x && out && x_strides && out_strides && positions && errors,
                "mpx_rope_at: null pointer argument");
  const int es = dtype == MPX_F32 ? 4 : 2;
  MPX_CHECK_ARG(((uintptr_t)x & 15u) == 0 && ((uintptr_t)out & 15u) == 0,
                "mpx_rope_at: tensors must be 16-byte aligned");
  for (int i = 0; i < 3; ++i)
    MPX_CHECK_ARG(x_strides[i] >= 0 && (x_strides[i] * es) % 16 == 0 && out_strides[i] >= 0 &&
                      (out_strides[i] * es) % 16 == 0,
                  "mpx_rope_at: strides must be non-negative multiples of 16 bytes");
  RopeParams p;
  p.x = x; p.out = out; p.cos = cos_cache; p.sin = sin_cache;
  p.x_sb = x_strides[0]; p.x_ss = x_strides[1]; p.x_sh = x_strides[2];
  p.o_sb = out_strides[0]; p.o_ss = out_strides[1]; p.o_sh = out_strides[2];
  p.B = B; p.S = S; p.H = H; p.D = D; p.offset = 0; p.n_pos = n_pos;
  p.rows = (int64_t)B * S * H;
  p.pos = positions; p.err = errors;
  const int64_t n = p.rows * (D / 16);
  const int blocks = (int)std::min<int64_t>((n + 255) / 256, 65536);
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (dtype == MPX_F32)
    e = launch_rope<MPX_F32>(p, cache_dtype, blocks, st);
  else if (dtype == MPX_F16)
    e = launch_rope<MPX_F16>(p, cache_dtype, blocks, st);
  else
    e = launch_rope<MPX_BF16>(p, cache_dtype, blocks, st);
  MPX_CHECK_HIP(e);
  return MPX_OK;
}

extern "C" int mpx_kv_append_rope(const void* k, const void* v, void* k_pool, void* v_pool,
                                  const int32_t* block_tables, const int32_t* start_pos,
                                  const int32_t* n_tokens, const int64_t* k_strides,
                                  const int64_t* v_strides, int B, int T, int H, int D,
                                  int num_blocks, int block_size, int max_blocks, int dtype,
                                  const void* cos_cache, const void* sin_cache, int n_pos,
                                  int cache_dtype, int32_t* errors, void* stream) {
  clear_error();
  int rc = check_rope_args("mpx_kv_append_rope", dtype, cache_dtype, D, cos_cache, sin_cache);
  if (rc != MPX_OK) return rc;
  MPX_CHECK_ARG(B >= 0 && T >= 0 && H >= 0 && num_blocks >= 0 && max_blocks >= 0 && n_pos >= 0,
                "mpx_kv_append_rope: negative size");
  MPX_CHECK_ARG(block_size > 0, "mpx_kv_append_rope: block_size must be positive");
  if ((long)B * T * H == 0) return MPX_OK;
  MPX_CHECK_ARG(k && v && k_pool && v_pool && block_tables && start_pos && n_tokens &&
                    k_strides && v_strides && errors,
                "mpx_kv_append_rope: null pointer argument");
  const int es = dtype == MPX_F32 ? 4 : 2;
  MPX_CHECK_ARG(((uintptr_t)k & 15u) == 0 && ((uintptr_t)v & 15u) == 0 &&
                    ((uintptr_t)k_pool & 15u) == 0 && ((uintptr_t)v_pool & 15u) == 0,
                "mpx_kv_append_rope: tensors must be 16-byte aligned");
  for (int i = 0; i < 3; ++i)
    MPX_CHECK_ARG(k_strides[i] >= 0 && (k_strides[i] * es) % 16 == 0 && v_strides[i] >= 0 &&
                      (v_strides[i] * es) % 16 == 0,
                  "mpx_kv_append_rope: strides must be non-negative multiples of 16 bytes");
  AppendRopeParams p;
  p.k = k; p.v = v; p.kpool = k_pool; p.vpool = v_pool; p.cos = cos_cache; p.sin = sin_cache;
  p.bt = block_tables; p.start = start_pos; p.ntok = n_tokens; p.err = errors;
  p.k_sb = k_strides[0]; p.k_st = k_strides[1]; p.k_sh = k_strides[2];
  p.v_sb = v_strides[0]; p.v_st = v_strides[1]; p.v_sh = v_strides[2];
  p.B = B; p.T = T; p.H = H; p.D = D; p.num_blocks = num_blocks; p.bs = block_size;
  p.max_blocks = max_blocks; p.n_pos = n_pos;
  const int64_t n = (int64_t)B * T * H * (D / 16);
  const int blocks = (int)std::min<int64_t>((n + 255) / 256, 65536);
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (dtype == MPX_F32)
    e = launch_append_rope<MPX_F32>(p, cache_dtype, blocks, st);
  else if (dtype == MPX_F16)
    e = launch_append_rope<MPX_F16>(p, cache_dtype, blocks, st);
  else
    e = launch_append_rope<MPX_BF16>(p, cache_dtype, blocks, st);
  MPX_CHECK_HIP(e);
  return MPX_OK;
}

