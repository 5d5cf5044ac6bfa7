// KV-cache append for gfx950: write new K/V token rows into their pages.
//
// The scatter of mlx_primitives/cache/kv_cache.py:219-264 (KVCache._store_kv)
// and cache/block_allocator.py:299-331 (BlockAllocator.set_block_data),
// batched over sequences: token t of sequence b goes to position
// start[b] + t, page block_tables[b, pos / bs], slot pos % bs of the pools
// (num_blocks, bs, H, D). Memory bound: one thread per 16-byte chunk of a
// token row, coalesced reads and writes.
//
// A token that cannot be placed is skipped and reported through the caller's
// int32[3] error words, each set to 1 with a plain store (no read-modify-write,
// so concurrent writers cannot lose a report): [0] a negative position (the
// reference raises ValueError, kv_cache.py:236-241), [1] a block index past the
// table (RuntimeError, kv_cache.py:250-254), [2] a page id outside the pool
// (ValueError from BlockAllocator._validate_block_id). Other tokens are written.
#include "mpx_common.h"

#include <algorithm>

namespace mpx {

#ifndef MPX_KV_NT
#define MPX_KV_NT 1
#endif

struct AppendParams {
  const unsigned char* k;
  const unsigned char* v;
  unsigned char* kpool;
  unsigned char* vpool;
  const int32_t* bt;
  const int32_t* start;
  const int32_t* ntok;
  int32_t* err;
  int64_t k_sb, k_st, k_sh, v_sb, v_st, v_sh;  // source strides in elements
  int B, T, H, cpr;                             // cpr: 16-byte chunks per head row
  int es;                                       // element bytes
  int num_blocks, bs, max_blocks;
};

// Grid: each workgroup handles 256 consecutive 16-byte chunks of one token
// row (b, t) (H * cpr chunks, split over nbr workgroups), so the row's
// position, page lookup and checks are per-workgroup scalar work and each
// thread only splits its chunk index into (head, chunk).
__global__ __launch_bounds__(256) void kv_append_kernel(AppendParams p, int nbr) {
  const int row_chunks = p.H * p.cpr;
  const int n_blk = p.B * p.T * nbr;  // < 2^31 (checked by the host)
  for (int blk = blockIdx.x; blk < n_blk; blk += gridDim.x) {
    const int row = blk / nbr;  // b * T + t
    const int rc = (blk - row * nbr) * 256 + (int)threadIdx.x;
    const int b = row / p.T;
    const int t = row - b * p.T;
    if (rc >= row_chunks || t >= p.ntok[b]) continue;
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
    const int h = rc / p.cpr;
    const int c = rc - h * p.cpr;
    const int64_t slot = ((int64_t)page * p.bs + (pos - bi * p.bs)) * p.H + h;
    const int64_t dst = (slot * p.cpr + c) * 16;
    const int64_t ks = ((int64_t)b * p.k_sb + (int64_t)t * p.k_st + (int64_t)h * p.k_sh) * p.es;
    const int64_t vs = ((int64_t)b * p.v_sb + (int64_t)t * p.v_st + (int64_t)h * p.v_sh) * p.es;
#if MPX_KV_NT
    // Every byte is moved once: non-temporal (streaming) loads and stores.
    const u32x4 kx = __builtin_nontemporal_load((const u32x4*)(p.k + ks + c * 16));
    const u32x4 vx = __builtin_nontemporal_load((const u32x4*)(p.v + vs + c * 16));
    __builtin_nontemporal_store(kx, (u32x4*)(p.kpool + dst));
    __builtin_nontemporal_store(vx, (u32x4*)(p.vpool + dst));
#else
    const u32x4 kx = *(const u32x4*)(p.k + ks + c * 16);
    const u32x4 vx = *(const u32x4*)(p.v + vs + c * 16);
    *(u32x4*)(p.kpool + dst) = kx;
    *(u32x4*)(p.vpool + dst) = vx;
#endif
  }
}

}  // namespace mpx

using namespace mpx;

extern "C" int mpx_kv_append(const void* k, const void* v, void* k_pool, void* v_pool,
                             const int32_t* block_tables, const int32_t* start_pos,
                             const int32_t* n_tokens, const int64_t* k_strides,
                             const int64_t* v_strides, int B, int T, int H, int D, int num_blocks,
                             int block_size, int max_blocks, int dtype, int32_t* errors,
                             void* stream) {
  clear_error();
  MPX_CHECK_ARG(dtype == MPX_F32 || dtype == MPX_F16 || dtype == MPX_BF16,
                "mpx_kv_append: unknown dtype code %d", dtype);
  MPX_CHECK_ARG(B >= 0 && T >= 0 && H >= 0 && D > 0 && num_blocks >= 0 && max_blocks >= 0,
                "mpx_kv_append: negative size");
  MPX_CHECK_ARG(block_size > 0, "mpx_kv_append: block_size must be positive");
  const int es = dtype == MPX_F32 ? 4 : 2;
  MPX_CHECK_ARG((D * es) % 16 == 0, "mpx_kv_append: head_dim * element size must be a multiple of 16 bytes");
  if ((long)B * T * H == 0) return MPX_OK;
  MPX_CHECK_ARG(k && v && k_pool && v_pool && block_tables && start_pos && n_tokens && k_strides &&
                    v_strides && errors,
                "mpx_kv_append: null pointer argument");
  MPX_CHECK_ARG(((uintptr_t)k & 15u) == 0 && ((uintptr_t)v & 15u) == 0 &&
                    ((uintptr_t)k_pool & 15u) == 0 && ((uintptr_t)v_pool & 15u) == 0,
                "mpx_kv_append: tensors must be 16-byte aligned");
  const int vec = 16 / es;
  for (int i = 0; i < 3; ++i)
    MPX_CHECK_ARG(k_strides[i] >= 0 && k_strides[i] % vec == 0 && v_strides[i] >= 0 &&
                      v_strides[i] % vec == 0,
                  "mpx_kv_append: strides must be non-negative multiples of %d elements", vec);
  AppendParams p;
  p.k = (const unsigned char*)k; p.v = (const unsigned char*)v;
  p.kpool = (unsigned char*)k_pool; p.vpool = (unsigned char*)v_pool;
  p.bt = block_tables; p.start = start_pos; p.ntok = n_tokens; p.err = errors;
  p.k_sb = k_strides[0]; p.k_st = k_strides[1]; p.k_sh = k_strides[2];
  p.v_sb = v_strides[0]; p.v_st = v_strides[1]; p.v_sh = v_strides[2];
  p.B = B; p.T = T; p.H = H; p.cpr = D * es / 16; p.es = es;
  p.num_blocks = num_blocks; p.bs = block_size; p.max_blocks = max_blocks;
  MPX_CHECK_ARG((int64_t)H * p.cpr < (1 << 30), "mpx_kv_append: head count too large");
  const int nbr = (H * p.cpr + 255) / 256;  // workgroups per token row
  const int64_t n_blk = (int64_t)B * T * nbr;
  MPX_CHECK_ARG(n_blk < (1L << 31), "mpx_kv_append: too many tokens in one call");
  const int blocks = (int)std::min<int64_t>(n_blk, 1 << 20);
  if (blocks > 0)
    hipLaunchKernelGGL(kv_append_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, p, nbr);
  MPX_CHECK_HIP(hipGetLastError());
  return MPX_OK;
}
