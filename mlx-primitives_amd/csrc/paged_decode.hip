// Paged-KV decode attention for gfx950 (MI355X).
//
// Semantics follow mlx_primitives/cache/paged_attention.py:108-208 (decode
// path of paged_attention): one query token per sequence, keys/values gathered
// through block_tables from pools laid out (num_blocks, block_size, H, D);
// token t is valid iff t < context_len and its page id is >= 0; optional ALiBi
// bias slope_h * (t - context_len) (163-178); exact softmax.
//
// Design (memory bound, ~1 FLOP/byte):
//   * split-K: each sequence's tokens are cut into partitions of PART tokens;
//     a workgroup = 2 or 4 waves = consecutive query heads of one (sequence,
//     partition), so its waves stream adjacent head rows of the same pages
//     (or, with grouped-query heads, share them);
//   * one pass over the partition: a token row of one head is read by LPT
//     lanes with 16-byte loads; the K and V rows of U tokens per lane are
//     requested together, partial dot products are reduced across the LPT
//     lanes, and every token group keeps its own running max and fp32
//     accumulator (online softmax), merged across the wave at the end;
//   * per-partition (o, m, l) go to the workspace; paged_decode_merge_kernel
//     combines them (online-softmax merge) and normalises by the exact sum.
// The page ids of a partition are staged once in LDS, invalid ids (< 0 or
// >= num_blocks) are masked and never dereferenced.
#include "mpx_common.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <mutex>

namespace mpx {

struct DecodeParams {
  const void* q;
  const void* kpool;
  const void* vpool;
  const int32_t* bt;
  const int32_t* cl;
  const float* slopes;
  void* o;
  int64_t q_sb, q_sh, o_sb, o_sh;
  float* ws_o;   // (B, H, max_parts, D)
  float* ws_ml;  // (B, H, max_parts, 2), m in log2 units
  int B, H, num_blocks, bs, max_blocks, max_parts;
  int H_kv, kv_group;  // K/V heads of the pools; query heads per K/V head
  int dp;   // head dim of q, the pools and o (elements, <= the kernel's D)
  float c;  // scale * log2(e)
  u32 pool_bytes;  // bytes of one pool; 0: 4 GiB - 256 bytes or more (64-bit addressing)
};

// Tokens per partition and 16-byte loads in flight per lane (overridable at
// build time for tuning builds).
#ifndef MPX_PD_PART
#define MPX_PD_PART 512
#endif
#ifndef MPX_PD_U
#define MPX_PD_U 16
#endif
constexpr int kPart = MPX_PD_PART;
// Query heads (waves) per workgroup: 4 with grouped-query heads, whose waves
// share K/V rows in L2; 2 when every K/V head serves one query head (measured
// 0.7% faster there, 14-23% slower with grouping).
template <bool NT>
constexpr int kHeadsPerWG = NT ? 2 : 4;

template <int DT>
__device__ __forceinline__ float elem(const u32x4& v, int i) {
  if constexpr (DT == MPX_F32) {
    return __uint_as_float(v[i]);
  } else {
    const u32 w = v[i >> 1];
    const uint16_t x = (uint16_t)((i & 1) ? (w >> 16) : (w & 0xffffu));
    return h2f<DT == MPX_BF16>(x);
  }
}

// K/V row load: non-temporal (streaming) when every row is read once per
// call (one query head per K/V head); with grouped-query heads the waves of a
// workgroup re-read the same rows, and the streaming hint would cost them
// their L2 hits (measured: 374 -> 478 us at 32 query heads over 8 K/V heads).
template <bool NT>
__device__ __forceinline__ u32x4 ld_kv(const u32x4* ptr) {
  if constexpr (NT) {
    return __builtin_nontemporal_load(ptr);
  } else {
    return *ptr;
  }
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, 64));
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

template <int D, int DT, bool NT>
__global__ __launch_bounds__(64 * kHeadsPerWG<NT>) void paged_decode_part_kernel(DecodeParams p) {
  constexpr int ES = DT == MPX_F32 ? 4 : 2;  // element bytes
  constexpr int EPC = 16 / ES;               // elements per 16-byte chunk
  constexpr int LPT = D / EPC;               // lanes per token row
  constexpr int TPI = 64 / LPT;              // tokens per wave-wide load
  constexpr int U = MPX_PD_U;                // tokens per lane per batch
  static_assert(LPT >= 1 && LPT <= 64 && 64 % LPT == 0, "head_dim");

  __shared__ int btl[kPart + 1];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = blockIdx.x * kHeadsPerWG<NT> + wave;
  const int part = blockIdx.y, b = blockIdx.z;
  const int ctx = max(0, min(p.cl[b], p.max_blocks * p.bs));
  const int p0 = part * kPart;
  if (p0 >= ctx) return;  // uniform over the workgroup
  const int p1 = min(p0 + kPart, ctx);
  const int pg0 = p0 / p.bs;
  const int npg = (p1 - 1) / p.bs - pg0 + 1;

  // Lane (tl, cidx): 16-byte chunk cidx of the head row of tokens tl, tl+TPI, ...
  const int cidx = lane % LPT, tl = lane / LPT;
  // Head rows of dp <= D elements: the lanes of chunks past dp read nothing
  // and hold zeros (they add nothing to q.k and their output is not written).
  const bool lane_on = cidx * EPC < p.dp;
  // The Q chunk and the ALiBi slope are requested before the page table, from
  // addresses that are always valid (a wave past the last head, a lane past
  // dp, no ALiBi: a row or word that is read and discarded), so that the
  // three loads share one latency.
  const int hq = min(h, p.H - 1);
  const u32x4 q_raw = *(const u32x4*)((const char*)p.q +
                                      ((int64_t)b * p.q_sb + (int64_t)hq * p.q_sh +
                                       (lane_on ? cidx * EPC : 0)) * ES);
  const float slope_any = *(p.slopes ? p.slopes + hq : (const float*)p.q);
  for (int i = tid; i < npg; i += 64 * kHeadsPerWG<NT>) {
    const int blk = p.bt[(int64_t)b * p.max_blocks + pg0 + i];
    btl[i] = (blk >= 0 && blk < p.num_blocks) ? blk : -1;
  }
  __syncthreads();
  if (h >= p.H) return;
  // Pool token rows hold H_kv heads; query head h reads K/V head h / kv_group.
  const int64_t row_elems = (int64_t)p.H_kv * p.dp;
  const int64_t hoff = (int64_t)(h / p.kv_group) * p.dp + cidx * EPC;
  const char* kbase = (const char*)p.kpool;
  const char* vbase = (const char*)p.vpool;

  float qv[EPC];
  {
    const u32x4 qr = lane_on ? q_raw : (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < EPC; ++i) qv[i] = elem<DT>(qr, i) * p.c;
  }
  const float slope2 = p.slopes ? slope_any * kLog2e : 0.f;

  // One pass over the partition: the K and V rows of a batch of U tokens per
  // lane are requested together; every token group (the LPT lanes of one
  // token slot) keeps its own running max m, so no cross-lane exchange is
  // needed until the end.
  float acc[EPC];
#pragma unroll
  for (int i = 0; i < EPC; ++i) acc[i] = 0.f;
  float m = -INFINITY, l = 0.f;
  for (int t0 = p0; t0 < p1; t0 += TPI * U) {
    u32x4 kr[U], vr[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int tk = t0 + u * TPI + tl;
      int blk = -1;
      if (tk < p1) blk = btl[tk / p.bs - pg0];
      ok[u] = blk >= 0;
      const bool ld = ok[u] && lane_on;
      const int64_t off = (((int64_t)blk * p.bs + tk % p.bs) * row_elems + hoff) * ES;
      kr[u] = ld ? ld_kv<NT>((const u32x4*)(kbase + off)) : (u32x4){0u, 0u, 0u, 0u};
      vr[u] = ld ? ld_kv<NT>((const u32x4*)(vbase + off)) : (u32x4){0u, 0u, 0u, 0u};
    }
    float sc[U];
    float mb = m;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float dot = 0.f;
#pragma unroll
      for (int i = 0; i < EPC; ++i) dot = fmaf(qv[i], elem<DT>(kr[u], i), dot);
#pragma unroll
      for (int off = LPT / 2; off >= 1; off >>= 1) dot += __shfl_xor(dot, off, 64);
      const int tk = t0 + u * TPI + tl;
      sc[u] = ok[u] ? dot + slope2 * (float)(tk - ctx) : -INFINITY;
      mb = fmaxf(mb, sc[u]);
    }
    if (mb > m) {
      const float alpha = m == -INFINITY ? 0.f : fast_exp2(m - mb);
      l *= alpha;
#pragma unroll
      for (int i = 0; i < EPC; ++i) acc[i] *= alpha;
      m = mb;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float w = sc[u] == -INFINITY ? 0.f : fast_exp2(sc[u] - m);
      l += w;
#pragma unroll
      for (int i = 0; i < EPC; ++i) acc[i] = fmaf(w, elem<DT>(vr[u], i), acc[i]);
    }
  }

  // Merge the token groups of the wave: rescale to the wave max, then sum
  // over the lanes holding the same dims.
  const float M = wave_max(m);
  const float f = m == -INFINITY ? 0.f : fast_exp2(m - M);
  l *= f;
#pragma unroll
  for (int i = 0; i < EPC; ++i) acc[i] *= f;
#pragma unroll
  for (int off = LPT; off < 64; off <<= 1) {
    l += __shfl_xor(l, off, 64);
#pragma unroll
    for (int i = 0; i < EPC; ++i) acc[i] += __shfl_xor(acc[i], off, 64);
  }

  const int64_t slot = ((int64_t)b * p.H + h) * p.max_parts + part;
  if (tl == 0) {
    float* wo = p.ws_o + slot * D + cidx * EPC;
#pragma unroll
    for (int i = 0; i < EPC; i += 4) *(f32x4*)(wo + i) = (f32x4){acc[i], acc[i + 1], acc[i + 2], acc[i + 3]};
  }
  if (lane == 0) {
    p.ws_ml[2 * slot] = M;
    p.ws_ml[2 * slot + 1] = l;
  }
}

// Combine the partitions of one (sequence, head): the online-softmax merge
// (mlx_primitives/attention/_online_softmax.py:42-106) over all partitions,
// then the exact normalisation o / l of the reference's softmax. One wave per
// (sequence, head): lane i takes the (m, l) of partition i and its weight
// 2^(m_i - M), lane l accumulates dims 2l, 2l+1 over the partitions (16
// partition rows in flight, each a coalesced 2 D-float read). D is the kernel
// head dim (the partials' row length); dp <= D columns are written. Head dims
// above 128 take one workgroup per 128 dims (blockIdx.y).
template <int DT>
__global__ __launch_bounds__(64) void paged_decode_merge_kernel(DecodeParams p, int D) {
  const int bh = blockIdx.x;
  const int b = bh / p.H, h = bh - (bh / p.H) * p.H;
  const int lane = threadIdx.x;
  const int ctx = max(0, min(p.cl[b], p.max_blocks * p.bs));
  const int nparts = (ctx + kPart - 1) / kPart;
  const int64_t base = (int64_t)bh * p.max_parts;
  const int d = 2 * lane + 128 * (int)blockIdx.y;
  const bool dl = d < D;
  // Online over chunks of 64 partitions (one chunk up to 32768 tokens): a
  // chunk's (m, l) and its first 16 partition rows are requested together.
  float M = -INFINITY, L = 0.f, acc0 = 0.f, acc1 = 0.f;
  for (int i0 = 0; i0 < nparts; i0 += 64) {
    const int n = min(64, nparts - i0);
    float mi = -INFINITY, li = 0.f;
    if (lane < n) {
      mi = p.ws_ml[2 * (base + i0 + lane)];
      li = p.ws_ml[2 * (base + i0 + lane) + 1];
    }
    float w = 0.f;
    for (int k = 0; k < n; k += 16) {
      float2 ov[16];
#pragma unroll
      for (int u = 0; u < 16; ++u)
        ov[u] = (k + u < n && dl) ? *(const float2*)(p.ws_o + (base + i0 + k + u) * D + d)
                                  : make_float2(0.f, 0.f);
      if (k == 0) {
        const float mn = fmaxf(M, wave_max(mi));
        const float keep = M == -INFINITY ? 0.f : fast_exp2(M - mn);
        acc0 *= keep;
        acc1 *= keep;
        L *= keep;
        M = mn;
        // 0 for partitions that saw no key (and while no partition has)
        w = (lane < n && M != -INFINITY) ? fast_exp2(mi - M) : 0.f;
        L += w * li;
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const float wk = __shfl(w, k + u, 64);
        acc0 = fmaf(wk, ov[u].x, acc0);
        acc1 = fmaf(wk, ov[u].y, acc1);
      }
    }
  }
  L = wave_sum(L);
  if (d >= p.dp) return;
  // no valid token: 0 / 0 = NaN, as the reference
  const float out0 = acc0 / L, out1 = acc1 / L;
  const int64_t off = (int64_t)b * p.o_sb + (int64_t)h * p.o_sh + d;
  if constexpr (DT == MPX_F32) {
    float* dst = (float*)p.o + off;
    dst[0] = out0;
    dst[1] = out1;
  } else {
    uint16_t* dst = (uint16_t*)p.o + off;
    const u32 pk = pack2<DT == MPX_BF16>(out0, out1);
    if (((uintptr_t)dst & 3u) == 0) {
      *(u32*)dst = pk;
    } else {
      dst[0] = (uint16_t)(pk & 0xffffu);
      dst[1] = (uint16_t)(pk >> 16);
    }
  }
}

// ---------------------------------------------------------------------------
// Grouped-query decode on MFMAs (16-bit, head dim 128, 2..16 query heads per
// K/V head). A wave owns one (sequence, K/V head, partition of kPart tokens)
// and scores every K row against all query heads of the group at once:
//   S^T (16 tokens x 16 heads) = K (16 x 128) Q^T (128 x 16): four 16x16x32
//   MFMAs per 16 tokens (columns past the group are zero heads);
//   O^T (16 dims x 16 heads) += V^T (16 dims x 32 tokens) P^T (32 x 16): eight
//   MFMAs per 32 tokens, one per 16 dims.
// So each K/V byte of the partition is read once for the whole group, and
// the per-(head, token) work is one exponential. K and V tiles of 32 tokens
// are staged in LDS by buffer-load DMA, two tiles in flight; 16-byte chunk c
// of token row r sits at chunk c ^ f(r), f(r) = r % 4 + 4 ((r / 8) % 4), so
// the 16 rows one operand read touches get 16 different XOR patterns. Lane
// l = i + 16 q reads the K operand as row i of a 16-token half (half h row i
// = token 8 (i / 4) + 4 h + i % 4), which makes the S^T values it holds (C
// rows 4q .. 4q+3 of both halves) the tokens 8q .. 8q+7 of its head: exactly
// its slice of the P^T operand. V^T comes through the transposing read
// (ds_read_b64_tr_b16). Waves are independent (no barriers): a wave whose
// partition starts past the context returns at once.
// ---------------------------------------------------------------------------
#ifndef MPX_GQA_WAVES
#define MPX_GQA_WAVES 1
#endif
#ifndef MPX_GQA_STAGES
#define MPX_GQA_STAGES 2
#endif
constexpr int kGqaWaves = MPX_GQA_WAVES;    // partitions per workgroup
constexpr int kGqaStages = MPX_GQA_STAGES;  // (K, V) tiles per wave in LDS
constexpr int kGqaTile = 32;                // tokens per step
constexpr u32 kGqaNoRow = 0xFFFFFF00u;  // DMA offset past any accepted pool: reads zeros

__device__ __forceinline__ int gqa_swz(int row) { return (row & 3) | (((row >> 3) & 3) << 2); }

// BIG: pools of 4 GiB - 256 bytes and more (pool_bytes == 0), whose rows the
// DMA reads through 64-bit addresses (rows without a page from kZeroChunk).
// POW2: page sizes that are powers of two, whose page index and slot come from
// a shift and a mask instead of a division.
template <bool BF16, bool BIG = false, bool POW2 = false>
__global__ __launch_bounds__(64 * kGqaWaves) void paged_decode_gqa_kernel(DecodeParams p) {
  constexpr int D = 128, ROWB = 2 * D, TILEB = kGqaTile * ROWB;
  // Per wave: kGqaStages stages of (K tile, V tile).
  __shared__ __align__(16) unsigned char kvt[kGqaWaves][kGqaStages][2][TILEB];
  __shared__ int btl[kGqaWaves][kPart + 1];
  static_assert(sizeof(kvt) + sizeof(btl) <= 131072, "LDS budget");
  static_assert(kGqaStages >= 2 && kGqaStages <= 4, "vmcnt counts up to 3 later tiles");

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // K/V heads vary fastest over the launch, so the workgroups running together
  // read all heads of the same token rows (whole rows of the pool's pages).
  const int hk = blockIdx.x, part = blockIdx.y * kGqaWaves + wave, b = blockIdx.z;
  const int ctx = max(0, min(p.cl[b], p.max_blocks * p.bs));
  const int p0 = part * kPart;
  if (p0 >= ctx) return;  // uniform over the wave
  const int p1 = min(p0 + kPart, ctx);
  const int bsh = POW2 ? __builtin_ctz((unsigned)p.bs) : 0;
  auto page_of = [&](int t) __attribute__((always_inline)) { return POW2 ? t >> bsh : t / p.bs; };
  auto slot_of = [&](int t) __attribute__((always_inline)) {
    return POW2 ? t & (p.bs - 1) : t % p.bs;
  };
  const int pg0 = page_of(p0);
  const int npg = page_of(p1 - 1) - pg0 + 1;

  const int i16 = lane & 15, q4 = lane >> 4;
  const int G = p.kv_group;
  const bool hv = i16 < G;        // column i16 is a query head of the group
  const int h = hk * G + i16;
  // Q rows first and unconditionally (columns past the group read the
  // group's first head and are zeroed below), so that the five loads of the
  // prologue share one latency instead of running one after another.
  u32x4 qb[4];
  const uint16_t* qrow = (const uint16_t*)p.q + (int64_t)b * p.q_sb +
                         (int64_t)(hv ? h : hk * G) * p.q_sh + 8 * q4;
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) qb[kb] = *(const u32x4*)(qrow + 32 * kb);
  // (without ALiBi a dummy read of Q's first word, discarded: no branch, no
  // wait of its own)
  const float* sp = p.slopes ? p.slopes + (hv ? h : hk * G) : (const float*)p.q;
  const float slope_any = *sp;
  const float slope_raw = p.slopes ? slope_any : 0.f;
  int* bl = btl[wave];
  for (int i = lane; i < npg; i += 64) {
    const int blk = p.bt[(int64_t)b * p.max_blocks + pg0 + i];
    bl[i] = (blk >= 0 && blk < p.num_blocks) ? blk : -1;
  }
  // (this wave's own LDS writes: its later reads see them in order)

  // Q^T operand (column i16, dims 32 kb + 8 q4 .. +7) times scale * log2(e),
  // rounded to the storage type: S^T comes out of the MFMAs in log2 units.
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    u32x4 x = hv ? qb[kb] : (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
    for (int w = 0; w < 4; ++w)
      x[w] = pack2<BF16>(h2f<BF16>((uint16_t)(x[w] & 0xffffu)) * p.c,
                         h2f<BF16>((uint16_t)(x[w] >> 16)) * p.c);
    qb[kb] = x;
  }
  const float slope2 = hv ? slope_raw * kLog2e : 0.f;
  // Q (and the table) have landed before any DMA, so the waits below count
  // DMAs only.
  __builtin_amdgcn_s_waitcnt(0x0F70);

  // Buffers of this K/V head's column of the pools (32-bit offsets: pools
  // below 4 GiB - 256 bytes; BIG: 64-bit addresses from the same bases).
  const u32 rec = p.pool_bytes - (u32)(hk * D * 2);
  const unsigned char* kbase = (const unsigned char*)p.kpool + (int64_t)hk * D * 2;
  const unsigned char* vbase = (const unsigned char*)p.vpool + (int64_t)hk * D * 2;
  const u32x4 krs = buffer_desc((const uint16_t*)p.kpool + (int64_t)hk * D, rec);
  const u32x4 vrs = buffer_desc((const uint16_t*)p.vpool + (int64_t)hk * D, rec);
  const u32 row_bytes = (u32)p.H_kv * (u32)D * 2u;

  // K and V rows of the tile at t0 into stage sb: 8 DMA instructions each;
  // lane l fills slot l % 16 of row 4v + l / 16 with its chunk (l % 16) ^ f(row).
  // The eight page ids are read first (clamped rows, no branch), so that
  // their LDS reads share one wait.
  auto load_tile = [&](int t0, int sb) __attribute__((always_inline)) {
    const u32 kdst = lds_addr(kvt[wave][sb][0]), vdst = lds_addr(kvt[wave][sb][1]);
    int pgs[kGqaTile / 4];
#pragma unroll
    for (int v = 0; v < kGqaTile / 4; ++v) pgs[v] = bl[page_of(min(t0 + 4 * v + q4, p1 - 1)) - pg0];
#pragma unroll
    for (int v = 0; v < kGqaTile / 4; ++v) {
      const int r = 4 * v + q4;
      const int t = t0 + r;
      const int pg = t < p1 ? pgs[v] : -1;
      if constexpr (BIG) {
        const uint64_t off = ((uint64_t)(u32)pg * (u32)p.bs + (u32)slot_of(t)) * row_bytes +
                             (u32)((i16 ^ gqa_swz(r)) * 16);
        dma16_global(kdst + 4 * v * ROWB, pg >= 0 ? (const void*)(kbase + off) : &kZeroChunk);
        dma16_global(vdst + 4 * v * ROWB, pg >= 0 ? (const void*)(vbase + off) : &kZeroChunk);
        continue;
      }
      const u32 off = pg >= 0 ? ((u32)pg * (u32)p.bs + (u32)slot_of(t)) * row_bytes +
                                    (u32)((i16 ^ gqa_swz(r)) * 16)
                              : kGqaNoRow;
      dma16(krs, kdst + 4 * v * ROWB, (int)off, 0);
      dma16(vrs, vdst + 4 * v * ROWB, (int)off, 0);
    }
  };

  f32x4 o[D / 16];
#pragma unroll
  for (int db = 0; db < D / 16; ++db) o[db] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, lsum = 0.f;

  const int n_tiles = (p1 - p0 + kGqaTile - 1) / kGqaTile;
#pragma unroll
  for (int i = 0; i < kGqaStages - 1; ++i)
    if (i < n_tiles) load_tile(p0 + i * kGqaTile, i);
  int sb = 0;
  for (int it = 0; it < n_tiles; ++it) {
    const int t0 = p0 + it * kGqaTile;
    if (it + kGqaStages - 1 < n_tiles)
      load_tile(t0 + (kGqaStages - 1) * kGqaTile,
                sb == 0 ? kGqaStages - 1 : sb - 1);
    // Tile it has landed once at most the 16 DMAs of each later tile are
    // pending.
    const int later = min(n_tiles - 1, it + kGqaStages - 1) - it;
    if (later >= 3) {
      asm volatile("s_waitcnt vmcnt(48)" ::: "memory");
    } else if (later == 2) {
      asm volatile("s_waitcnt vmcnt(32)" ::: "memory");
    } else if (later == 1) {
      asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    const unsigned char* kt = kvt[wave][sb][0];
    const unsigned char* vt = kvt[wave][sb][1];
    // S^T of the two 16-token halves.
    f32x4 s[2];
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      const int r = 8 * (i16 >> 2) + 4 * f + (i16 & 3);
      s[f] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const u32x4 ka = *(const u32x4*)(kt + r * ROWB + (((4 * kb + q4) ^ gqa_swz(r)) * 16));
        s[f] = mfma16x16x32<BF16>(ka, qb[kb], s[f]);
      }
    }
    // Masks (missing pages, the context end), ALiBi, the tile max of head i16.
    const int tl = t0 + (lane & 31);
    const uint64_t vm = __ballot(tl < p1 && bl[page_of(min(tl, p1 - 1)) - pg0] >= 0);
    float mx = -INFINITY;
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tok = 8 * q4 + 4 * f + r;
        float x = s[f][r] + slope2 * (float)(t0 + tok - ctx);
        x = ((vm >> tok) & 1ull) ? x : -INFINITY;
        s[f][r] = x;
        mx = fmaxf(mx, x);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    if (__any(mx > m)) {
      const float mn = fmaxf(m, mx);
      const float alpha = m == -INFINITY ? 0.f : fast_exp2(m - mn);
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < D / 16; ++db) o[db] *= alpha;
      m = mn;
    }
    const float msub = m == -INFINITY ? 0.f : m;
    // P^T slice of this lane: tokens 8 q4 .. 8 q4 + 7 of head i16.
    u32x4 pb;
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
      for (int r2 = 0; r2 < 2; ++r2) {
        const u32 pk = pack2<BF16>(fast_exp2(s[f][2 * r2] - msub),
                                   fast_exp2(s[f][2 * r2 + 1] - msub));
        pb[2 * f + r2] = pk;
        lsum = dot2_sum<BF16>(pk, lsum);
      }
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      const int c = 2 * db + ((i16 & 3) >> 1);
      const int r0 = 8 * q4 + (i16 >> 2);
      const u32x2 lo = lds_read_tr16(vt + r0 * ROWB + ((c ^ gqa_swz(r0)) * 16) + (i16 & 1) * 8);
      const u32x2 hi =
          lds_read_tr16(vt + (r0 + 4) * ROWB + ((c ^ gqa_swz(r0 + 4)) * 16) + (i16 & 1) * 8);
      o[db] = mfma16x16x32<BF16>((u32x4){lo[0], lo[1], hi[0], hi[1]}, pb, o[db]);
    }
    // Every read of stage sb is done before a later iteration's DMAs refill
    // it (the MFMAs above consumed them).
    sb = sb + 1 == kGqaStages ? 0 : sb + 1;
  }

  // Sum of head i16 over the four lanes holding its tokens.
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);
  if (hv) {
    const int64_t slot = ((int64_t)b * p.H + h) * p.max_parts + part;
    float* wo = p.ws_o + slot * D + 4 * q4;
#pragma unroll
    for (int db = 0; db < D / 16; ++db) *(f32x4*)(wo + 16 * db) = o[db];
    if (q4 == 0) {
      p.ws_ml[2 * slot] = m;
      p.ws_ml[2 * slot + 1] = lsum;
    }
  }
}

namespace {

int max_parts_for(int block_size, int max_blocks) {
  const long tokens = (long)block_size * max_blocks;
  return (int)((tokens + kPart - 1) / kPart);
}

// Kernel head dim serving pools of head dim D (<= 256): 32, 64, 128 or 256.
int kernel_dim(int D) { return D <= 32 ? 32 : D <= 64 ? 64 : D <= 128 ? 128 : 256; }

// Merge workgroups per (sequence, head): one per 128 dims.
dim3 merge_grid(const DecodeParams& p, int D) {
  return dim3(p.B * p.H, D > 128 ? D / 128 : 1);
}

// The grouped-query MFMA kernel serves 16-bit pools of head dim 128 with 2 to
// 16 query heads per K/V head (pools of 4 GiB - 256 bytes and more,
// pool_bytes == 0, through its 64-bit address form).
template <int D, int DT>
constexpr bool kGqaMfmaType = D == 128 && DT != MPX_F32;

template <int D, int DT>
hipError_t launch_decode(const DecodeParams& p, hipStream_t st) {
  if constexpr (kGqaMfmaType<D, DT>) {
    if (p.kv_group >= 2 && p.kv_group <= 16 && p.dp == D) {
      const dim3 grid(p.H_kv, (p.max_parts + kGqaWaves - 1) / kGqaWaves, p.B);
      const bool pow2 = (p.bs & (p.bs - 1)) == 0;
      if (p.pool_bytes != 0) {
        if (pow2)
          hipLaunchKernelGGL((paged_decode_gqa_kernel<DT == MPX_BF16, false, true>), grid,
                             dim3(64 * kGqaWaves), 0, st, p);
        else
          hipLaunchKernelGGL((paged_decode_gqa_kernel<DT == MPX_BF16>), grid,
                             dim3(64 * kGqaWaves), 0, st, p);
      } else {
        if (pow2)
          hipLaunchKernelGGL((paged_decode_gqa_kernel<DT == MPX_BF16, true, true>), grid,
                             dim3(64 * kGqaWaves), 0, st, p);
        else
          hipLaunchKernelGGL((paged_decode_gqa_kernel<DT == MPX_BF16, true>), grid,
                             dim3(64 * kGqaWaves), 0, st, p);
      }
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL(paged_decode_merge_kernel<DT>, merge_grid(p, D), dim3(64), 0, st, p, D);
      return hipGetLastError();
    }
  }
  if (p.kv_group == 1) {
    constexpr int W = kHeadsPerWG<true>;
    const dim3 grid((p.H + W - 1) / W, p.max_parts, p.B);
    hipLaunchKernelGGL((paged_decode_part_kernel<D, DT, true>), grid, dim3(64 * W), 0, st, p);
  } else {
    constexpr int W = kHeadsPerWG<false>;
    const dim3 grid((p.H + W - 1) / W, p.max_parts, p.B);
    hipLaunchKernelGGL((paged_decode_part_kernel<D, DT, false>), grid, dim3(64 * W), 0, st, p);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(paged_decode_merge_kernel<DT>, merge_grid(p, D), dim3(64), 0, st, p, D);
  return hipGetLastError();
}

template <int DT>
hipError_t dispatch_decode_d(const DecodeParams& p, int D, hipStream_t st) {
  switch (D) {
    case 32: return launch_decode<32, DT>(p, st);
    case 64: return launch_decode<64, DT>(p, st);
    case 256: return launch_decode<256, DT>(p, st);
    default: return launch_decode<128, DT>(p, st);
  }
}

// Workspace bytes of one call: (o, m, l) per (sequence, head, partition).
size_t decode_ws_bytes(int B, int H, int D, int block_size, int max_blocks) {
  const int parts = std::max(1, max_parts_for(block_size, max_blocks));
  return (size_t)B * H * parts * (kernel_dim(D) + 2) * sizeof(float);
}

// Validation, parameters and launches shared by the workspace entry and the
// no-allocation entry. `workspace` == nullptr with need > 0 is an error.
int paged_decode_run(const void* q, const void* k_pool, const void* v_pool,
                     const int32_t* block_tables, const int32_t* context_lens,
                     const float* alibi_slopes, void* o, const int64_t* q_strides,
                     const int64_t* o_strides, int B, int H, int H_kv, int D, int num_blocks,
                     int block_size, int max_blocks, float scale, int dtype, void* workspace,
                     size_t workspace_bytes, void* stream, const char* who) {
  MPX_CHECK_ARG(dtype == MPX_F32 || dtype == MPX_F16 || dtype == MPX_BF16,
                "%s: unknown dtype code %d", who, dtype);
  MPX_CHECK_ARG(B >= 0 && H >= 0 && num_blocks >= 0 && max_blocks >= 0, "%s: negative size",
                who);
  MPX_CHECK_ARG(H_kv > 0 ? H % H_kv == 0 : H == 0,
                "%s: %d query heads are not a multiple of %d K/V heads", who, H, H_kv);
  MPX_CHECK_ARG(block_size > 0, "%s: block_size must be positive", who);
  const int vec = dtype == MPX_F32 ? 4 : 8;
  if (D <= 0 || D > 256 || D % vec != 0) {
    set_error("%s: head_dim %d not supported (a multiple of %d elements up to 256)", who, D,
              vec);
    return MPX_EUNSUPPORTED;
  }
  MPX_CHECK_ARG(std::isfinite(scale), "%s: scale must be finite", who);
  if ((long)B * H == 0) return MPX_OK;
  MPX_CHECK_ARG(q && o && context_lens && q_strides && o_strides, "%s: null pointer argument",
                who);
  MPX_CHECK_ARG(max_blocks == 0 || (k_pool && v_pool && block_tables) || num_blocks == 0,
                "%s: null pool/table pointer", who);
  MPX_CHECK_ARG(((uintptr_t)q & 15u) == 0 && ((uintptr_t)k_pool & 15u) == 0 &&
                    ((uintptr_t)v_pool & 15u) == 0,
                "%s: q and pools must be 16-byte aligned", who);
  MPX_CHECK_ARG(q_strides[0] % vec == 0 && q_strides[1] % vec == 0,
                "%s: q strides must be multiples of %d elements", who, vec);
  const long max_tokens = (long)max_blocks * block_size;
  MPX_CHECK_ARG(max_tokens < (1L << 30), "%s: block table too large", who);

  const int kd = kernel_dim(D);
  DecodeParams p;
  p.q = q; p.kpool = k_pool; p.vpool = v_pool; p.bt = block_tables; p.cl = context_lens;
  p.slopes = alibi_slopes; p.o = o;
  p.q_sb = q_strides[0]; p.q_sh = q_strides[1]; p.o_sb = o_strides[0]; p.o_sh = o_strides[1];
  p.B = B; p.H = H; p.num_blocks = num_blocks; p.bs = block_size; p.max_blocks = max_blocks;
  p.H_kv = H_kv; p.kv_group = H / H_kv;
  p.dp = D;
  p.max_parts = std::max(1, max_parts_for(block_size, max_blocks));
  p.c = scale * kLog2e;
  const uint64_t pool_bytes =
      (uint64_t)num_blocks * block_size * H_kv * D * (dtype == MPX_F32 ? 4 : 2);
  p.pool_bytes = pool_bytes < 0xFFFFFF00ull ? (u32)pool_bytes : 0u;
  const size_t need = decode_ws_bytes(B, H, D, block_size, max_blocks);
  MPX_CHECK_ARG(workspace != nullptr && workspace_bytes >= need && ((uintptr_t)workspace & 15u) == 0,
                "%s: 16-byte aligned workspace of %zu bytes required, %zu given", who, need,
                workspace_bytes);
  MPX_CHECK_ARG(p.max_parts <= 65535 && B <= 65535, "%s: grid too large", who);
  p.ws_o = (float*)workspace;
  p.ws_ml = (float*)workspace + (size_t)B * H * p.max_parts * kd;
  if (num_blocks == 0 || max_blocks == 0) {
    // No page can be valid; the partition kernel has no work, the merge writes NaN.
    p.max_blocks = 0;
  }

  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (dtype == MPX_F32)
    e = dispatch_decode_d<MPX_F32>(p, kd, st);
  else if (dtype == MPX_BF16)
    e = dispatch_decode_d<MPX_BF16>(p, kd, st);
  else
    e = dispatch_decode_d<MPX_F16>(p, kd, st);
  MPX_CHECK_HIP(e);
  return MPX_OK;
}

// ---- device scratch of the no-allocation entry --------------------------------
//
// mpx_paged_decode_noalloc keeps its (o, m, l) partials in this file-scope
// array instead of a caller workspace. Every GPU the library runs on holds its
// own copy (MPX_NOALLOC_SCRATCH_BYTES) until the process ends. In host code
// the name `scratch` is only a stand-in for the symbol: its device address is
// looked up once per device with hipGetSymbolAddress, and only that address is
// handed to kernels.
static __device__ __align__(256) unsigned char scratch[MPX_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on the calling thread's current device, which
// must also be the device of `stream`.
int scratch_for_stream(void* stream, void** out) {
  int dev = -1;
  MPX_CHECK_HIP(hipGetDevice(&dev));
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    MPX_CHECK_HIP(hipStreamGetDevice((hipStream_t)stream, &sdev));
    MPX_CHECK_ARG(sdev == dev,
                  "mpx_paged_decode_noalloc: the stream belongs to device %d, the current "
                  "device is %d",
                  (int)sdev, dev);
  }
  MPX_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "mpx_paged_decode_noalloc: device %d out of range",
                dev);
  void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ptr = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (ptr == nullptr) {
      MPX_CHECK_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
      MPX_CHECK_ARG(ptr != nullptr && ((uintptr_t)ptr & 255u) == 0,
                    "mpx_paged_decode_noalloc: no device address for the scratch array");
      g_scratch_ptr[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return MPX_OK;
}

}  // namespace
}  // namespace mpx

using namespace mpx;

extern "C" size_t mpx_paged_decode_workspace_bytes(int B, int H, int D, int block_size,
                                                   int max_blocks) {
  if (B <= 0 || H <= 0 || D <= 0 || block_size <= 0 || max_blocks <= 0) return 0;
  return decode_ws_bytes(B, H, D, block_size, max_blocks);
}

extern "C" int mpx_paged_decode_gqa(const void* q, const void* k_pool, const void* v_pool,
                                    const int32_t* block_tables, const int32_t* context_lens,
                                    const float* alibi_slopes, void* o,
                                    const int64_t* q_strides, const int64_t* o_strides, int B,
                                    int H, int H_kv, int D, int num_blocks, int block_size,
                                    int max_blocks, float scale, int dtype, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  clear_error();
  return paged_decode_run(q, k_pool, v_pool, block_tables, context_lens, alibi_slopes, o,
                          q_strides, o_strides, B, H, H_kv, D, num_blocks, block_size,
                          max_blocks, scale, dtype, workspace, workspace_bytes, stream,
                          "mpx_paged_decode");
}

extern "C" int mpx_paged_decode(const void* q, const void* k_pool, const void* v_pool,
                                const int32_t* block_tables, const int32_t* context_lens,
                                const float* alibi_slopes, void* o, const int64_t* q_strides,
                                const int64_t* o_strides, int B, int H, int D, int num_blocks,
                                int block_size, int max_blocks, float scale, int dtype,
                                void* workspace, size_t workspace_bytes, void* stream) {
  return mpx_paged_decode_gqa(q, k_pool, v_pool, block_tables, context_lens, alibi_slopes, o,
                              q_strides, o_strides, B, H, H > 0 ? H : 1, D, num_blocks,
                              block_size, max_blocks, scale, dtype, workspace, workspace_bytes,
                              stream);
}

extern "C" int mpx_paged_decode_noalloc(const void* q, const void* k_pool, const void* v_pool,
                                        const int32_t* block_tables, const int32_t* context_lens,
                                        const float* alibi_slopes, void* o,
                                        const int64_t* q_strides, const int64_t* o_strides,
                                        int B, int H, int H_kv, int D, int num_blocks,
                                        int block_size, int max_blocks, float scale, int dtype,
                                        void* stream) {
  clear_error();
  if (B > 0 && H > 0 && D > 0 && block_size > 0 && max_blocks >= 0) {
    const size_t need = decode_ws_bytes(B, H, D, block_size, max_blocks);
    MPX_CHECK_ARG(need <= (size_t)MPX_NOALLOC_SCRATCH_BYTES,
                  "mpx_paged_decode_noalloc: the call needs %zu bytes of partials, more than "
                  "the %zu-byte device scratch (B * H * ceil(max_blocks * block_size / 512) * "
                  "(kernel head dim + 2) * 4 bytes); use mpx_paged_decode with a workspace",
                  need, (size_t)MPX_NOALLOC_SCRATCH_BYTES);
  }
  void* ws = nullptr;
  const int rc = scratch_for_stream(stream, &ws);
  if (rc != MPX_OK) return rc;
  return paged_decode_run(q, k_pool, v_pool, block_tables, context_lens, alibi_slopes, o,
                          q_strides, o_strides, B, H, H_kv, D, num_blocks, block_size,
                          max_blocks, scale, dtype, ws, (size_t)MPX_NOALLOC_SCRATCH_BYTES, stream,
                          "mpx_paged_decode_noalloc");
}
