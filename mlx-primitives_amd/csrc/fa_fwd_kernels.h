// Exact-softmax attention forward for gfx950 (MI355X): flash / sliding-window /
// chunked-cross attention of mlx-primitives on MFMA.
//
// Algorithm: the reference's tiled online softmax
// (mlx_primitives/attention/_online_softmax.py:42-176, attention/flash.py:257-316),
// restated for CDNA4:
//   * one workgroup = BM = 32*NW query rows of one (batch, head) and a range of
//     KV tiles of BN keys; every wave owns 32 query rows;
//   * scores are computed transposed, S^T = K Q^T, so that every lane holds 32
//     scores of a single query row: the row max needs one exchange with lane^32
//     and the row sum none until the end;
//   * P^T (bf16/f16) produced in the MFMA accumulator layout is fed straight
//     back as the B operand of O^T += V^T P^T; V is transposed once per tile
//     when it is staged into LDS (shared by all waves), K rows are permuted so
//     that each lane's P^T values are contiguous keys;
//   * K/V tiles are double-buffered in LDS with one barrier per tile; the
//     next tile's global loads are in flight while the current one computes;
//   * masks are index arithmetic (causal, left/right window, Sk tail); whole
//     tiles outside the mask are never visited (WG range) or skipped (wave);
//   * softmax in base 2 with scale*log2(e) folded in; the running max is only
//     moved when a row max grows by more than 2^8, so O is rarely rescaled;
//   * long KV ranges are split across workgroups (split-KV); partial
//     (O, m, l) are merged by fa_split_merge_kernel, the reference's
//     online_softmax_merge.
//
// This header holds the kernels; fa_fwd.hip holds the launches and entry
// points, fa_fwd_drop.hip the dropout launches (a translation unit of its own,
// so that the two can be built with different scheduler options).
#pragma once

#include "mpx_common.h"

#include <algorithm>
#include <cmath>

namespace mpx {

struct FwdParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  float* ws_o;   // split partials O: (splits, B, H, Sq, D) fp32, unnormalised
  float* ws_ml;  // split partials (m, l): (splits, B, H, Sq, 2) fp32, m in log2 units
  int B, H, Sq, Sk;
  int kv_group;  // query heads per K/V head (grouped-query attention; 1 = one each)
  int win_left, win_right;  // -1 = unbounded
  int n_qtiles, num_splits, tiles_per_split;
  int n_slots;  // q-tile slots per (batch, head)
  // > 0: every q-tile has its own split count, max(1, ceil(its KV tiles /
  // tiles_per_split)), and var_split is their sum per (batch, head); 0: every
  // q-tile has num_splits splits.
  int var_split;
  int bm, bn;  // query rows per q-tile, keys per KV tile of the launch
  // Windowed launches: the first q-tile whose KV range has the full window
  // length (slot_qtile), else -1.
  int win_first;
  int paired;   // a slot runs q-tiles n_qtiles-1-slot and slot (causal balance)
  // Paired launches, > 0: the last tail_bh (batch, head)s of every XCD's slice
  // run their q-tiles one per workgroup, longest first (B * H % 8 == 0).
  int tail_bh;
  float c;  // |scale| * log2(e)
  int neg;  // scale < 0: Q is negated on load (exact) and |scale| used
  float eps;      // normaliser epsilon: O / (l + eps)
  int nan_empty;  // rows that see no key give NaN (exact softmax) instead of 0
  // Optional (B, H, Sq) float32 log-sum-exp of each row in log2 units,
  // m + log2(l + eps), +inf for a row that sees no key: with it
  // P = exp2(s * c - lse) is recomputed by the backward kernels.
  float* lse;
  // Optional rotary embedding of Q on load (16-bit kernels): query row i is
  // rotated to position rope_offset + i with the (positions, D/2) cos / sin
  // tables (element type rope_cdt), as the RoPE kernel would before the call.
  const void* rope_cos;
  const void* rope_sin;
  int rope_offset, rope_cdt;
  // Paged K/V (prefill over a block-table cache; the PAGED kernels only): k
  // and v are the pools (num_blocks, bs, H, D), k_ss / v_ss their token row
  // stride H*D; the rows of batch b come through bt[b, pos / bs].
  const int32_t* bt;    // (B, max_blocks) page ids, < 0 or >= num_blocks = none
  const int32_t* ctx;   // (B,) context lengths: keys [0, ctx[b]) exist
  const float* slopes;  // (H,) ALiBi slopes (bias slope * (kv - q)) or null
  int bs, bs_log2;      // page size in tokens; log2(bs) or -1 if not a power of 2
  int max_blocks, num_blocks;
  uint32_t pool_bytes;  // bytes of one pool from its base (bounds of the buffer loads)
  // Dropout on the weights (the dropout kernels only): keep threshold and seed
  // words of the keep-mask hash, and the 1 / (1 - p) of the kept weights.
  uint32_t drop_thresh, seed0, seed1;
  float drop_scale;
};

// Page-table slice of one work item staged in LDS (entries).
constexpr int kMaxItemPages = 2048;

// Eight consecutive cos or sin entries of a RoPE table as floats.
__device__ __forceinline__ void load_angles8(const void* table, int64_t idx, int cdt,
                                             float (&out)[8]) {
  if (cdt == MPX_F32) {
    const f32x4 a = *(const f32x4*)((const float*)table + idx);
    const f32x4 b = *(const f32x4*)((const float*)table + idx + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[i] = a[i];
      out[4 + i] = b[i];
    }
  } else {
    const u32x4 w = *(const u32x4*)((const uint16_t*)table + idx);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = cdt == MPX_BF16 ? h2f<true>((uint16_t)(w[i] & 0xffffu))
                                   : h2f<false>((uint16_t)(w[i] & 0xffffu));
      out[2 * i + 1] = cdt == MPX_BF16 ? h2f<true>((uint16_t)(w[i] >> 16))
                                       : h2f<false>((uint16_t)(w[i] >> 16));
    }
  }
}

// Rotate a lane's Q fragments (dims 16 ks + 8 g .. +7 for ks < NKS) to position
// pos: the half-split partner of dim 16 ks + 8 g + i is dim 16 (ks + NKS/2) +
// 8 g + i, held by the same lane, so the rotation needs no data exchange. The
// arithmetic and rounding are those of the RoPE kernel (rope_pair, one
// rounding to the 16-bit type).
template <int NKS, bool BF16>
__device__ __forceinline__ void rope_q_frags(const FwdParams& p, int pos, int g,
                                             u32x4 (&qreg)[NKS]) {
  constexpr int HALF = NKS * 8;
#pragma unroll
  for (int ks = 0; ks < NKS / 2; ++ks) {
    float c[8], sn[8];
    const int64_t idx = (int64_t)pos * HALF + 16 * ks + 8 * g;
    load_angles8(p.rope_cos, idx, p.rope_cdt, c);
    load_angles8(p.rope_sin, idx, p.rope_cdt, sn);
    u32x4 lo = qreg[ks], hi = qreg[ks + NKS / 2];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      float y1a, y2a, y1b, y2b;
      rope_pair(h2f<BF16>((uint16_t)(lo[w] & 0xffffu)), h2f<BF16>((uint16_t)(hi[w] & 0xffffu)),
                c[2 * w], sn[2 * w], y1a, y2a);
      rope_pair(h2f<BF16>((uint16_t)(lo[w] >> 16)), h2f<BF16>((uint16_t)(hi[w] >> 16)),
                c[2 * w + 1], sn[2 * w + 1], y1b, y2b);
      lo[w] = pack2<BF16>(y1a, y1b);
      hi[w] = pack2<BF16>(y2a, y2b);
    }
    qreg[ks] = lo;
    qreg[ks + NKS / 2] = hi;
  }
}

__device__ __forceinline__ int page_of(const FwdParams& p, int pos) {
  return p.bs_log2 >= 0 ? pos >> p.bs_log2 : pos / p.bs;
}

// Tile configuration (overridable at build time for tuning builds).
// 16-bit kernel: 8 waves x 32 rows = 256 query rows per workgroup, two waves
// per SIMD (<= 256 registers each) so one wave's softmax overlaps the other's
// MFMAs. fp32 kernel: 4 waves.
#ifndef MPX_FA_NWAVES
#define MPX_FA_NWAVES 8
#endif
#ifndef MPX_FA_WAVES_PER_EU
#define MPX_FA_WAVES_PER_EU 2
#endif
#ifndef MPX_FA_SCHED
#define MPX_FA_SCHED 2
#endif
#ifndef MPX_FA_NWAVES_F32
#define MPX_FA_NWAVES_F32 4
#endif
// Keys per KV tile of the direct 16-bit kernels (D = 64, 128); the paged,
// D = 32 and register-staged 16-bit kernels take 64.
#ifndef MPX_FA_BN16
#define MPX_FA_BN16 128
#endif
// K/V tiles held in registers ahead of their LDS staging: 2 (tile i+2 is
// loaded while tile i computes) or 1 (tile i+1).
#ifndef MPX_FA_DEPTH
#define MPX_FA_DEPTH 2
#endif
// 1: D = 128 tiles are staged by direct global->LDS loads (see fa16_rows_direct).
#ifndef MPX_FA_DIRECT
#define MPX_FA_DIRECT 1
#endif
// LDS stages of the direct path (tile i+NST-1 in flight while tile i
// computes); 0 = as many as fit 128 KB, at most 4.
#ifndef MPX_FA_DSTAGES
#define MPX_FA_DSTAGES 0
#endif
// LDS stages of the register-staged 16-bit kernel.
constexpr int kFa16Stages = 2;


// Rescale threshold of the lazy running max, in log2 units.
constexpr float kRescaleThreshold = 8.0f;

// Work of a workgroup: one slot (batch*head, slot, split). Consecutive
// workgroup ids are dealt round-robin to the 8 XCDs; the remap gives every XCD
// a contiguous slice of the work so the q-tiles of one (batch, head) share that
// XCD's L2 for their K/V reads.
struct WorkSlot {
  int bh, slot, split;
  int single;  // >= 0: the slot is this one q-tile alone
};

struct WorkItem {
  int b, h, qt, split;
};

// KV tiles of q-tile qt (rows [qt*BM, +BM) against keys [0, Sk) under the
// window / causal bounds): the count kv_range gives, on host and device.
__host__ __device__ inline int qtile_kv_tiles(int qt, int BM, int BN, int Sq, int Sk, int wl,
                                              int wr) {
  const int q0 = qt * BM, q_last = (q0 + BM < Sq ? q0 + BM : Sq) - 1;
  int lo = wl >= 0 ? (q0 - wl > 0 ? q0 - wl : 0) : 0;
  lo -= lo % BN;
  const int hi = wr >= 0 ? (Sk < q_last + wr + 1 ? Sk : q_last + wr + 1) : Sk;
  return hi > lo ? (hi - lo + BN - 1) / BN : 0;
}

// Splits of q-tile qt when each q-tile has its own count (var_split).
__host__ __device__ inline int qtile_splits(int qt, int BM, int BN, int Sq, int Sk, int wl, int wr,
                                            int tiles_per_split) {
  const int n = qtile_kv_tiles(qt, BM, BN, Sq, Sk, wl, wr);
  return n > tiles_per_split ? (n + tiles_per_split - 1) / tiles_per_split : 1;
}

__device__ __forceinline__ int slot_qtile(const FwdParams& p, int slot) {
  if (p.win_first < 0) return p.n_qtiles - 1 - slot;
  const int k = p.win_first, n_long = p.n_qtiles - k;
  return slot < n_long ? k + slot : k - 1 - (slot - n_long);
}

__device__ __forceinline__ WorkSlot decode_slot(const FwdParams& p) {
  const int L = blockIdx.x, N = gridDim.x;
  if (p.tail_bh > 0) {
    // XCD L % 8 takes (batch, head)s [x * bpx, (x + 1) * bpx) in dispatch
    // order L / 8: first the paired slots of all but the last tail_bh of
    // them, then the q-tiles of those one by one, longest first across the
    // tail heads. The CUs that finish their last pair early take the long
    // single q-tiles, the last ones the short ones, so the XCD's CUs end
    // closer together than after a last round of equal pairs.
    const int x = L & 7, idx = L >> 3;
    const int bpx = (p.B * p.H) >> 3, t = p.tail_bh;
    const int n_pair = (bpx - t) * p.n_slots;
    WorkSlot ws;
    ws.split = 0;
    if (idx < n_pair) {
      const int hb = idx / p.n_slots;
      ws.bh = x * bpx + hb;
      ws.slot = idx - hb * p.n_slots;
      ws.single = -1;
    } else {
      const int k = idx - n_pair, r = k / t;
      ws.bh = x * bpx + (bpx - t) + (k - r * t);
      ws.slot = 0;
      ws.single = p.n_qtiles - 1 - r;
    }
    return ws;
  }
  const int w = (N & 7) == 0 ? (L & 7) * (N >> 3) + (L >> 3) : L;
  if (p.var_split > 0) {
    // Slot s is q-tile slot_qtile(s); the splits of the slots follow each
    // other within a (batch, head).
    WorkSlot ws;
    ws.single = -1;
    ws.bh = w / p.var_split;
    int r = w - ws.bh * p.var_split, slot = 0;
    for (; slot < p.n_qtiles - 1; ++slot) {
      const int c = qtile_splits(slot_qtile(p, slot), p.bm, p.bn, p.Sq, p.Sk, p.win_left,
                                 p.win_right, p.tiles_per_split);
      if (r < c) break;
      r -= c;
    }
    ws.slot = slot;
    ws.split = r;
    return ws;
  }
  const int per_bh = p.n_slots * p.num_splits;
  WorkSlot ws;
  ws.single = -1;
  ws.bh = w / per_bh;
  const int r = w - ws.bh * per_bh;
  ws.slot = r / p.num_splits;
  ws.split = r - ws.slot * p.num_splits;
  return ws;
}

// A slot runs q-tile n_qtiles-1-slot (the longest KV range first) and, in a
// paired launch, then q-tile `slot`: under a causal mask the two ranges add up
// to the same number of KV tiles for every slot, so all workgroups finish
// together instead of the last-dispatched long q-tiles trailing the launch.
// Windowed launches order a head's q-tiles differently: first the q-tiles
// whose window has its full length, in ascending order, so the workgroups
// resident on one XCD sweep neighbouring windows left to right together and
// each K/V tile comes from HBM about once (longest first, their windows drift
// apart and a head's K/V, 4 MB at 8192 x 128 bf16, is refetched several times
// through the XCD's 4 MB L2); then the shorter leading q-tiles (prefixes of
// the sequence, which share their first tiles anyway) in descending order,
// which fill the end of the launch as the longest-first order does.
__device__ __forceinline__ int slot_items(const FwdParams& p, const WorkSlot& ws) {
  return p.paired && ws.single < 0 && ws.slot < p.n_qtiles - 1 - ws.slot ? 2 : 1;
}

__device__ __forceinline__ WorkItem slot_item(const FwdParams& p, const WorkSlot& ws, int item) {
  WorkItem wi;
  wi.qt = ws.single >= 0 ? ws.single : (item == 0 ? slot_qtile(p, ws.slot) : ws.slot);
  wi.split = ws.split;
  wi.b = ws.bh / p.H;
  wi.h = ws.bh - wi.b * p.H;
  return wi;
}

// KV tile range [t_begin, t_end) (tiles of BN keys from kv_lo) for query rows
// [q0, q0 + BM).
template <int BM, int BN>
__device__ __forceinline__ void kv_range(const FwdParams& p, int q0, int split, int& kv_lo,
                                         int& t_begin, int& t_end) {
  const int q_last = min(q0 + BM, p.Sq) - 1;
  int lo = p.win_left >= 0 ? max(0, q0 - p.win_left) : 0;
  lo -= lo % BN;
  const int hi = p.win_right >= 0 ? min(p.Sk, q_last + p.win_right + 1) : p.Sk;
  const int n_tiles = hi > lo ? (hi - lo + BN - 1) / BN : 0;
  kv_lo = lo;
  t_begin = split * p.tiles_per_split;
  t_end = min(n_tiles, t_begin + p.tiles_per_split);
}

__device__ __forceinline__ bool kv_valid(const FwdParams& p, int q, int kv) {
  return kv < p.Sk && (p.win_right < 0 || kv <= q + p.win_right) &&
         (p.win_left < 0 || kv >= q - p.win_left);
}

// Per-wave classification of the tile [kv0, kv0 + BN) for rows [qa, qb].
template <int BN>
__device__ __forceinline__ void classify_tile(const FwdParams& p, int kv0, int qa, int qb,
                                              bool& skip, bool& full) {
  skip = kv0 >= p.Sk || (p.win_right >= 0 && kv0 > qb + p.win_right) ||
         (p.win_left >= 0 && kv0 + BN - 1 < qa - p.win_left);
  full = kv0 + BN <= p.Sk && (p.win_right < 0 || kv0 + BN - 1 <= qa + p.win_right) &&
         (p.win_left < 0 || kv0 >= qb - p.win_left);
}

// ---------------------------------------------------------------------------
// bf16 / f16 kernel: 32x32x16 MFMA.
//
// MFMA 32x32 register layouts used below (lane = j + 32*g, j in [0,32)):
//   A (32 x 16):  lane holds row j, 8 values of one k-group g;
//   B (16 x 32):  lane holds column j, 8 values of k-group g (same k-groups as A);
//   C (32 x 32):  element e of lane holds row 8*(e/4) + 4*g + e%4, column j.
// S^T = K Q^T: A row i of key block nb is LDS key row 32*nb + swap23(i) (bits 2
// and 3 of i exchanged); C element e then holds key 32*nb + 16*(e/8) + 8*g + e%8
// of query j, so elements 8h..8h+7 are 8 consecutive keys: exactly the B operand
// of the PV step over keys [16*(2nb+h), +16) with k-group g = keys +8g..+8g+7.
// ---------------------------------------------------------------------------
// LDS stage of the 16-bit kernel: BN K rows of stride D+8 (16-byte pad,
// conflict-free b128 reads) and D V^T rows of stride BN+8, in elements.
template <int D, int BN>
constexpr int fa16_stage_elems() {
  return BN * (D + 8) + D * (BN + 8);
}

// Query rows [32*NW*wi.qt, +32*NW) of one (batch, head) against its KV range.
// PAGED: K/V rows come from pools through the page table (prefill over a
// paged cache); invalid rows load as zeros and are masked.
// BIG (paged, pools of 4 GiB and more): page rows through 64-bit addresses.
template <int D, int BN, int NW, bool BF16, bool PAGED, bool DROP = false, bool BIG = false>
__device__ __forceinline__ void fa16_rows(const FwdParams& pin, const WorkItem wi,
                                          uint16_t* __restrict__ smem, int* __restrict__ pages) {
  FwdParams p = pin;
  if constexpr (PAGED) p.Sk = max(0, min(pin.ctx[wi.b], pin.max_blocks * pin.bs));
  constexpr int BM = 32 * NW, NT = 64 * NW;
  constexpr int KS = D + 8;   // K row stride (elements)
  constexpr int VS = BN + 8;  // V^T row stride (elements)
  constexpr int K_ELEMS = BN * KS, V_ELEMS = D * VS, STAGE = K_ELEMS + V_ELEMS;
  static_assert(STAGE == fa16_stage_elems<D, BN>(), "stage layout");
  constexpr int NB = BN / 32, NSL = BN / 16, NKS = D / 16, NDB = D / 32;
  constexpr int CPR = D / 8;  // 16-byte chunks per row
  constexpr int K_CHUNKS = BN * CPR;
  constexpr int K_PER_T = (K_CHUNKS + NT - 1) / NT;
  // V is staged as V^T in units of 2 keys x 8 dims (two 16-byte row chunks,
  // eight 4-byte transposed words).
  constexpr int V_UNITS = (BN / 2) * CPR;
  constexpr int V_PER_T = (V_UNITS + NT - 1) / NT;
  constexpr int VXM = BN / 8 - 1;  // XOR mask of the V^T layout, in 16-byte chunks
  static_assert(D % 32 == 0 && BN % 32 == 0 && BN <= 64, "tile shape");

  // The wave index is made an SGPR value so per-wave tile decisions (skip,
  // diagonal masking) compile to scalar branches.
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 31, g = lane >> 5;

  const int q0 = wi.qt * BM;
  int kv_lo, t_begin, t_end;
  kv_range<BM, BN>(p, q0, wi.split, kv_lo, t_begin, t_end);

  const uint16_t* __restrict__ Qp = (const uint16_t*)p.q + wi.b * p.q_sb + wi.h * p.q_sh;
  // K/V of this (batch, head) through buffer resources: SGPR base, 32-bit
  // offsets (the host guarantees Sk * seq_stride * 2 < 2^31, or for pools
  // pool_bytes < 2^32), no per-load address arithmetic. Paged: the record
  // count is the pool's extent, so an offset past it loads zeros.
  const int kvh = wi.h / p.kv_group;  // K/V head of this query head
  const int krec = PAGED ? (int)(p.pool_bytes - (uint32_t)(kvh * p.k_sh * 2)) : 0x7fffffff;
  const int vrec = PAGED ? (int)(p.pool_bytes - (uint32_t)(kvh * p.v_sh * 2)) : 0x7fffffff;
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const uint16_t*)p.k + wi.b * p.k_sb + kvh * p.k_sh), 0, krec, kBufferFlags);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const uint16_t*)p.v + wi.b * p.v_sb + kvh * p.v_sh), 0, vrec, kBufferFlags);
  constexpr int kNoRow = (int)0xFFFFFFF0u;  // beyond any pool: loads zeros

  // Paged: this item's slice of the page table, validated, in LDS.
  int pg_first = 0;
  if constexpr (PAGED) {
    const int kv_a = kv_lo + t_begin * BN, kv_b = min(kv_lo + t_end * BN, p.Sk);
    pg_first = page_of(p, kv_a);
    const int npg = kv_b > kv_a ? page_of(p, kv_b - 1) - pg_first + 1 : 0;
    const int32_t* row = p.bt + (int64_t)wi.b * p.max_blocks + pg_first;
    for (int i = tid; i < npg; i += NT) {
      const int blk = row[i];
      pages[i] = (blk >= 0 && blk < p.num_blocks) ? blk : -1;
    }
    __syncthreads();
  }
  // Byte offset of the 16-byte chunk `col` of key row `pos` (paged: through
  // the page table; missing rows -> kNoRow).
  // (32-bit arithmetic: the host guarantees pool_bytes < 2^32.)
  auto paged_off = [&](int pos, int col, uint32_t row_bytes) __attribute__((always_inline)) {
    uint32_t off = (uint32_t)kNoRow;
    if (pos < p.Sk) {
      const int pg = page_of(p, pos);
      const int page = pages[pg - pg_first];
      if (page >= 0)
        off = ((uint32_t)page * (uint32_t)p.bs + (uint32_t)(pos - pg * p.bs)) * row_bytes +
              (uint32_t)col * 16u;
    }
    return (int)off;
  };
  // BIG: the same chunk's 64-bit address (missing rows: kZeroChunk).
  const unsigned char* kbase = (const unsigned char*)p.k + (wi.b * p.k_sb + kvh * p.k_sh) * 2;
  const unsigned char* vbase = (const unsigned char*)p.v + (wi.b * p.v_sb + kvh * p.v_sh) * 2;
  auto paged_chunk = [&](const unsigned char* base, int pos, int col, uint32_t row_bytes)
                         __attribute__((always_inline)) -> u32x4 {
    const u32x4* a = &kZeroChunk;
    if (pos < p.Sk) {
      const int pg = page_of(p, pos);
      const int page = pages[pg - pg_first];
      if (page >= 0)
        a = (const u32x4*)(base +
                           ((uint64_t)(uint32_t)page * (uint32_t)p.bs + (uint32_t)(pos - pg * p.bs)) *
                               row_bytes +
                           (uint32_t)col * 16u);
    }
    return *a;
  };

  // Q^T as B operand, k-group g of 16-dim step ks = dims 16*ks + 8*g .. +8.
  // Rows past Sq read the last row (never stored).
  const int wq0 = q0 + wave * 32;
  const int myq = wq0 + j;
  // Dropout: this row's key of the keep-mask hash.
  const u32 drop_rk =
      DROP ? drop_row_key((u32)(((int64_t)wi.b * p.H + wi.h) * p.Sq + myq), p.seed0) : 0u;
  u32x4 qreg[NKS];
  {
    const u32x4* src = (const u32x4*)(Qp + (int64_t)min(myq, p.Sq - 1) * p.q_ss);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) qreg[ks] = src[2 * ks + g];
  }
  if (p.rope_cos) rope_q_frags<NKS, BF16>(p, p.rope_offset + min(myq, p.Sq - 1), g, qreg);
  if (p.neg) {
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) qreg[ks] ^= 0x80008000u;
  }
  // Drain Q now, so that the MFMAs reading qreg never wait on the K/V
  // prefetches issued inside the loop (vmcnt completes in order).
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)

  // Per-thread byte offsets of the prefetch loads inside a tile: one lane
  // offset each for K and V; load i of a thread sits NT/CPR rows further (a
  // wave-uniform step, passed as the scalar offset of the buffer load).
  static_assert(NT % CPR == 0, "whole rows per load round");
  constexpr int ROWS_PER_ROUND = NT / CPR;
  const int koff = (int)(((tid / CPR) * p.k_ss + (tid % CPR) * 8) * 2);
  const int kstep = ROWS_PER_ROUND * (int)p.k_ss * 2;
  // V unit u: row pair kp = u / CPR, 16-byte column chunk dq = u % CPR (a wave
  // reads whole rows); the second row of the pair is one seq stride further.
  const int voff = (int)(((2 * (tid / CPR)) * p.v_ss + (tid % CPR) * 8) * 2);
  const int vstep = 2 * ROWS_PER_ROUND * (int)p.v_ss * 2, vrow = (int)p.v_ss * 2;

  // Prefetch registers, two sets: tile i+2 is loaded into set i%2 while tile
  // i computes and tile i+1 (loaded one iteration earlier) is staged to LDS,
  // so a load has two tile times to arrive.
  // (The paged variant prefetches one tile ahead: its page lookups need the
  // registers of the second set.)
  // (D = 256: one set too, for registers)
  constexpr int NSET = (PAGED || D > 128) ? 1 : MPX_FA_DEPTH;
  u32x4 kbuf[NSET][K_PER_T];
  u32x4 vbuf[NSET][V_PER_T][2];
  // Rows of a staged tile at or past v_rows are zeroed when V is stored (BN
  // except for the tail tile).
  int v_rows[NSET];

  // The loads never depend on data (no selects): a select on a loaded value
  // would make the compiler wait for the prefetch right after issuing it.
  auto load_tile = [&](int kv0, auto SET) __attribute__((always_inline)) {
    constexpr int S = decltype(SET)::value;
    if constexpr (PAGED) {
      v_rows[S] = BN;  // missing rows already load as zeros
#pragma unroll
      for (int i = 0; i < K_PER_T; ++i) {
        const int c = tid + i * NT;
        if (K_CHUNKS % NT == 0 || c < K_CHUNKS) {
          if constexpr (BIG)
            kbuf[S][i] = paged_chunk(kbase, kv0 + c / CPR, c % CPR, (uint32_t)p.k_ss * 2u);
          else
            kbuf[S][i] = __builtin_amdgcn_raw_buffer_load_b128(
                krs, paged_off(kv0 + c / CPR, c % CPR, (uint32_t)p.k_ss * 2u), 0, 0);
        }
      }
#pragma unroll
      for (int i = 0; i < V_PER_T; ++i) {
        const int u = tid + i * NT;
        if (V_UNITS % NT == 0 || u < V_UNITS) {
          const int kp = u / CPR, dq = u % CPR;
#pragma unroll
          for (int r = 0; r < 2; ++r) {
            if constexpr (BIG)
              vbuf[S][i][r] = paged_chunk(vbase, kv0 + 2 * kp + r, dq, (uint32_t)p.v_ss * 2u);
            else
              vbuf[S][i][r] = __builtin_amdgcn_raw_buffer_load_b128(
                  vrs, paged_off(kv0 + 2 * kp + r, dq, (uint32_t)p.v_ss * 2u), 0, 0);
          }
        }
      }
      return;
    }
    const int kso = kv0 * (int)p.k_ss * 2, vso = kv0 * (int)p.v_ss * 2;
    if (kv0 + BN <= p.Sk) {
      v_rows[S] = BN;
#pragma unroll
      for (int i = 0; i < K_PER_T; ++i)
        if (K_CHUNKS % NT == 0 || tid + i * NT < K_CHUNKS)
          kbuf[S][i] = __builtin_amdgcn_raw_buffer_load_b128(krs, koff, kso + i * kstep, 0);
#pragma unroll
      for (int i = 0; i < V_PER_T; ++i)
        if (V_UNITS % NT == 0 || tid + i * NT < V_UNITS) {
          vbuf[S][i][0] = __builtin_amdgcn_raw_buffer_load_b128(vrs, voff, vso + i * vstep, 0);
          vbuf[S][i][1] =
              __builtin_amdgcn_raw_buffer_load_b128(vrs, voff, vso + i * vstep + vrow, 0);
        }
    } else {
      // Tail tile: rows past Sk re-read the last valid row (K rows there are
      // masked; V rows are zeroed at store time).
      asm volatile("" ::: "memory");
      v_rows[S] = p.Sk - kv0;
      const int lim = p.Sk - 1 - kv0;
#pragma unroll
      for (int i = 0; i < K_PER_T; ++i) {
        const int c = tid + i * NT;
        if (K_CHUNKS % NT == 0 || c < K_CHUNKS) {
          const int row = min(c / CPR, lim), col = c - (c / CPR) * CPR;
          kbuf[S][i] = __builtin_amdgcn_raw_buffer_load_b128(
              krs, (row * (int)p.k_ss + col * 8) * 2, kso, 0);
        }
      }
#pragma unroll
      for (int i = 0; i < V_PER_T; ++i) {
        const int u = tid + i * NT;
        if (V_UNITS % NT == 0 || u < V_UNITS) {
          const int kp = u / CPR, dq = u - (u / CPR) * CPR;
#pragma unroll
          for (int r = 0; r < 2; ++r)
            vbuf[S][i][r] = __builtin_amdgcn_raw_buffer_load_b128(
                vrs, (min(2 * kp + r, lim) * (int)p.v_ss + dq * 8) * 2, vso, 0);
        }
      }
    }
  };

  // V^T layout: element (d, kv) sits in 4-byte word (kv/2) ^ (4 * ((d/16) & VXM))
  // of row d. The XOR keeps 16-byte groups of 8 keys intact for the b128
  // operand reads and spreads one store instruction over all 64 banks.
  // Register set S is staged into LDS stage `stage`.
  auto store_tile = [&](auto SET, int stage) __attribute__((always_inline)) {
    constexpr int S = decltype(SET)::value;
    uint16_t* Ks = smem + stage * STAGE;
    uint16_t* Vt = Ks + K_ELEMS;
#pragma unroll
    for (int i = 0; i < K_PER_T; ++i) {
      const int c = tid + i * NT;
      if (K_CHUNKS % NT == 0 || c < K_CHUNKS) {
        const int row = c / CPR, col = c - (c / CPR) * CPR;
        *(u32x4*)(Ks + row * KS + col * 8) = kbuf[S][i];
      }
    }
    if (v_rows[S] < BN) {
      asm volatile("" ::: "memory");
#pragma unroll
      for (int i = 0; i < V_PER_T; ++i) {
        const int kp = (tid + i * NT) / CPR;
#pragma unroll
        for (int r = 0; r < 2; ++r)
          if (2 * kp + r >= v_rows[S]) vbuf[S][i][r] = (u32x4){0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int i = 0; i < V_PER_T; ++i) {
      const int u = tid + i * NT;
      if (V_UNITS % NT == 0 || u < V_UNITS) {
        const int kp = u / CPR, dq = u - (u / CPR) * CPR;
        const int word = kp ^ (4 * ((dq >> 1) & VXM));
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const u32 r0 = vbuf[S][i][0][jj], r1 = vbuf[S][i][1][jj];
          const int d = dq * 8 + 2 * jj;
          *(u32*)(Vt + d * VS + 2 * word) = __builtin_amdgcn_perm(r1, r0, 0x05040100u);
          *(u32*)(Vt + (d + 1) * VS + 2 * word) = __builtin_amdgcn_perm(r1, r0, 0x07060302u);
        }
      }
    }
  };

  f32x16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = (f32x16){};
  float m_run = -INFINITY;  // reference point of o and l_run (log2 units)
  float m_max = -INFINITY;  // true running max (log2 units)
  float l_run = 0.f;        // this lane's half of the row sum
  const float c = p.c;

  const int krow_perm = (j & ~12) | ((j & 4) << 1) | ((j & 8) >> 1);
  // Visible keys of this lane's query row: [kv_first, kv_last].
  const int kv_first = p.win_left >= 0 ? myq - p.win_left : -(1 << 30);
  const int kv_last = min(p.win_right >= 0 ? myq + p.win_right : (1 << 30), p.Sk - 1);
  // V^T operand of lane (j, g) for dims 32*db + j and keys 16*sl + 8*g .. +8:
  // chunk (2*sl + g) ^ ((2*db + j/16) & VXM) = 2*(sl ^ (db & VXM/2)) + (g ^ j/16),
  // so one lane base plus compile-time offsets addresses every operand.
  const int vlane = j * (VS / 8) + (g ^ ((j >> 4) & 1));
  // Paged: validity of the tile's keys (bit r = key kv0 + r) and the ALiBi
  // slope divided by |scale| (the bias is added to raw scores). The bias
  // slope * (kv - q) is applied as slope * (kv - kv_last): the two differ by a
  // per-row constant, which softmax ignores, and the second is small for the
  // keys that carry the weight, so its float32 rounding stays small when the
  // context is much longer than the query range.
  uint64_t vmask = ~0ull;
  const float alibi = (PAGED && p.slopes) ? p.slopes[wi.h] * kLog2e / p.c : 0.f;

  // Scores S^T of this wave's rows against the K tile staged at Ks.
  auto qk_tile = [&](const uint16_t* Ks, f32x16 (&s)[NB]) __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const u32x4* kp = (const u32x4*)(Ks + (nb * 32 + krow_perm) * KS) + g;
      u32x4 ka[NKS];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) ka[ks] = kp[2 * ks];
      s[nb] = (f32x16){};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) s[nb] = mfma32x32x16<BF16>(ka[ks], qreg[ks], s[nb]);
    }
#if MPX_FA_SCHED >= 1
    // Keep the K operand reads of block nb+1 in flight under the MFMAs of block nb.
    __builtin_amdgcn_sched_group_barrier(0x100, NKS, 0);
#pragma unroll
    for (int i = 0; i < NKS * (NB - 1); ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, NKS, 0);
#endif
  };

  // Masks and online softmax of the tile at kv0: P^T (packed 16-bit) in pop.
  auto softmax_p = [&](int kv0, bool full, f32x16 (&s)[NB], u32x4 (&pop)[NSL])
      __attribute__((always_inline)) {
    if (!full) {
      // The empty volatile asm keeps this a real (scalar) branch: without it
      // the selects are folded into unconditional code run on every tile.
      asm volatile("" ::: "memory");
      // Paged: this lane's keys are kv0 + 8g + (compile-time offset).
      const uint64_t vm = PAGED ? vmask >> (8 * g) : 0;
      const float dq0 = PAGED ? (float)(kv0 + 8 * g - kv_last) : 0.f;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int kc = nb * 32 + 16 * (e >> 3) + (e & 7);
          const int kv = kv0 + kc + 8 * g;
          bool ok = (kv >= kv_first) & (kv <= kv_last);
          float sv = s[nb][e];
          if constexpr (PAGED) {
            ok = ok & (((vm >> kc) & 1ull) != 0);
            sv += alibi * (dq0 + (float)kc);
          }
          s[nb][e] = ok ? sv : -INFINITY;
        }
    }

    float mt = -INFINITY;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int e = 0; e < 16; ++e) mt = fmaxf(mt, s[nb][e]);
    mt = pair_max32(mt) * c;
    m_max = fmaxf(m_max, mt);

    if (__any(mt > m_run + kRescaleThreshold)) {
      asm volatile("" ::: "memory");  // a real branch, not selects on all of o
      const float m_new = fmaxf(m_run, mt);
      const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[db][e] *= alpha;
      m_run = m_new;
    }
    const float msub = m_run == -INFINITY ? 0.f : m_run;

    // P = exp2(s*c - m), packed to 16 bits; the row sum accumulates the
    // packed (rounded) weights, the exact weights the PV product uses.
    // Dropout: the PV operand keeps the kept keys' weights only (the row sum
    // takes them all); element pair e2 of half hh of block nb holds keys
    // kv0 + 32 nb + 16 hh + 8 g + 2 e2 + {0, 1}, the hash's key pair
    // kv0 / 2 + 16 nb + 8 hh + 4 g + e2.
    const u32 pair0 = DROP ? drop_pair_key((u32)(kv0 >> 1) + 4u * g, p.seed1) : 0u;
    float lsum = 0.f;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          const float x0 = fast_exp2(s[nb][8 * hh + 2 * e2] * c - msub);
          const float x1 = fast_exp2(s[nb][8 * hh + 2 * e2 + 1] * c - msub);
          const u32 pk = pack2<BF16>(x0, x1);
          if constexpr (DROP)
            pop[2 * nb + hh][e2] =
                pk & drop_mask2(drop_bits(drop_rk, pair0 + (u32)(16 * nb + 8 * hh + e2) *
                                                               0x85EBCA77u),
                                p.drop_thresh);
          else
            pop[2 * nb + hh][e2] = pk;
          lsum = dot2_sum<BF16>(pk, lsum);
        }
    l_run += lsum;
  };

  // O += P V for the V^T tile staged at Vt.
  auto pv_tile = [&](const uint16_t* Vt, const u32x4 (&pop)[NSL]) __attribute__((always_inline)) {
    const u32x4* vp = (const u32x4*)Vt + vlane;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      u32x4 va[NSL];
#pragma unroll
      for (int sl = 0; sl < NSL; ++sl)
        va[sl] = vp[db * 32 * (VS / 8) + 2 * (sl ^ (db & (VXM >> 1)))];
#pragma unroll
      for (int sl = 0; sl < NSL; ++sl) o[db] = mfma32x32x16<BF16>(va[sl], pop[sl], o[db]);
    }
#if MPX_FA_SCHED >= 2
    __builtin_amdgcn_sched_group_barrier(0x100, NSL, 1);
#pragma unroll
    for (int i = 0; i < NSL * (NDB - 1); ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, NSL, 1);
#endif
  };

  auto softmax_pv = [&](const uint16_t* Vt, int kv0, bool full, f32x16 (&s)[NB])
      __attribute__((always_inline)) {
    u32x4 pop[NSL];
    softmax_p(kv0, full, s, pop);
    pv_tile(Vt, pop);
  };


  // Attention of this wave's rows to the tile at kv0 staged in LDS stage `stage`.
  auto compute_tile = [&](int stage, int kv0) __attribute__((always_inline)) {
    bool skip, full;
    classify_tile<BN>(p, kv0, wq0, wq0 + 31, skip, full);
    if (skip) return;
    if constexpr (PAGED) {
      const int key = kv0 + (lane % BN);
      bool ok = key < p.Sk;
      if (ok) ok = pages[page_of(p, key) - pg_first] >= 0;
      vmask = __ballot(ok);
      if (BN < 64) vmask &= (1ull << BN) - 1;
      if (vmask != (BN < 64 ? (1ull << BN) - 1 : ~0ull) || alibi != 0.f) full = false;
    }
    const uint16_t* Ks = smem + stage * STAGE;
    f32x16 s[NB];
    qk_tile(Ks, s);
    softmax_pv(Ks + K_ELEMS, kv0, full, s);
  };

  const int n_tiles = t_end - t_begin;
  if (n_tiles > 0) {
    load_tile(kv_lo + t_begin * BN, Const<0>{});
    store_tile(Const<0>{}, 0);
    if (NSET == 2 && n_tiles > 1) load_tile(kv_lo + (t_begin + 1) * BN, Const<NSET - 1>{});
  }
  __syncthreads();

  // Tile i: computed from stage i%2; tile i+2 loaded into register set i%2;
  // tile i+1 staged from register set (i+1)%2 into stage (i+1)%2.
  auto step = [&](int i, auto PAR) __attribute__((always_inline)) {
    constexpr int P = decltype(PAR)::value;
    const int kv0 = kv_lo + (t_begin + i) * BN;
    if constexpr (NSET == 2) {
      if (i + 2 < n_tiles) load_tile(kv0 + 2 * BN, Const<P>{});
    } else {
      if (i + 1 < n_tiles) load_tile(kv0 + BN, Const<0>{});
    }
    compute_tile(P, kv0);
    if (i + 1 < n_tiles) store_tile(Const<NSET == 2 ? 1 - P : 0>{}, 1 - P);
    __syncthreads();
  };
  for (int i = 0; i < n_tiles; i += 2) {
    step(i, Const<0>{});
    if (i + 1 < n_tiles) step(i + 1, Const<1>{});
  }

  // Epilogue: move o and l to the true max, then normalise (or emit partials).
  const float l_tot = pair_sum32(l_run);
  const float f = m_max == -INFINITY ? 0.f : fast_exp2(m_run - m_max);
  // (dropout: kept weights times 1 / (1 - p); the row sums stay unscaled)
  const float fo = DROP ? f * p.drop_scale : f;
  if (p.num_splits == 1) {
    if (myq < p.Sq) {
      const float inv = m_max == -INFINITY ? (p.nan_empty ? __builtin_nanf("") : 0.f)
                                           : fo / (l_tot * f + p.eps);
      if (p.lse && g == 0)
        p.lse[((int64_t)wi.b * p.H + wi.h) * p.Sq + myq] =
            m_max == -INFINITY ? INFINITY : m_max + log2f(l_tot * f + p.eps);
      uint16_t* Op = (uint16_t*)p.o + wi.b * p.o_sb + wi.h * p.o_sh + (int64_t)myq * p.o_ss;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
          const int d = db * 32 + 8 * e4 + 4 * g;
          const u32x2 val = {pack2<BF16>(o[db][4 * e4] * inv, o[db][4 * e4 + 1] * inv),
                             pack2<BF16>(o[db][4 * e4 + 2] * inv, o[db][4 * e4 + 3] * inv)};
          *(u32x2*)(Op + d) = val;
        }
    }
  } else if (myq < p.Sq) {
    const int64_t row = (((int64_t)wi.split * p.B + wi.b) * p.H + wi.h) * p.Sq + myq;
    float* wo = p.ws_o + row * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int d = db * 32 + 8 * e4 + 4 * g;
        *(f32x4*)(wo + d) = (f32x4){o[db][4 * e4] * fo, o[db][4 * e4 + 1] * fo,
                                    o[db][4 * e4 + 2] * fo, o[db][4 * e4 + 3] * fo};
      }
    if (g == 0) {
      p.ws_ml[2 * row] = m_max;
      p.ws_ml[2 * row + 1] = l_tot * f;
    }
  }
}

// ---------------------------------------------------------------------------
// D = 128 / 64 with direct global->LDS staging (gfx950 LDS DMA): the K and V
// tiles (BN = 128 keys by default, 64 for the paged kernels) go from HBM/L2
// straight into LDS with buffer_load ... lds, without passing through
// registers; NST LDS stages hold tile i (computing) and tiles i+1 .. i+NST-1
// (landed or in flight): two stages at D = 128 with 128-key tiles (128 KB),
// four at D = 64.
//
// LDS rows are 256 bytes (D = 128), unpadded (a DMA instruction writes 64 consecutive
// 16-byte slots), so bank conflicts are avoided by XOR-swizzling 16-byte
// chunks instead:
//   K row r: chunk c stored at slot c ^ (r & 15)      (QK operand reads:
//            16 lanes read 16 different rows at one logical chunk);
//   V row r: chunk c stored at slot c ^ (4 * (r & 3)) (PV operand reads:
//            ds_read_b64_tr_b16 takes 4 rows x 64 bytes per 32 lanes).
// V stays row-major: the transposing LDS read delivers V^T operands. For a
// group of 16 lanes whose lane s addresses row base + s/4, columns
// c0 + 4*(s%4) .. +3, lane s receives column c0 + s of rows base .. base + 3.
// ---------------------------------------------------------------------------
// Offset of a key row without a page: past any pool the host accepts, so its
// buffer loads return zeros.
constexpr u32 kNoRowDirect = 0xFFFFFF00u;


// PAGED: K/V rows come from the pools through this item's page-table slice,
// staged in LDS (pages); each lane's DMA offset is its row's (page, slot), and
// a row without a page gets an offset past the pool, which the buffer range
// check turns into zeros; those keys are masked.
// Swizzle of the D = 64 direct tiles (128-byte rows, 8 chunks): chunk c of row
// r sits at slot c ^ swz64(r), conflict-free both for 16 lanes reading one
// chunk of 16 consecutive rows (K operands) and for the transposing read of 4
// consecutive rows x 4 consecutive chunks (V^T operands).
__device__ __forceinline__ int swz64(int r) { return (((r >> 1) & 1) << 2) | ((r >> 2) & 3); }

// BIG (paged, pools of 4 GiB and more): the page rows are read by the DMA's
// 64-bit address form (rows without a page from kZeroChunk) instead of 32-bit
// buffer offsets.
template <int D, int BN, int NW, bool BF16, int NST, bool PAGED, bool DROP = false,
          bool BIG = false>
__device__ __forceinline__ void fa16_rows_direct(const FwdParams& pin, const WorkItem wi,
                                                 unsigned char* __restrict__ st0,
                                                 unsigned char* __restrict__ st1,
                                                 unsigned char* __restrict__ st2,
                                                 unsigned char* __restrict__ st3,
                                                 int* __restrict__ pages) {
  constexpr int BM = 32 * NW;
  constexpr int NB = BN / 32, NSL = BN / 16, NKS = D / 16, NDB = D / 32;
  // Paged, 64-key tiles: the item's page ids are staged in LDS (any page
  // size, ALiBi). Paged, 128-key tiles: page ids come from the block table,
  // one per DMA instruction of a wave; the host picks this form for
  // power-of-two page sizes of at least RPD tokens (so the RPD rows one wave's
  // instruction stages lie in one page) and no ALiBi. A tile with a page that
  // is missing (-1) or past the pool has each key checked against the table.
  constexpr bool kSlice = PAGED && BN == 64;
  constexpr bool kScalarPages = PAGED && BN == 128;
  constexpr bool kChecked = kScalarPages;
  static_assert(!PAGED || kSlice || kScalarPages, "paged tiles are 64 or 128 keys");
  constexpr int ROWB = 2 * D;          // bytes per K or V row
  constexpr int KBYTES = BN * ROWB;    // one K (or V) tile
  constexpr int STAGEB = 2 * KBYTES;   // K then V
  constexpr int RPD = 1024 / ROWB;     // rows per DMA instruction (64 lanes x 16 bytes)
  constexpr int RSTEP = RPD * NW;      // rows one DMA instruction of every wave covers
  constexpr int NDMA = BN / RSTEP;     // DMA instructions per wave per K (or V) tile
  static_assert((NW == 8 || NW == 4) && (D == 128 || D == 64 || (D == 256 && NW == 4)) &&
                    NDMA * RSTEP == BN,
                "each wave stages rows RPD*wave .. +RPD-1, +RSTEP, ...");
  // The row swizzles depend on row bits below RSTEP only (bits 0-3 at D = 128,
  // 1-3 at D = 64), so every DMA instruction of a lane uses the same chunk. At
  // D = 256 (RSTEP = 8) the K swizzle takes bits 0-3: a lane's rows of even and
  // odd instructions differ in bit 3, and each kind has its own chunk.
  static_assert(RSTEP % 16 == 0 || D == 256, "swizzle period");
  static_assert((NST - 2) * 2 * NDMA <= 15, "vmcnt immediate");
  // Paged: keys exist up to this sequence's context length.
  FwdParams p = pin;
  if constexpr (PAGED) p.Sk = max(0, min(pin.ctx[wi.b], pin.max_blocks * pin.bs));

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 31, g = lane >> 5;

  const int q0 = wi.qt * BM;
  int kv_lo, t_begin, t_end;
  kv_range<BM, BN>(p, q0, wi.split, kv_lo, t_begin, t_end);

  const uint16_t* __restrict__ Qp = (const uint16_t*)p.q + wi.b * p.q_sb + wi.h * p.q_sh;
  // Paged: the record count is the pool's extent past this head's offset.
  const int kvh = wi.h / p.kv_group;  // K/V head of this query head
  const u32 krec = PAGED ? p.pool_bytes - (u32)(kvh * p.k_sh * 2) : 0x7fffffffu;
  const u32 vrec = PAGED ? p.pool_bytes - (u32)(kvh * p.v_sh * 2) : 0x7fffffffu;
  const u32x4 krs = buffer_desc((const uint16_t*)p.k + wi.b * p.k_sb + kvh * p.k_sh, krec);
  const u32x4 vrs = buffer_desc((const uint16_t*)p.v + wi.b * p.v_sb + kvh * p.v_sh, vrec);
  // BIG: the same bases for 64-bit addresses.
  const unsigned char* kbase = (const unsigned char*)p.k + (wi.b * p.k_sb + kvh * p.k_sh) * 2;
  const unsigned char* vbase = (const unsigned char*)p.v + (wi.b * p.v_sb + kvh * p.v_sh) * 2;
  static_assert(!BIG || PAGED, "64-bit DMA addressing is for paged pools");

  // Paged: this item's slice of the page table, validated, in LDS.
  int pg_first = 0;
  const int32_t* __restrict__ bt_row = PAGED ? p.bt + (int64_t)wi.b * p.max_blocks : nullptr;
  if constexpr (kSlice) {
    const int kv_a = kv_lo + t_begin * BN, kv_b = min(kv_lo + t_end * BN, p.Sk);
    pg_first = page_of(p, kv_a);
    const int npg = kv_b > kv_a ? page_of(p, kv_b - 1) - pg_first + 1 : 0;
    const int32_t* row = p.bt + (int64_t)wi.b * p.max_blocks + pg_first;
    for (int i = tid; i < npg; i += 64 * NW) {
      const int blk = row[i];
      pages[i] = (blk >= 0 && blk < p.num_blocks) ? blk : -1;
    }
    __syncthreads();
  }

  const int wq0 = q0 + wave * 32;
  const int myq = wq0 + j;
  // Dropout: this row's key of the keep-mask hash.
  const u32 drop_rk =
      DROP ? drop_row_key((u32)(((int64_t)wi.b * p.H + wi.h) * p.Sq + myq), p.seed0) : 0u;
  u32x4 qreg[NKS];
  {
    const u32x4* src = (const u32x4*)(Qp + (int64_t)min(myq, p.Sq - 1) * p.q_ss);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) qreg[ks] = src[2 * ks + g];
  }
  if (p.rope_cos) rope_q_frags<NKS, BF16>(p, p.rope_offset + min(myq, p.Sq - 1), g, qreg);
  // Q times the signed softmax scale in log2 units, rounded to the storage
  // type: Q K^T then comes out of the MFMAs in log2 units, and with the
  // accumulators started at -m (below) it is already the exponent.
  {
    const float cq = p.neg ? -p.c : p.c;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const u32 x = qreg[ks][w];
        qreg[ks][w] = pack2<BF16>(h2f<BF16>((uint16_t)(x & 0xffffu)) * cq,
                                  h2f<BF16>((uint16_t)(x >> 16)) * cq);
      }
  }
  // Q has landed (and the previous item's stores retired) before any tile
  // DMA, so the explicit vmcnt waits below count tile loads only.
  __builtin_amdgcn_s_waitcnt(0x0F70);

  // DMA lane mapping: this wave's first instruction fills LDS rows
  // RPD*wave .. +RPD-1 (lane -> row lr, slot lane % (ROWB/16)); instruction r
  // fills rows lr + RSTEP*r.
  int lr, kchunk, vchunk, kchunk_odd = 0;
  if constexpr (D == 128) {
    lr = 4 * wave + (lane >> 4);
    kchunk = (lane & 15) ^ (lr & 15);
    vchunk = (lane & 15) ^ (4 * (lr & 3));
  } else if constexpr (D == 256) {
    // 512-byte rows, two per instruction: instruction r fills rows lr + 8 r,
    // lr < 8; K row r has chunk c at slot c ^ (r & 15), V row r at c ^ 4 (r & 3).
    lr = 2 * wave + (lane >> 5);
    kchunk = (lane & 31) ^ lr;
    kchunk_odd = (lane & 31) ^ (lr + 8);
    vchunk = (lane & 31) ^ (4 * (lr & 3));
  } else {
    lr = 8 * wave + (lane >> 3);
    kchunk = vchunk = (lane & 7) ^ swz64(lr);
  }
  const int kgo = (lr * (int)p.k_ss + kchunk * 8) * 2;
  const int kgo_odd = (lr * (int)p.k_ss + kchunk_odd * 8) * 2;  // (D = 256)
  // Paged, 128-key tiles: the lane part of a DMA offset (row lr % RPD of the
  // instruction's RPD rows, this lane's chunk).
  const int klane = ((lr % RPD) * (int)p.k_ss + kchunk * 8) * 2;
  const int vlane = ((lr % RPD) * (int)p.v_ss + vchunk * 8) * 2;
  const int vgo = (lr * (int)p.v_ss + vchunk * 8) * 2;
  const int kstep = RSTEP * (int)p.k_ss * 2, vstep = RSTEP * (int)p.v_ss * 2;
  auto stage_ptr = [&](auto ST) __attribute__((always_inline)) -> unsigned char* {
    constexpr int S = decltype(ST)::value;
    return S == 0 ? st0 : (S == 1 ? st1 : (S == 2 ? st2 : st3));
  };
  // Paged, 128-key tiles: lane l of pg_cur holds the table entry of page l of
  // the next tile to stage, counted from the page of its first key (a tile
  // spans max(1, 128 / page size) pages; lanes past the context read the last
  // page's entry). A step issues the next tile's DMAs, then loads the entries
  // of the tile after it, which land under the step's compute and are waited
  // for by its closing vmcnt(0) (two stages); pg_cur is read only after that.
  // tile_ok_next / tile_ok: every page a key of the staged / computed tile
  // lies in is valid (else compute_tile checks each key against the table).
  static_assert(!kScalarPages || NST == 2, "paged 128-key tiles use two stages");
  int pg_idx[NDMA];
  u32 pg_in[NDMA];
  if constexpr (kScalarPages) {
#pragma unroll
    for (int r = 0; r < NDMA; ++r) {
      const int row = RPD * wave + RSTEP * r;  // row of the tile instruction r starts at
      pg_idx[r] = row >> p.bs_log2;
      pg_in[r] = (u32)(row & ((1 << p.bs_log2) - 1)) * (u32)p.k_ss * 2u;
    }
  }
  int pg_cur = 0;
  bool tile_ok = true, tile_ok_next = true;
  auto fetch_pages = [&](int kv0) __attribute__((always_inline)) {
    const int last = (p.Sk - 1) >> p.bs_log2;
    pg_cur = bt_row[min((kv0 >> p.bs_log2) + lane, last)];
  };
  auto load_tile = [&](int kv0, unsigned char* stbase) __attribute__((always_inline)) {
    const u32 kdst = lds_addr(stbase + wave * RPD * ROWB);
    const u32 vdst = kdst + KBYTES;
    if constexpr (kScalarPages) {
      // Row lr + RSTEP * r of the tile sits in page pg_next[r] (32-bit
      // offsets: the host keeps each pool below 4 GiB - 256 bytes).
      const u32 row_bytes = (u32)p.k_ss * 2u;
      const int bmask = (1 << p.bs_log2) - 1;
      const int pg0 = kv0 >> p.bs_log2;
      if constexpr (kChecked) {
        // Pages of the tile's keys below the context length: lanes 0 .. npg-1.
        const int npg = ((min(kv0 + BN, p.Sk) - 1) >> p.bs_log2) - pg0 + 1;
        tile_ok_next = !__any((lane < npg) & ((pg_cur < 0) | (pg_cur >= p.num_blocks)));
      }
      if ((!kChecked || tile_ok_next) && kv0 + BN <= p.Sk) {
        // Every row exists: the page part of the offset is uniform (row
        // RPD * wave + RSTEP * r of the tile, in the scalar offset); the lane
        // part (row lr % RPD, chunk) is fixed. The tile starts on a page
        // boundary, so instruction r reads page entry pg_idx[r] at in-page
        // byte offset pg_in[r], both fixed for the kernel.
        if constexpr (BIG) {
          // The page base of instruction r in 64 bits, in scalar registers.
          const uint64_t page_bytes = (uint64_t)row_bytes << p.bs_log2;
#pragma unroll
          for (int r = 0; r < NDMA; ++r) {
            const u32 page = (u32)__builtin_amdgcn_readlane(pg_cur, pg_idx[r]);
            const uint64_t off = (uint64_t)page * page_bytes + pg_in[r];
            dma16_global_s(kdst + r * RSTEP * ROWB, kbase + off, (u32)klane);
            dma16_global_s(vdst + r * RSTEP * ROWB, vbase + off, (u32)vlane);
          }
          return;
        }
        const u32 pg_bytes = (u32)pg_cur * (row_bytes << p.bs_log2);
#pragma unroll
        for (int r = 0; r < NDMA; ++r) {
          const u32 soff = __builtin_amdgcn_readlane(pg_bytes, pg_idx[r]) + pg_in[r];
          dma16(krs, kdst + r * RSTEP * ROWB, klane, (int)soff);
          dma16(vrs, vdst + r * RSTEP * ROWB, vlane, (int)soff);
        }
        return;
      }
#pragma unroll
      for (int r = 0; r < NDMA; ++r) {
        const int page = __builtin_amdgcn_readlane(
            pg_cur, ((kv0 + RPD * wave + RSTEP * r) >> p.bs_log2) - pg0);
        const int pos = kv0 + lr + RSTEP * r;
        const bool ok = pos < p.Sk && page >= 0 && page < p.num_blocks;
        if constexpr (BIG) {
          const uint64_t base =
              ((uint64_t)((u32)page << p.bs_log2) + (u32)(pos & bmask)) * row_bytes;
          dma16_global(kdst + r * RSTEP * ROWB,
                       ok ? (const void*)(kbase + base + (u32)kchunk * 16u) : &kZeroChunk);
          dma16_global(vdst + r * RSTEP * ROWB,
                       ok ? (const void*)(vbase + base + (u32)vchunk * 16u) : &kZeroChunk);
          continue;
        }
        const u32 base = (((u32)page << p.bs_log2) + (u32)(pos & bmask)) * row_bytes;
        dma16(krs, kdst + r * RSTEP * ROWB, (int)(ok ? base + (u32)kchunk * 16u : kNoRowDirect),
              0);
        dma16(vrs, vdst + r * RSTEP * ROWB, (int)(ok ? base + (u32)vchunk * 16u : kNoRowDirect),
              0);
      }
      return;
    }
    if constexpr (PAGED) {
      // Rows lr (and lr + 32) through the page table (32-bit offsets: the
      // host keeps each pool below 4 GiB - 256 bytes).
      const u32 row_bytes = (u32)p.k_ss * 2u;
#pragma unroll
      for (int r = 0; r < NDMA; ++r) {
        const int pos = kv0 + lr + RSTEP * r;
        if constexpr (BIG) {
          const void* ka = &kZeroChunk;
          const void* va = &kZeroChunk;
          if (pos < p.Sk) {
            const int pg = page_of(p, pos);
            const int page = pages[pg - pg_first];
            if (page >= 0) {
              const uint64_t base =
                  ((uint64_t)(u32)page * (u32)p.bs + (u32)(pos - pg * p.bs)) * row_bytes;
              ka = kbase + base + (u32)kchunk * 16u;
              va = vbase + base + (u32)vchunk * 16u;
            }
          }
          dma16_global(kdst + r * RSTEP * ROWB, ka);
          dma16_global(vdst + r * RSTEP * ROWB, va);
          continue;
        }
        u32 koff = kNoRowDirect, voff = kNoRowDirect;
        if (pos < p.Sk) {
          const int pg = page_of(p, pos);
          const int page = pages[pg - pg_first];
          if (page >= 0) {
            const u32 base = ((u32)page * (u32)p.bs + (u32)(pos - pg * p.bs)) * row_bytes;
            koff = base + (u32)kchunk * 16u;
            voff = base + (u32)vchunk * 16u;
          }
        }
        dma16(krs, kdst + r * RSTEP * ROWB, (int)koff, 0);
        dma16(vrs, vdst + r * RSTEP * ROWB, (int)voff, 0);
      }
      return;
    }
    const int kso = kv0 * (int)p.k_ss * 2, vso = kv0 * (int)p.v_ss * 2;
    if (kv0 + BN <= p.Sk) {
#pragma unroll
      for (int r = 0; r < NDMA; ++r)
        dma16(krs, kdst + r * RSTEP * ROWB, (D == 256 && (r & 1)) ? kgo_odd : kgo,
              kso + r * kstep);
#pragma unroll
      for (int r = 0; r < NDMA; ++r) dma16(vrs, vdst + r * RSTEP * ROWB, vgo, vso + r * vstep);
    } else {
      // Tail tile: rows past Sk re-read the last valid row (their scores are
      // masked, so their weights are exactly 0).
      const int lim = p.Sk - 1 - kv0;
#pragma unroll
      for (int r = 0; r < NDMA; ++r) {
        const int row = min(lr + RSTEP * r, lim);
        const int kc = (D == 256 && (r & 1)) ? kchunk_odd : kchunk;
        dma16(krs, kdst + r * RSTEP * ROWB, (row * (int)p.k_ss + kc * 8) * 2, kso);
        dma16(vrs, vdst + r * RSTEP * ROWB, (row * (int)p.v_ss + vchunk * 8) * 2, vso);
      }
    }
  };

  // QK operand (A = K rows) of lane (j, g): row nb*32 + krow_perm, logical
  // chunk 2*ks + g, stored at slot (2*ks + g) ^ (row & 15).
  const int krow_perm = (j & ~12) | ((j & 4) << 1) | ((j & 8) >> 1);
  const int ky = D >= 128 ? krow_perm & 15 : swz64(krow_perm);
  int kaddr[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks)
    kaddr[ks] = krow_perm * ROWB + 32 * (ks ^ (ky >> 1)) + 16 * (g ^ (ky & 1));
  // PV operand (A = V^T) of lane L = j + 32g: rows 16*sl + 8g + 4h + s/4,
  // columns 32*db + 16*(L/16 % 2) + 4*(s%4) of the transposing read, s = L%16.
  const int s16 = lane & 15;
  int vaddr[NDB], vaddr_hi[NDB];  // rows +16 sl (lo), +16 sl + 4 (hi)
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    if constexpr (D >= 128) {
      vaddr[db] = (8 * g + (s16 >> 2)) * ROWB + 64 * (db ^ (s16 >> 2)) +
                  32 * ((lane >> 4) & 1) + 8 * (s16 & 3);
      vaddr_hi[db] = vaddr[db] + 4 * ROWB;
    } else {
      // the swizzle of D = 64 depends on bit 2 of the row, so hi is not lo + 4 rows
      const int chunk = 4 * db + 2 * ((lane >> 4) & 1) + ((s16 & 3) >> 1);
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int r = 8 * g + 4 * hf + (s16 >> 2);
        (hf ? vaddr_hi : vaddr)[db] = r * ROWB + 16 * (chunk ^ swz64(r)) + 8 * (s16 & 1);
      }
    }
  }

  f32x16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = (f32x16){};
  // m_run: reference point of o and l_run (log2 units); the S^T accumulators
  // start at -m_run (negm), so a tile's scores arrive relative to it.
  float m_run = -INFINITY, m_max = -INFINITY, l_run = 0.f;
  f32x16 negm = {};
  const int kv_first = p.win_left >= 0 ? myq - p.win_left : -(1 << 30);
  const int kv_last = min(p.win_right >= 0 ? myq + p.win_right : (1 << 30), p.Sk - 1);
  // Paged: validity of the tile's keys (bit r = key kv0 + r) and the ALiBi
  // slope in log2 units (added to the scores, which are in log2 units), applied
  // as slope * (kv - kv_last): it differs from slope * (kv - q) by a per-row
  // constant, which softmax ignores, and stays small for the keys that carry
  // the weight.
  uint64_t vmask = ~0ull, vmask_hi = ~0ull;  // keys kv0 .. +63, kv0 + 64 .. +127
  const float alibi = (kSlice && p.slopes) ? p.slopes[wi.h] * kLog2e : 0.f;

  // S^T of this wave's rows against the K tile at Kb (MFMAs only; the
  // caller orders them against other work).
  auto qk_mfma = [&](const unsigned char* Kb, f32x16 (&s)[NB]) __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      u32x4 ka[NKS];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) ka[ks] = *(const u32x4*)(Kb + kaddr[ks] + nb * 32 * ROWB);
      s[nb] = mfma32x32x16<BF16>(ka[0], qreg[0], negm);
#pragma unroll
      for (int ks = 1; ks < NKS; ++ks) s[nb] = mfma32x32x16<BF16>(ka[ks], qreg[ks], s[nb]);
    }
  };
  // K reads of block nb+1 in flight under the MFMAs of block nb.
  auto qk_sched = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_sched_group_barrier(0x100, NKS, 0);
#pragma unroll
    for (int i = 0; i < NKS * (NB - 1); ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, NKS, 0);
  };
  // Masks, row max and (rare) rescale of O for the tile at kv0. Scores are
  // relative to m_run (to 0 while it is -inf); a rescale moves m_run, O,
  // l_run, this tile's scores and negm to the new reference.
  // pmask (paged, 64-key tiles): the tile needs the per-key page mask or the
  // ALiBi bias; otherwise its masks are the dense kernel's. (The 128-key
  // kernel always takes the paged masks: a second copy of the mask loop costs
  // it registers.)
  auto max_rescale = [&](f32x16 (&s)[NB], int kv0, bool full, bool pmask)
                         __attribute__((always_inline)) {
    if (!full && !(PAGED && (kScalarPages || pmask))) {
      asm volatile("" ::: "memory");
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int kv = kv0 + nb * 32 + 16 * (e >> 3) + (e & 7) + 8 * g;
          s[nb][e] = ((kv >= kv_first) & (kv <= kv_last)) ? s[nb][e] : -INFINITY;
        }
    } else if (!full) {
      asm volatile("" ::: "memory");
      const uint64_t vm = PAGED ? vmask >> (8 * g) : 0;
      const uint64_t vm_hi = PAGED ? vmask_hi >> (8 * g) : 0;
      const float dq0 = PAGED ? (float)(kv0 + 8 * g - kv_last) : 0.f;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int kc = nb * 32 + 16 * (e >> 3) + (e & 7);
          const int kv = kv0 + kc + 8 * g;
          bool ok = (kv >= kv_first) & (kv <= kv_last);
          float sv = s[nb][e];
          if constexpr (PAGED) {
            ok = ok & ((((kc < 64 ? vm : vm_hi) >> (kc & 63)) & 1ull) != 0);
            sv += alibi * (dq0 + (float)kc);
          }
          s[nb][e] = ok ? sv : -INFINITY;
        }
    }
    // Four independent max chains (not one serial chain of 64).
    float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int e = 0; e < 16; ++e) mx[e & 3] = fmaxf(mx[e & 3], s[nb][e]);
    float mt = fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3]));
    mt = pair_max32(mt);  // relative to msub
    const float msub = m_run == -INFINITY ? 0.f : m_run;
    m_max = fmaxf(m_max, mt + msub);
    if (__any(m_run == -INFINITY ? mt > -INFINITY : mt > kRescaleThreshold)) {
      asm volatile("" ::: "memory");
      const float m_new = fmaxf(m_run, mt + msub);
      const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m_run - m_new);
      const float delta = m_new == -INFINITY ? 0.f : m_new - msub;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[db][e] *= alpha;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int e = 0; e < 16; ++e) s[nb][e] -= delta;
      m_run = m_new;
      const float nm = m_new == -INFINITY ? 0.f : -m_new;
#pragma unroll
      for (int e = 0; e < 16; ++e) negm[e] = nm;
    }
  };
  // P^T = exp2(s), s already relative to m_run, packed to 16 bits and O += P V, fused slice by slice:
  // the four PV MFMAs of 16-key slice sl need only that slice's weights, so
  // the exponentials of slice sl+1 run while the MFMAs of slice sl execute.
  // The row sum accumulates the packed (rounded) weights, the exact weights
  // the PV product uses. V^T operands come through the transposing read, one
  // slice ahead of their MFMAs. Dropout: the PV operand keeps the weights of
  // the kept keys only (the row sum takes them all; 1 / (1 - p) is applied
  // with the normalisation); element pair e2 of slice sl holds keys
  // kv0 + 16 sl + 8 g + 2 e2 + {0, 1}, the hash's key pair kv0 / 2 + 8 sl + 4 g + e2.
  auto exp_pv = [&](const f32x16 (&s)[NB], const unsigned char* Vb, int kv0)
                    __attribute__((always_inline)) {
    float lsum[2] = {0.f, 0.f};
    const u32 pair0 = DROP ? drop_pair_key((u32)(kv0 >> 1) + 4u * g, p.seed1) : 0u;
    auto vread = [&](int sl, u32x4 (&va)[NDB]) __attribute__((always_inline)) {
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const u32x2 lo = lds_read_tr16(Vb + vaddr[db] + (16 * sl) * ROWB);
        const u32x2 hi = lds_read_tr16(Vb + vaddr_hi[db] + (16 * sl) * ROWB);
        va[db] = (u32x4){lo[0], lo[1], hi[0], hi[1]};
      }
    };
    u32x4 vcur[NDB], vnext[NDB];
    vread(0, vcur);
#pragma unroll
    for (int sl = 0; sl < NSL; ++sl) {
      const int nb = sl >> 1, hh = sl & 1;
      u32x4 pk4;
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const float x0 = fast_exp2(s[nb][8 * hh + 2 * e2]);
        const float x1 = fast_exp2(s[nb][8 * hh + 2 * e2 + 1]);
        const u32 pk = pack2<BF16>(x0, x1);
        if constexpr (DROP)
          pk4[e2] = pk & drop_mask2(drop_bits(drop_rk, pair0 + (u32)(8 * sl + e2) * 0x85EBCA77u),
                                    p.drop_thresh);
        else
          pk4[e2] = pk;
        lsum[e2 & 1] = dot2_sum<BF16>(pk, lsum[e2 & 1]);
      }
      if (sl + 1 < NSL) vread(sl + 1, vnext);
#pragma unroll
      for (int db = 0; db < NDB; ++db) o[db] = mfma32x32x16<BF16>(vcur[db], pk4, o[db]);
      if (sl + 1 < NSL) {
#pragma unroll
        for (int db = 0; db < NDB; ++db) vcur[db] = vnext[db];
      }
    }
    l_run += lsum[0] + lsum[1];
  };

  auto compute_tile = [&](const unsigned char* Kb, int kv0) __attribute__((always_inline)) {
    bool skip, full;
    classify_tile<BN>(p, kv0, wq0, wq0 + 31, skip, full);
    if (skip) return;
    bool pmask = false;
    if constexpr (kSlice) {
      // Lane l checks key kv0 + l (one 64-bit ballot per tile).
      const int key = kv0 + lane;
      bool ok = key < p.Sk;
      if (ok) ok = pages[page_of(p, key) - pg_first] >= 0;
      vmask = __ballot(ok);
      pmask = vmask != ~0ull || alibi != 0.f;
    }
    if constexpr (kChecked) {
      if (!tile_ok) {
        // Lane l checks keys kv0 + l and kv0 + 64 + l against the table. The
        // loads are waited for here (vmcnt(0)), so the tile waits below
        // still count DMA loads only.
        const int k0 = kv0 + lane, k1 = k0 + 64;
        const int b0 = bt_row[min(k0, p.Sk - 1) >> p.bs_log2];
        const int b1 = bt_row[min(k1, p.Sk - 1) >> p.bs_log2];
        __builtin_amdgcn_s_waitcnt(0x0F70);
        vmask = __ballot((k0 < p.Sk) & (b0 >= 0) & (b0 < p.num_blocks));
        vmask_hi = __ballot((k1 < p.Sk) & (b1 >= 0) & (b1 < p.num_blocks));
      } else {
        vmask = vmask_hi = ~0ull;  // (a previous tile may have set them)
      }
      pmask = !tile_ok;
    }
    if (pmask) full = false;
    f32x16 s[NB];
    qk_mfma(Kb, s);
    // (D = 256: the compiler's own order; the pattern's K reads of block nb + 1
    // under block nb would hold 128 registers of operands)
    if constexpr (D <= 128) qk_sched();
    max_rescale(s, kv0, full, pmask);
    exp_pv(s, Kb + KBYTES, kv0);
  };

  // Every tile is 2 * NDMA DMA instructions per wave (4 at D = 128, 2 at
  // D = 64); after issuing tiles up to `last`, tile t has landed once at most
  // 2 * NDMA * (last - t) loads are pending.
  constexpr int kTileLoads = 2 * NDMA;
  auto wait_tiles_after = [&](int pending_tiles) __attribute__((always_inline)) {
    if (pending_tiles >= 2) {
      __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * kTileLoads));  // vmcnt(2 tiles)
    } else if (pending_tiles == 1) {
      __builtin_amdgcn_s_waitcnt(0x0F70 | kTileLoads);  // vmcnt(1 tile)
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
  };
  const int n_tiles = t_end - t_begin;
  if constexpr (kScalarPages) {
    if (n_tiles > 0) fetch_pages(kv_lo + t_begin * BN);
  }
  if (n_tiles > 0) load_tile(kv_lo + t_begin * BN, st0);
  if constexpr (kChecked) tile_ok = tile_ok_next;
  if constexpr (kScalarPages) {
    if (n_tiles > 1) fetch_pages(kv_lo + (t_begin + 1) * BN);
  }
  if (NST >= 3 && n_tiles > 1) load_tile(kv_lo + (t_begin + 1) * BN, st1);
  if (NST == 4 && n_tiles > 2) load_tile(kv_lo + (t_begin + 2) * BN, st2);
  wait_tiles_after(min(n_tiles, NST - 1) - 1);  // tile 0 landed
  stage_barrier();
  // Tile i computes from stage i%NST; tile i+NST-1 goes to the stage tile
  // i-1 used (every wave finished reading it before the last barrier).
  auto step = [&](int i, auto ST) __attribute__((always_inline)) {
    constexpr int S = decltype(ST)::value;
    const int kv0 = kv_lo + (t_begin + i) * BN;
    if (i + NST - 1 < n_tiles)
      load_tile(kv0 + (NST - 1) * BN, stage_ptr(Const<(S + NST - 1) % NST>{}));
    if constexpr (kScalarPages) {
      if (i + NST < n_tiles) fetch_pages(kv0 + NST * BN);
    }
    compute_tile(stage_ptr(Const<S>{}), kv0);
    if constexpr (kChecked) tile_ok = tile_ok_next;
    // Tile i+1 must have landed before the barrier that hands it to every
    // wave; the tiles issued after it may stay in flight.
    wait_tiles_after(min(n_tiles - 1, i + NST - 1) - (i + 1));
    stage_barrier();
  };
  for (int i = 0; i < n_tiles; i += NST) {
    step(i, Const<0>{});
    if (i + 1 < n_tiles) step(i + 1, Const<1>{});
    if (NST >= 3 && i + 2 < n_tiles) step(i + 2, Const<2 % NST>{});
    if (NST == 4 && i + 3 < n_tiles) step(i + 3, Const<3 % NST>{});
  }

  const float l_tot = pair_sum32(l_run);
  const float f = m_max == -INFINITY ? 0.f : fast_exp2(m_run - m_max);
  // (dropout: kept weights times 1 / (1 - p); the row sums stay unscaled)
  const float fo = DROP ? f * p.drop_scale : f;
  if (p.num_splits == 1 && NW * 32 * ROWB <= 2 * STAGEB) {
    // O goes out through LDS so that each store instruction writes whole rows
    // (16 bytes a lane, CPR lanes a row): straight from the accumulators an
    // instruction would write 8-byte pieces of 32 rows. The stages are free
    // here (the last tile step ended with no DMA in flight and every wave past
    // its reads). Wave w's 32 rows sit in its own region, the 16-byte chunk c
    // of row r at slot c ^ oswz(r), so that the writes (two lanes per row and
    // chunk) and the row reads are free of bank conflicts.
    constexpr int CPR = ROWB / 16, RPI = 64 / CPR, OWB = 32 * ROWB;
    auto oswz = [](int r) { return CPR >= 16 ? (r & 15) : ((r >> 1) & 7); };
    unsigned char* const eb = NW * OWB <= STAGEB
                                  ? st0 + wave * OWB
                                  : (wave < NW / 2 ? st0 : st1) + (wave % (NW / 2)) * OWB;
    // (the lane index taken afresh: addresses derived from it are not hoisted
    // into registers the tile loop needs)
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int jr = ln & 31, gr = ln >> 5;
    if (myq < p.Sq) {
      const float inv = m_max == -INFINITY ? (p.nan_empty ? __builtin_nanf("") : 0.f)
                                           : fo / (l_tot * f + p.eps);
      if (p.lse && g == 0)
        p.lse[((int64_t)wi.b * p.H + wi.h) * p.Sq + myq] =
            m_max == -INFINITY ? INFINITY : m_max + log2f(l_tot * f + p.eps);
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
          // dims 8c + 4g .. + 3 of row j, c = 4 db + e4
          const int c = 4 * db + e4;
          const u32x2 val = {pack2<BF16>(o[db][4 * e4] * inv, o[db][4 * e4 + 1] * inv),
                             pack2<BF16>(o[db][4 * e4 + 2] * inv, o[db][4 * e4 + 3] * inv)};
          *(u32x2*)(eb + jr * ROWB + (c ^ oswz(jr)) * 16 + 8 * gr) = val;
        }
    }
    uint16_t* const Ob = (uint16_t*)p.o + wi.b * p.o_sb + wi.h * p.o_sh;
#pragma unroll
    for (int i = 0; i < 32 / RPI; ++i) {
      const int r = RPI * i + ln / CPR, c = ln % CPR;
      const u32x4 val = *(const u32x4*)(eb + r * ROWB + (c ^ oswz(r)) * 16);
      if (wq0 + r < p.Sq) *(u32x4*)(Ob + (int64_t)(wq0 + r) * p.o_ss + 8 * c) = val;
    }
    stage_barrier();  // every wave's rows read before the next item restages LDS
  } else if (p.num_splits == 1) {
    if (myq < p.Sq) {
      const float inv = m_max == -INFINITY ? (p.nan_empty ? __builtin_nanf("") : 0.f)
                                           : fo / (l_tot * f + p.eps);
      if (p.lse && g == 0)
        p.lse[((int64_t)wi.b * p.H + wi.h) * p.Sq + myq] =
            m_max == -INFINITY ? INFINITY : m_max + log2f(l_tot * f + p.eps);
      uint16_t* Op = (uint16_t*)p.o + wi.b * p.o_sb + wi.h * p.o_sh + (int64_t)myq * p.o_ss;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
          const int d = db * 32 + 8 * e4 + 4 * g;
          const u32x2 val = {pack2<BF16>(o[db][4 * e4] * inv, o[db][4 * e4 + 1] * inv),
                             pack2<BF16>(o[db][4 * e4 + 2] * inv, o[db][4 * e4 + 3] * inv)};
          *(u32x2*)(Op + d) = val;
        }
    }
  } else if (myq < p.Sq) {
    const int64_t row = (((int64_t)wi.split * p.B + wi.b) * p.H + wi.h) * p.Sq + myq;
    float* wo = p.ws_o + row * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int d = db * 32 + 8 * e4 + 4 * g;
        *(f32x4*)(wo + d) = (f32x4){o[db][4 * e4] * fo, o[db][4 * e4 + 1] * fo,
                                    o[db][4 * e4 + 2] * fo, o[db][4 * e4 + 3] * fo};
      }
    if (g == 0) {
      p.ws_ml[2 * row] = m_max;
      p.ws_ml[2 * row + 1] = l_tot * f;
    }
  }
}

template <int D, int BN, int NW, bool BF16, bool PAGED, bool BIG = false>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(MPX_FA_WAVES_PER_EU)))
void fa_fwd16_kernel(FwdParams p) {
  // Stay within 128 KB of LDS per workgroup (a 136 KB configuration gave wrong
  // results on gfx950).
  constexpr bool kDirect = MPX_FA_DIRECT && (D == 128 || D == 64) && (BN == 64 || BN == 128) &&
                           (NW == 8 || NW == 4);
  // Paged with 64-key tiles: three stages, which leaves room for the
  // page-table slice.
  constexpr bool kSlice = PAGED && BN == 64;
  constexpr int kDStages =
      kSlice ? 3
            : (MPX_FA_DSTAGES > 0 ? MPX_FA_DSTAGES
                                  : (131072 / (4 * BN * D) < 4 ? 131072 / (4 * BN * D) : 4));
  constexpr int kLdsBytes =
      kDirect ? kDStages * 2 * BN * 2 * D : kFa16Stages * fa16_stage_elems<D, BN>() * 2;
  static_assert(kLdsBytes + (kSlice ? kMaxItemPages * 4 : 0) <= 131072, "LDS budget");
  // Direct staging uses three separate stage arrays (so alias analysis can
  // tell a stage being read from the stage a DMA is writing); smem is used by
  // the register-staged path.
  constexpr int kStageB = kDirect ? 2 * BN * 2 * D : 16;
  __shared__ __align__(16) uint16_t smem[kDirect ? 8 : kLdsBytes / 2];
  __shared__ __align__(16) unsigned char dst0[kStageB];
  __shared__ __align__(16) unsigned char dst1[kStageB];
  __shared__ __align__(16) unsigned char dst2[kDStages >= 3 ? kStageB : 16];
  __shared__ __align__(16) unsigned char dst3[kDStages == 4 ? kStageB : 16];
  __shared__ int pages[kSlice ? kMaxItemPages : 1];
  const WorkSlot ws = decode_slot(p);
  const int n_items = slot_items(p, ws);
  // Every item ends with a barrier after its last LDS read, so the next item
  // may restage LDS at once.
#pragma nounroll
  for (int item = 0; item < n_items; ++item) {
    if constexpr (kDirect)
      fa16_rows_direct<D, BN, NW, BF16, kDStages, PAGED, false, BIG>(
          p, slot_item(p, ws, item), dst0, dst1, dst2, dst3, pages);
    else
      fa16_rows<D, BN, NW, BF16, PAGED, false, BIG>(p, slot_item(p, ws, item), smem, pages);
  }
}

// The same with dropout on the weights (dense K/V, D = 64 or 128: the direct
// kernels).
template <int D, int BN, int NW, bool BF16>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(MPX_FA_WAVES_PER_EU)))
void fa_fwd16_drop_kernel(FwdParams p) {
  constexpr int kDStages = MPX_FA_DSTAGES > 0 ? MPX_FA_DSTAGES
                                              : (131072 / (4 * BN * D) < 4 ? 131072 / (4 * BN * D) : 4);
  static_assert(MPX_FA_DIRECT && (D == 128 || D == 64) && (BN == 64 || BN == 128) &&
                    (NW == 8 || NW == 4) && kDStages * 2 * BN * 2 * D <= 131072,
                "dropout runs on the direct kernels");
  constexpr int kStageB = 2 * BN * 2 * D;
  __shared__ __align__(16) unsigned char dst0[kStageB];
  __shared__ __align__(16) unsigned char dst1[kStageB];
  __shared__ __align__(16) unsigned char dst2[kDStages >= 3 ? kStageB : 16];
  __shared__ __align__(16) unsigned char dst3[kDStages == 4 ? kStageB : 16];
  const WorkSlot ws = decode_slot(p);
  const int n_items = slot_items(p, ws);
#pragma nounroll
  for (int item = 0; item < n_items; ++item)
    fa16_rows_direct<D, BN, NW, BF16, kDStages, false, true>(p, slot_item(p, ws, item), dst0, dst1,
                                                             dst2, dst3, nullptr);
}

// Head dims 129 .. 256 (zero-padded to 256): four waves of one wave per SIMD,
// since the Q fragments (64 registers) and the O accumulators (128) leave too
// little of the 256 registers of two waves per SIMD. Dense K/V: the direct
// (DMA-staged) rows with 64-key tiles. PAGED (prefill over a paged cache): the
// register-staged rows with 32-key tiles and the item's page-table slice.
constexpr int kNumWavesWide = 4;
template <int D, int BN, int NW, bool BF16, bool PAGED = false, bool DROP = false,
          bool BIG = false>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(1, 1)))
void fa_fwd16_wide_kernel(FwdParams p) {
  // Dense K/V with 64-key tiles: direct (DMA) staging, two stages of 64 KB.
  constexpr bool kDirect = !PAGED && BN == 64;
  constexpr int kLdsBytes = kDirect ? 16 : kFa16Stages * fa16_stage_elems<D, BN>() * 2;
  constexpr int kStageB = kDirect ? 2 * BN * 2 * D : 16;
  static_assert(kLdsBytes + 2 * kStageB + (PAGED ? kMaxItemPages * 4 : 0) <= 131072 + 16,
                "LDS budget");
  __shared__ __align__(16) uint16_t smem[kLdsBytes / 2];
  __shared__ __align__(16) unsigned char dst0[kStageB];
  __shared__ __align__(16) unsigned char dst1[kStageB];
  __shared__ __align__(16) unsigned char unused2[16], unused3[16];  // (stages 2, 3: none)
  __shared__ int pages[PAGED ? kMaxItemPages : 1];
  const WorkSlot ws = decode_slot(p);
  const int n_items = slot_items(p, ws);
  // Every item ends with a barrier after its last LDS read.
#pragma nounroll
  for (int item = 0; item < n_items; ++item) {
    if constexpr (kDirect)
      fa16_rows_direct<D, BN, NW, BF16, 2, false, DROP>(p, slot_item(p, ws, item), dst0, dst1,
                                                         unused2, unused3, nullptr);
    else
      fa16_rows<D, BN, NW, BF16, PAGED, DROP, BIG>(p, slot_item(p, ws, item), smem, pages);
  }
}

// ---------------------------------------------------------------------------
// fp32 kernel: 32x32x2 f32 MFMA (true fp32 products, for fp32 parity).
// S^T = K Q^T with k index (4-dim run) dims 8*(ks/4) + 4*g + ks%4; C element e
// of lane (j, g) holds key 32*nb + 8*(e/4) + 4*g + e%4. PV step (nb, e) has
// k = g <-> that key, so P^T needs no repacking and V stays row-major in LDS.
// ---------------------------------------------------------------------------
template <int D, int BN, int NW, bool PAGED, bool DROP = false>
__global__ __launch_bounds__(64 * NW) void fa_fwd32_kernel(FwdParams pin) {
  constexpr int BM = 32 * NW, NT = 64 * NW;
  constexpr int KS = D + 4;  // conflict-free 16-byte reads along rows
  constexpr int VS = D + 8;  // rows kv and kv+4 land on opposite bank halves
  constexpr int K_ELEMS = BN * KS, V_ELEMS = BN * VS, STAGE = K_ELEMS + V_ELEMS;
  constexpr int NB = BN / 32, NDB = D / 32, NQ4 = D / 8;
  constexpr int CPR = D / 4;  // 16-byte chunks per row
  constexpr int CHUNKS = BN * CPR;
  constexpr int PER_T = (CHUNKS + NT - 1) / NT;
  static_assert(D % 32 == 0 && BN % 32 == 0, "tile shape");
  // D = 256: one LDS stage (two do not fit 128 KB); the next tile is loaded
  // once every wave has finished reading the current one (not under the
  // compute: its registers would spill).
  constexpr int NSTG = D > 128 ? 1 : 2;
  static_assert(NSTG * STAGE * 4 <= 131072, "LDS budget");

  __shared__ __align__(16) float smem[NSTG * STAGE];
  __shared__ int pages[PAGED ? kMaxItemPages : 1];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, g = lane >> 5;

  const WorkItem wi = slot_item(pin, decode_slot(pin), 0);
  FwdParams p = pin;
  if constexpr (PAGED) p.Sk = max(0, min(pin.ctx[wi.b], pin.max_blocks * pin.bs));
  const int q0 = wi.qt * BM;
  int kv_lo, t_begin, t_end;
  kv_range<BM, BN>(p, q0, wi.split, kv_lo, t_begin, t_end);

  const float* __restrict__ Qp = (const float*)p.q + wi.b * p.q_sb + wi.h * p.q_sh;
  const int kvh = wi.h / p.kv_group;  // K/V head of this query head
  const float* __restrict__ Kp = (const float*)p.k + wi.b * p.k_sb + kvh * p.k_sh;
  const float* __restrict__ Vp = (const float*)p.v + wi.b * p.v_sb + kvh * p.v_sh;

  const int wq0 = q0 + wave * 32;
  const int myq = wq0 + j;
  // Dropout: this row's key of the keep-mask hash.
  const u32 drop_rk =
      DROP ? drop_row_key((u32)(((int64_t)wi.b * p.H + wi.h) * p.Sq + myq), p.seed0) : 0u;
  f32x4 qf[NQ4];
  if (myq < p.Sq) {
    const f32x4* src = (const f32x4*)(Qp + (int64_t)myq * p.q_ss);
#pragma unroll
    for (int jj = 0; jj < NQ4; ++jj) qf[jj] = src[2 * jj + g];
  } else {
#pragma unroll
    for (int jj = 0; jj < NQ4; ++jj) qf[jj] = (f32x4){};
  }
  if (p.neg) {
#pragma unroll
    for (int jj = 0; jj < NQ4; ++jj) qf[jj] = -qf[jj];
  }

  // Paged: this item's slice of the page table, validated, in LDS.
  int pg_first = 0;
  if constexpr (PAGED) {
    const int kv_a = kv_lo + t_begin * BN, kv_b = min(kv_lo + t_end * BN, p.Sk);
    pg_first = page_of(p, kv_a);
    const int npg = kv_b > kv_a ? page_of(p, kv_b - 1) - pg_first + 1 : 0;
    const int32_t* row = p.bt + (int64_t)wi.b * p.max_blocks + pg_first;
    for (int i = tid; i < npg; i += NT) {
      const int blk = row[i];
      pages[i] = (blk >= 0 && blk < p.num_blocks) ? blk : -1;
    }
    __syncthreads();
  }

  // Rows past Sk re-read the last valid row (no data-dependent selects at
  // load time); their V values are zeroed when stored. Paged: missing rows
  // read row 0 of the pool and are zeroed / masked the same way.
  f32x4 kbuf[PER_T], vbuf[PER_T];
  bool vok[PER_T];
  int v_rows = BN;
  auto load_tile = [&](int kv0) {
    v_rows = min(BN, p.Sk - kv0);
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int cc = tid + i * NT;
      if (CHUNKS % NT == 0 || cc < CHUNKS) {
        const int row = cc / CPR, col = cc - (cc / CPR) * CPR;
        int64_t kr, vr;
        if constexpr (PAGED) {
          const int pos = kv0 + row;
          int64_t prow = -1;
          if (pos < p.Sk) {
            const int pg = page_of(p, pos);
            const int page = pages[pg - pg_first];
            if (page >= 0) prow = (int64_t)page * p.bs + (pos - pg * p.bs);
          }
          vok[i] = prow >= 0;
          kr = max(prow, (int64_t)0);
          vr = kr;
        } else {
          vok[i] = true;
          kr = vr = min(kv0 + row, p.Sk - 1);
        }
        kbuf[i] = *(const f32x4*)(Kp + kr * p.k_ss + col * 4);
        vbuf[i] = *(const f32x4*)(Vp + vr * p.v_ss + col * 4);
      }
    }
  };
  auto store_tile = [&](int stage) {
    float* Ks = smem + stage * STAGE;
    float* Vs = Ks + K_ELEMS;
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int cc = tid + i * NT;
      if (CHUNKS % NT == 0 || cc < CHUNKS) {
        const int row = cc / CPR, col = cc - (cc / CPR) * CPR;
        *(f32x4*)(Ks + row * KS + col * 4) = kbuf[i];
        *(f32x4*)(Vs + row * VS + col * 4) = (row < v_rows && vok[i]) ? vbuf[i] : (f32x4){};
      }
    }
  };

  f32x16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = (f32x16){};
  float m_run = -INFINITY, m_max = -INFINITY, l_run = 0.f;
  const float c = p.c;
  // ALiBi as in the 16-bit kernel: slope / |scale| on raw scores, measured
  // from the row's last visible key.
  const float alibi = (PAGED && p.slopes) ? p.slopes[wi.h] * kLog2e / p.c : 0.f;
  const int kv_anchor = min(p.win_right >= 0 ? myq + p.win_right : (1 << 30), p.Sk - 1);

  if (t_begin < t_end) {
    load_tile(kv_lo + t_begin * BN);
    store_tile(0);
  }
  __syncthreads();

  for (int t = t_begin; t < t_end; ++t) {
    const int stage = NSTG == 1 ? 0 : (t - t_begin) & 1;
    const int kv0 = kv_lo + t * BN;
    const bool has_next = t + 1 < t_end;
    if (NSTG == 2 && has_next) load_tile(kv0 + BN);

    bool skip, full;
    classify_tile<BN>(p, kv0, wq0, wq0 + 31, skip, full);
    uint64_t vmask = ~0ull;
    if constexpr (PAGED) {
      if (!skip) {
        const int key = kv0 + (lane % BN);
        bool ok = key < p.Sk;
        if (ok) ok = pages[page_of(p, key) - pg_first] >= 0;
        vmask = __ballot(ok);
        if (BN < 64) vmask &= (1ull << BN) - 1;
        if (vmask != (BN < 64 ? (1ull << BN) - 1 : ~0ull) || alibi != 0.f) full = false;
      }
    }
    if (!skip) {
      const float* Ks = smem + stage * STAGE;
      const float* Vs = Ks + K_ELEMS;

      f32x16 s[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        s[nb] = (f32x16){};
        const f32x4* kp = (const f32x4*)(Ks + (nb * 32 + j) * KS) + g;
#pragma unroll
        for (int jj = 0; jj < NQ4; ++jj) {
          const f32x4 a = kp[2 * jj];
#pragma unroll
          for (int t4 = 0; t4 < 4; ++t4) s[nb] = mfma32x32x2f32(a[t4], qf[jj][t4], s[nb]);
        }
      }

      if (!full) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int kr = nb * 32 + 8 * (e >> 2) + 4 * g + (e & 3);
            const int kv = kv0 + kr;
            bool ok = kv_valid(p, myq, kv);
            if constexpr (PAGED) {
              ok = ok && ((vmask >> kr) & 1ull) != 0;
              s[nb][e] += alibi * (float)(kv - kv_anchor);
            }
            if (!ok) s[nb][e] = -INFINITY;
          }
      }

      float mt = -INFINITY;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int e = 0; e < 16; ++e) mt = fmaxf(mt, s[nb][e]);
      mt = pair_max32(mt) * c;
      m_max = fmaxf(m_max, mt);

      if (__any(mt > m_run + kRescaleThreshold)) {
        asm volatile("" ::: "memory");  // a real branch, not selects on all of o
        const float m_new = fmaxf(m_run, mt);
        const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[db][e] *= alpha;
        m_run = m_new;
      }
      const float msub = m_run == -INFINITY ? 0.f : m_run;

      float lsum = 0.f;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float x = fast_exp2(s[nb][e] * c - msub);
          s[nb][e] = x;
          lsum += x;
        }
      l_run += lsum;
      if constexpr (DROP) {
        // Keep mask on the PV operand: elements 2 e2, 2 e2 + 1 of block nb hold
        // keys kv0 + 32 nb + 8 (e2 / 2) + 4 g + 2 (e2 % 2) + {0, 1}, the hash's
        // key pair kv0 / 2 + 16 nb + 4 (e2 / 2) + 2 g + e2 % 2.
        const u32 pair0 = drop_pair_key((u32)(kv0 >> 1) + 2u * g, p.seed1);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int e2 = 0; e2 < 8; ++e2) {
            const u32 bits =
                drop_bits(drop_rk, pair0 + (u32)(16 * nb + 4 * (e2 >> 1) + (e2 & 1)) * 0x85EBCA77u);
            if ((bits & 0xffffu) < p.drop_thresh) s[nb][2 * e2] = 0.f;
            if (bits < (p.drop_thresh << 16)) s[nb][2 * e2 + 1] = 0.f;
          }
      }

#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int kv = nb * 32 + 8 * (e >> 2) + 4 * g + (e & 3);
            o[db] = mfma32x32x2f32(Vs[kv * VS + db * 32 + j], s[nb][e], o[db]);
          }
    }

    if (has_next) {
      if constexpr (NSTG == 1) {
        __syncthreads();
        load_tile(kv0 + BN);
      }
      store_tile(NSTG == 1 ? 0 : stage ^ 1);
    }
    __syncthreads();
  }

  const float l_tot = pair_sum32(l_run);
  const float f = m_max == -INFINITY ? 0.f : fast_exp2(m_run - m_max);
  // (dropout: kept weights times 1 / (1 - p); the row sums stay unscaled)
  const float fo = DROP ? f * p.drop_scale : f;
  if (p.num_splits == 1) {
    if (myq < p.Sq) {
      const float inv = m_max == -INFINITY ? (p.nan_empty ? __builtin_nanf("") : 0.f)
                                           : fo / (l_tot * f + p.eps);
      if (p.lse && g == 0)
        p.lse[((int64_t)wi.b * p.H + wi.h) * p.Sq + myq] =
            m_max == -INFINITY ? INFINITY : m_max + log2f(l_tot * f + p.eps);
      float* Op = (float*)p.o + wi.b * p.o_sb + wi.h * p.o_sh + (int64_t)myq * p.o_ss;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
          const int d = db * 32 + 8 * e4 + 4 * g;
          *(f32x4*)(Op + d) = (f32x4){o[db][4 * e4] * inv, o[db][4 * e4 + 1] * inv,
                                      o[db][4 * e4 + 2] * inv, o[db][4 * e4 + 3] * inv};
        }
    }
  } else if (myq < p.Sq) {
    const int64_t row = (((int64_t)wi.split * p.B + wi.b) * p.H + wi.h) * p.Sq + myq;
    float* wo = p.ws_o + row * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int d = db * 32 + 8 * e4 + 4 * g;
        *(f32x4*)(wo + d) = (f32x4){o[db][4 * e4] * fo, o[db][4 * e4 + 1] * fo,
                                    o[db][4 * e4 + 2] * fo, o[db][4 * e4 + 3] * fo};
      }
    if (g == 0) {
      p.ws_ml[2 * row] = m_max;
      p.ws_ml[2 * row + 1] = l_tot * f;
    }
  }
}

// ---------------------------------------------------------------------------
// Split-KV merge: the reference's online_softmax_merge
// (mlx_primitives/attention/_online_softmax.py:42-106) folded over all splits,
// then O / (l + eps) (rows that saw no key: 0, or NaN for the exact softmax).
// One thread per (row, 4 dims), one pass over the splits in batches of
// kMergeBatch: the batch's (m, l) and O loads are all issued before any is
// used, then the batch is folded in against the running maximum.
// ---------------------------------------------------------------------------
constexpr int kMergeBatch = 8;

// (The attention launch's split layout: each q-tile's split count when it
// has its own, var_split, as in decode_slot.)
struct MergeShape {
  int var_split, bm, bn, Sk, win_left, win_right, tiles_per_split;
};

template <int DT>
__global__ __launch_bounds__(256) void fa_split_merge_kernel(const float* __restrict__ ws_o,
                                                             const float* __restrict__ ws_ml,
                                                             void* o, int64_t o_sb, int64_t o_sh,
                                                             int64_t o_ss, int B, int H, int Sq,
                                                             int D, int splits, float eps,
                                                             int nan_empty, float* lse,
                                                             MergeShape ms) {
  const int chunks = D / 4;
  const int64_t rows = (int64_t)B * H * Sq;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * chunks) return;
  const int64_t row = idx / chunks;
  const int c4 = (int)(idx - row * chunks);
  if (ms.var_split > 0)
    splits = qtile_splits((int)(row % Sq) / ms.bm, ms.bm, ms.bn, Sq, ms.Sk, ms.win_left,
                          ms.win_right, ms.tiles_per_split);
  float M = -INFINITY, L = 0.f;
  f32x4 acc = {};
  for (int s0 = 0; s0 < splits; s0 += kMergeBatch) {
    float2 ml[kMergeBatch];
    f32x4 os[kMergeBatch];
#pragma unroll
    for (int i = 0; i < kMergeBatch; ++i) {
      ml[i] = make_float2(-INFINITY, 0.f);
      os[i] = (f32x4){};
      if (s0 + i < splits) {
        const int64_t r = (s0 + i) * rows + row;
        ml[i] = *(const float2*)(ws_ml + 2 * r);
        os[i] = *(const f32x4*)(ws_o + r * D + 4 * c4);
      }
    }
    float mb = M;
#pragma unroll
    for (int i = 0; i < kMergeBatch; ++i) mb = fmaxf(mb, ml[i].x);
    if (mb == -INFINITY) continue;  // nothing seen yet
    const float keep = fast_exp2(M - mb);  // 0 while M is -inf
    L *= keep;
    acc *= keep;
#pragma unroll
    for (int i = 0; i < kMergeBatch; ++i) {
      const float wgt = fast_exp2(ml[i].x - mb);  // 0 for splits that saw no key
      L += wgt * ml[i].y;
      acc += wgt * os[i];
    }
    M = mb;
  }
  if (M != -INFINITY) {
    acc = acc / (L + eps);
  } else if (nan_empty) {
    acc = (f32x4){} + __builtin_nanf("");
  }
  if (lse && c4 == 0) lse[row] = M == -INFINITY ? INFINITY : M + log2f(L + eps);
  const int q = (int)(row % Sq);
  const int bh = (int)(row / Sq);
  const int b = bh / H, h = bh - (bh / H) * H;
  const int64_t off = b * o_sb + h * o_sh + (int64_t)q * o_ss + 4 * c4;
  if constexpr (DT == MPX_F32) {
    *(f32x4*)((float*)o + off) = acc;
  } else {
    const u32x2 val = {pack2<DT == MPX_BF16>(acc[0], acc[1]), pack2<DT == MPX_BF16>(acc[2], acc[3])};
    *(u32x2*)((uint16_t*)o + off) = val;
  }
}

// Launch shapes shared by the launch code of both translation units.
constexpr int kNumWaves16 = MPX_FA_NWAVES;     // waves per workgroup, 16-bit kernel
constexpr int kNumWaves32 = MPX_FA_NWAVES_F32; // waves per workgroup, fp32 kernel

// KV tile of the 16-bit kernels (the paged, D = 32 and register-staged ones
// take 64 keys).
template <bool PAGED, int D>
constexpr int kBN16 = PAGED || D < 64 || !MPX_FA_DIRECT ? 64 : MPX_FA_BN16;

}  // namespace mpx
