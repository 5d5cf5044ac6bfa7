// Attention backward for gfx950 (MI355X), bf16 / f16, head_dim 64 or 128.
//
// Gradients of O = softmax(scale * Q K^T + mask) V (with the forward's
// O / (l + eps) normaliser) for mlx_primitives' flash_attention
// (attention/flash.py:52-254; the reference differentiates its tiled path with
// mx.grad, tests/attention/test_flash.py:338-362). With the forward's row
// log-sum-exp lse (log2 units), P = exp2(s * c - lse), c = scale * log2(e):
//   Dvec_i = sum_d dO[i, d] * O[i, d]                 (fa_bwd_dq_kernel)
//   dP = dO V^T,  dS = P * (dP - Dvec_i)
//   dQ = scale * dS K                                 (fa_bwd_dq_kernel)
//   dV = P^T dO,  dK = scale * dS^T Q                 (fa_bwd_dkdv_kernel,
//                                                      fa_bwd_dkdv_fused_kernel)
// Two MFMA kernels, no atomics: dQ is query-parallel (each workgroup owns 128
// query rows and streams K and V; it also writes Dvec), dK/dV key-parallel
// (each workgroup owns 128 keys and streams Q and dO). Both recompute S and
// dP; tiles go from HBM straight into LDS (buffer_load ... lds), double
// buffered: the tile after the current one is in flight while the current one
// is computed.
//
// MFMA 32x32x16 layouts (lane = j + 32*g, j in [0,32)): A (32 x 16) lane holds
// row j, k-group g (8 values); B (16 x 32) column j, k-group g; C (32 x 32)
// element e of lane holds row 8*(e/4) + 4*g + e%4, column j. Streamed row
// operands are read with rows permuted (bits 2 and 3 of the row index
// exchanged) so that C elements 8h..8h+7 of a lane are 8 consecutive rows:
// packed, they are directly the B operand of the next product over those rows.
// Transposed operands come from the row-major tiles through ds_read_b64_tr_b16.
#include "fa_bwd.h"

#include <algorithm>
#include <cmath>

namespace mpx {


// LDS tiles are (64, D) row-major without padding; the 16-byte chunk c of row
// r sits at slot c ^ swz(r). Each tile is read two ways, and the swizzle keeps
// both conflict-free: 16 lanes reading one chunk of 16 consecutive rows (row
// operands) hit 16 distinct bank groups, and 32 lanes of a transposing read (4
// consecutive rows x 4 consecutive chunks) hit all 64 banks once.
template <int D>
__device__ __forceinline__ int swz(int r) {
  if constexpr (D == 128) {
    return ((r & 3) << 2) | ((r >> 2) & 3);
  } else if constexpr (D == 256) {
    // 512-byte rows: a DMA block is 2 rows and a wave's blocks are 8 rows
    // apart, so the swizzle may use row bits 0-2 only (row operand reads of 16
    // rows then pair up on 8 bank groups).
    return ((r & 3) << 2) | ((r >> 2) & 1);
  } else {
    return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
  }
}

// DMA of ROWS (64 by default) rows of a 16-bit (rows, D) slice into a swizzled
// LDS tile. A DMA instruction fills 1 KB of LDS (RPD rows); wave w issues the
// blocks w, w + 4, ... . Lane l lands at slot l % CPR of row l / CPR of its block, so it
// loads logical chunk (l % CPR) ^ swz(row); the swizzle only depends on the
// low 4 row bits (3 at D = 256), which are the same in all of a lane's blocks. Rows past the
// slice end re-read its last row (callers mask them or weight them by 0).
template <int D, int ROWS = kBwdTile>
struct TileDma {
  static constexpr int CPR = D / 8;                            // 16-byte chunks per row
  static constexpr int RPD = 64 / CPR;                         // rows per DMA (1 KB)
  static constexpr int NDMA = ROWS / (RPD * kBwdWaves);        // DMAs per wave per tile
  static_assert(NDMA * RPD * kBwdWaves == ROWS, "whole DMA rounds per tile");
  int row_bytes, lrow, lchunk, voff;
  u32 lds_off;
  __device__ __forceinline__ void init(int64_t row_stride, int wave, int lane) {
    row_bytes = (int)row_stride * 2;
    lrow = wave * RPD + lane / CPR;
    lchunk = (lane % CPR) ^ swz<D>(lrow);
    voff = lrow * row_bytes + lchunk * 16;
    lds_off = (u32)wave * 1024u;
  }
  // Rows row0 .. row0 + ROWS - 1 of the slice at base (rows rows) into the LDS tile at lds.
  __device__ __forceinline__ void load(const void* base, u32 lds, int row0, int rows) const {
    const u32x4 rs = buffer_desc(base);
    const int so = row0 * row_bytes;
    if (row0 + ROWS <= rows) {
#pragma unroll
      for (int r = 0; r < NDMA; ++r)
        dma16(rs, lds + lds_off + r * kBwdWaves * 1024u, voff,
              so + r * kBwdWaves * RPD * row_bytes);
    } else {
#pragma unroll
      for (int r = 0; r < NDMA; ++r) {
        const int row = min(lrow + r * kBwdWaves * RPD, rows - 1 - row0);
        dma16(rs, lds + lds_off + r * kBwdWaves * 1024u, row * row_bytes + lchunk * 16, so);
      }
    }
  }
};

// s_waitcnt vmcnt(0) lgkmcnt(0): every load and LDS access of this wave done.
__device__ __forceinline__ void wait_all() { __builtin_amdgcn_s_waitcnt(0x0070); }

// Per-lane LDS element offsets into a swizzled (64, D) tile. row[ks]: A
// operand rows 32*nb + perm(j), k-step ks (add nb * 32 * D). tr[db][hf]: the
// transposing read for A = X^T over rows 16*sl + 8g + 4hf + s/4, columns
// 32*db + 16*((lane/16) % 2) + 4*(s % 4), s = lane % 16 (add 16 * sl * D); for a
// group of 16 lanes it returns to lane s column 32*db + 16*((lane/16) % 2) + s
// of the 4 rows, i.e. row j = dim of the A operand, k-group g = 8 rows.
template <int D>
struct Addr {
  static constexpr int NKS = D / 16, NDB = D / 32;
  int row[NKS];
  int tr[NDB][2];
  __device__ __forceinline__ void init(int lane) {
    const int j = lane & 31, g = lane >> 5;
    const int perm = (j & ~12) | ((j & 4) << 1) | ((j & 8) >> 1);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) row[ks] = perm * D + 8 * ((2 * ks + g) ^ swz<D>(perm));
    const int s = lane & 15, half = (lane >> 4) & 1;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int r = 8 * g + 4 * hf + (s >> 2);
#pragma unroll
      for (int db = 0; db < NDB; ++db)
        tr[db][hf] = r * D + 8 * ((4 * db + 2 * half + ((s & 3) >> 1)) ^ swz<D>(r)) + 4 * (s & 1);
    }
  }
};

// 16-bit row of a tensor as MFMA B-operand fragments (column j = this row,
// k-group g): NKS fragments of 8 values.
template <int NKS>
__device__ __forceinline__ void load_row_frags(const uint16_t* row, int g, u32x4 (&f)[NKS]) {
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) f[ks] = *(const u32x4*)(row + 16 * ks + 8 * g);
}

// Store an accumulator set (NDB C blocks, lane = output row, elements = dims)
// times `mul` as one 16-bit row.
template <int NDB, bool BF16>
__device__ __forceinline__ void store_row(uint16_t* row, int g, const f32x16 (&acc)[NDB],
                                          float mul) {
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) {
      const int d = db * 32 + 8 * e4 + 4 * g;
      const u32x2 val = {pack2<BF16>(acc[db][4 * e4] * mul, acc[db][4 * e4 + 1] * mul),
                         pack2<BF16>(acc[db][4 * e4 + 2] * mul, acc[db][4 * e4 + 3] * mul)};
      *(u32x2*)(row + d) = val;
    }
}

// The same for the wave's 32 rows (row0 + j) at once, through the wave's own
// LDS region eb (32 rows of 2 D bytes, free for the wave): each lane writes
// its 8-byte pieces there, then every store instruction writes whole rows,
// 16 bytes a lane, instead of 8-byte pieces of 32 rows. Rows at or past
// `limit` are not written. The 16-byte chunk c of row r sits at slot
// c ^ oswz(r), which keeps the writes and the row reads free of bank
// conflicts. The caller puts a barrier between this and the next DMA into the
// region.
template <int NDB, bool BF16>
__device__ __forceinline__ void store_rows_lds(unsigned char* eb, uint16_t* base, int64_t stride,
                                               int row0, int limit, const f32x16 (&acc)[NDB],
                                               float mul) {
  constexpr int ROWB = 64 * NDB, CPR = ROWB / 16, RPI = 64 / CPR;
  static_assert(RPI >= 1, "rows up to 1 KB");
  auto oswz = [](int r) { return CPR >= 16 ? (r & 15) : ((r >> 1) & 7); };
  // (the lane index taken afresh: addresses derived from it are not hoisted
  // into the registers of the kernel's main loop)
  int ln = threadIdx.x & 63;
  asm volatile("" : "+v"(ln));
  const int jr = ln & 31, gr = ln >> 5;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) {
      // dims 8c + 4g .. + 3 of row j, c = 4 db + e4
      const int c = 4 * db + e4;
      const u32x2 val = {pack2<BF16>(acc[db][4 * e4] * mul, acc[db][4 * e4 + 1] * mul),
                         pack2<BF16>(acc[db][4 * e4 + 2] * mul, acc[db][4 * e4 + 3] * mul)};
      *(u32x2*)(eb + jr * ROWB + (c ^ oswz(jr)) * 16 + 8 * gr) = val;
    }
#pragma unroll
  for (int i = 0; i < 32 / RPI; ++i) {
    const int r = RPI * i + ln / CPR, c = ln % CPR;
    const u32x4 val = *(const u32x4*)(eb + r * ROWB + (c ^ oswz(r)) * 16);
    if (row0 + r < limit) *(u32x4*)(base + (int64_t)(row0 + r) * stride + 8 * c) = val;
  }
}

#ifndef MPX_BWD_TAIL_SLOTS
#define MPX_BWD_TAIL_SLOTS 64
#endif
// The same tail for the recomputing dQ / dK/dV launches (off: see bwd_tail_heads).
#ifndef MPX_BWD_TAIL_DQ
#define MPX_BWD_TAIL_DQ 0
#endif
#ifndef MPX_BWD_TAIL_DKDV
#define MPX_BWD_TAIL_DKDV 0
#endif
// Paired launches over n_heads x n_tiles tiles (n_pair = ceil(n_tiles / 2)
// workgroups per head) with n_heads a multiple of the 8 XCDs: the number of
// heads per XCD whose tiles run one per workgroup at the end of the XCD's
// share (about one round of the two workgroups per CU, 64 per XCD), or 0.
// Taken by the stored-dS launches (dropout +0.9% at the headline shape); the
// recomputing dQ and dK/dV pair measured 2% slower with it (tail = false).
__host__ __device__ inline int bwd_tail_heads(int n_heads, int n_tiles, bool tail) {
  const int n_pair = (n_tiles + 1) / 2;
  if (!tail || MPX_BWD_TAIL_SLOTS <= 0 || n_heads % 8 != 0 || n_pair < 2) return 0;
  const int t = (MPX_BWD_TAIL_SLOTS + n_pair - 1) / n_pair;
  return t < n_heads / 8 ? t : 0;
}

// Workgroups of a paired launch (see grid_pair).
inline long bwd_pair_grid(int n_heads, int n_tiles, bool tail) {
  const int n_pair = (n_tiles + 1) / 2, t = bwd_tail_heads(n_heads, n_tiles, tail);
  return (long)n_heads * n_pair + 8L * t * (n_tiles - n_pair);
}

// Workgroup -> (tile pair, head) of a paired launch, as grid_tile over
// n_heads x n_pair, except that the last bwd_tail_heads heads of each XCD run
// their n_tiles tiles one per workgroup after every pair of the XCD: single
// = the rank of this workgroup's tile in longest-first order (else -1). The
// CUs that finish their pairs early take the long tiles, the last ones the
// short ones.
__device__ __forceinline__ void grid_tile(int n_heads, int n_tiles, int& tile, int& head);

__device__ __forceinline__ void grid_pair(int n_heads, int n_tiles, bool tail, int& pt,
                                          int& head, int& single) {
  const int n_pair = (n_tiles + 1) / 2, t = bwd_tail_heads(n_heads, n_tiles, tail);
  single = -1;
  if (t == 0) {
    grid_tile(n_heads, n_pair, pt, head);
    return;
  }
  const int i = blockIdx.x, xcd = i % 8, local = i / 8;
  const int n_paired = (n_heads / 8 - t) * n_pair;
  if (local < n_paired) {
    pt = local % n_pair;
    head = (local / n_pair) * 8 + xcd;
  } else {
    const int k = local - n_paired, r = k / t;
    pt = 0;
    head = (n_heads / 8 - t + (k - r * t)) * 8 + xcd;
    single = r;
  }
}

// Workgroup -> (tile, head) of a launch over n_heads x n_tiles. Workgroup i
// runs on XCD i % 8; with n_heads a multiple of 8, XCD x takes heads x, x + 8,
// ... one at a time, all tiles of a head before the next, so the workgroups
// an XCD runs together share one or two heads' streamed tiles in its L2.
// Otherwise: tile-major (each XCD cycles over all heads).
__device__ __forceinline__ void grid_tile(int n_heads, int n_tiles, int& tile, int& head) {
  const int i = blockIdx.x;
  if (n_heads % 8 == 0) {
    const int xcd = i % 8, local = i / 8;
    tile = local % n_tiles;
    head = (local / n_tiles) * 8 + xcd;
  } else {
    tile = i / n_heads;
    head = i % n_heads;
  }
}

// ---------------------------------------------------------------------------
// dQ: a workgroup owns query rows [128 * qt, +128) of one (batch, head); wave
// w rows +32w. Per KV tile: S^T = K Q^T and dP^T = V dO^T (K, V rows from LDS,
// Q, dO in registers), dS^T = P^T * (dP^T - Dvec), dQ^T += K^T dS^T. Two
// workgroups per CU (two waves per SIMD) hide each other's VALU phases. The
// kernel also forms Dvec = rowsum(dO * O) of its rows in float32 (from the dO
// fragments it holds and the O row) and writes it for the dK/dV kernel that
// runs after it.
// ---------------------------------------------------------------------------
template <int D, bool BF16, bool DROP = false>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(D > 128 ? 1 : 2, D > 128 ? 1 : 2)))
void fa_bwd_dq_kernel(BwdParams p) {
  constexpr int NKS = D / 16, NDB = D / 32, TILE = kBwdTile * D;
  // Stage s: K tile at [2s], V tile at [2s + 1].
  __shared__ __align__(1024) uint16_t lds[4 * TILE];

  const int n_qt = (p.Sq + kBwdOwn - 1) / kBwdOwn;
  // A workgroup runs query tiles n_qt - 1 - pt and pt, the longer (under a
  // causal mask, the last) first: their key-tile counts add up to the same
  // total for every pair, so all workgroups carry equal work.
  int pt, bh, single;
  grid_pair(p.B * p.H, n_qt, MPX_BWD_TAIL_DQ, pt, bh, single);
  const int b = bh / p.H, h = bh % p.H;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 31, g = lane >> 5;

  const int kvh = h / p.kv_group;
  const uint16_t* Q = (const uint16_t*)p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* K = (const uint16_t*)p.k + b * p.k_sb + kvh * p.k_sh;
  const uint16_t* V = (const uint16_t*)p.v + b * p.v_sb + kvh * p.v_sh;
  const uint16_t* dO = (const uint16_t*)p.dout + b * p.do_sb + h * p.do_sh;
  Addr<D> ad;
  ad.init(lane);
  TileDma<D> kd, vd;
  kd.init(p.k_ss, wave, lane);
  vd.init(p.v_ss, wave, lane);
  const u32 lbase = lds_addr(lds);

  for (int pass = 0; pass < 2; ++pass) {
    const int qt = single >= 0 ? n_qt - 1 - single : (pass == 0 ? n_qt - 1 - pt : pt);
    // odd n_qt: the middle tile runs alone
    if (pass == 1 && (single >= 0 || qt == n_qt - 1 - pt)) break;
    const int q0 = qt * kBwdOwn, wq0 = q0 + wave * 32, myq = wq0 + j;
    const int qrow = min(myq, p.Sq - 1);
    u32x4 qf[NKS], df[NKS];
    load_row_frags<NKS>(Q + (int64_t)qrow * p.q_ss, g, qf);
    load_row_frags<NKS>(dO + (int64_t)qrow * p.do_ss, g, df);
    const int64_t rix = (int64_t)bh * p.Sq + qrow;
    const float lse = myq < p.Sq ? p.lse[rix] : INFINITY;
    // Dropout: this row's key of the forward's keep-mask hash.
    const u32 drop_rk = DROP ? drop_row_key((u32)((int64_t)bh * p.Sq + myq), p.seed0) : 0u;
    float dvc;
    {
      // This lane's half of the row (dims 16 ks + 8 g + 0..7), then the pair sum.
      u32x4 of[NKS];
      load_row_frags<NKS>((const uint16_t*)p.o + b * p.o_sb + h * p.o_sh + (int64_t)qrow * p.o_ss,
                          g, of);
      float part = 0.f;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          part += h2f<BF16>((uint16_t)(of[ks][w] & 0xffffu)) *
                  h2f<BF16>((uint16_t)(df[ks][w] & 0xffffu));
          part += h2f<BF16>((uint16_t)(of[ks][w] >> 16)) * h2f<BF16>((uint16_t)(df[ks][w] >> 16));
        }
      dvc = pair_sum32(part);
      if (g == 0 && myq < p.Sq) p.dvec[rix] = dvc;
    }
    // Keys this row sees: [kv_first, kv_last] (rows past Sq have lse = +inf, so
    // their probabilities vanish without a mask).
    const int kv_first = p.win_left >= 0 ? myq - p.win_left : -(1 << 30);
    const int kv_last = min(p.win_right >= 0 ? myq + p.win_right : (1 << 30), p.Sk - 1);

    // KV range of this workgroup's rows.
    const int q_last = min(q0 + kBwdOwn, p.Sq) - 1;
    const int kv_lo = p.win_left >= 0 ? max(0, q0 - p.win_left) : 0;
    const int kv_hi = p.win_right >= 0 ? min(p.Sk, q_last + p.win_right + 1) : p.Sk;
    const int t0 = kv_lo / kBwdTile;
    const int n_t = kv_hi > kv_lo ? (kv_hi - 1) / kBwdTile - t0 + 1 : 0;

    f32x16 dq[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) dq[db] = (f32x16){};

    auto load = [&](int t, int S) __attribute__((always_inline)) {
      const int kv0 = (t0 + t) * kBwdTile;
      kd.load(K, lbase + (2 * S) * TILE * 2, kv0, p.Sk);
      vd.load(V, lbase + (2 * S + 1) * TILE * 2, kv0, p.Sk);
    };
    if (n_t > 0) {
      wait_all();  // Q, dO fragments, lse and Dvec landed before the first DMA
      load(0, 0);
      wait_all();
      stage_barrier();
    }
    // Step t computes stage t % 2 while tile t + 1 lands in the other stage
    // (whose previous tile every wave finished before the last barrier).
    for (int t = 0; t < n_t; ++t) {
      const int S = t & 1;
      if (t + 1 < n_t) load(t + 1, S ^ 1);
      const int kv0 = (t0 + t) * kBwdTile;
      // Wave-level skip of tiles outside every row's window; tiles inside every
      // row's window and below Sk need no mask.
      const bool skip = wq0 >= p.Sq ||
                        (p.win_right >= 0 && kv0 > wq0 + 31 + p.win_right) ||
                        (p.win_left >= 0 && kv0 + kBwdTile - 1 < wq0 - p.win_left);
      const bool full = kv0 + kBwdTile <= p.Sk &&
                        (p.win_right < 0 || kv0 + kBwdTile - 1 <= wq0 + p.win_right) &&
                        (p.win_left < 0 || kv0 >= wq0 + 31 - p.win_left);
      if (!skip) {
        const uint16_t* Kt = lds + 2 * S * TILE;
        const uint16_t* Vt = Kt + TILE;
        // One 32-key block at a time: S^T and dP^T, then dS^T, then its dQ^T terms.
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          f32x16 sb = {}, dpb = {};
          __builtin_amdgcn_s_setprio(1);
#pragma unroll
          for (int kk = 0; kk < NKS; ++kk) {
            const u32x4 ka = *(const u32x4*)(Kt + nb * 32 * D + ad.row[kk]);
            const u32x4 va = *(const u32x4*)(Vt + nb * 32 * D + ad.row[kk]);
            sb = mfma32x32x16<BF16>(ka, qf[kk], sb);
            dpb = mfma32x32x16<BF16>(va, df[kk], dpb);
          }
          __builtin_amdgcn_s_setprio(0);
          // Element 8h + i of the block is key kv0 + 32nb + 16h + 8g + i.
          if (!full) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const int key = kv0 + nb * 32 + 16 * (e >> 3) + 8 * g + (e & 7);
              sb[e] = (key >= kv_first) & (key <= kv_last) ? sb[e] : -INFINITY;
            }
          }
          // dsp[hh]: dS^T of keys 32nb + 16hh + 8g + 0..7, the B operand of k-step 2nb + hh.
          // Dropout: dS = P (dP keep / (1 - p) - Dvec); element pair e2 of half
          // hh is the hash's key pair kv0 / 2 + 16 nb + 8 hh + 4 g + e2.
          u32x4 dsp[2];
          const u32 pair0 =
              DROP ? drop_pair_key((u32)(kv0 >> 1) + 16u * nb + 4u * g, p.seed1) : 0u;
#pragma unroll
          for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int e2 = 0; e2 < 4; ++e2) {
              const int e = 8 * hh + 2 * e2;
              const float p0 = fast_exp2(sb[e] * p.c - lse);
              const float p1 = fast_exp2(sb[e + 1] * p.c - lse);
              if constexpr (DROP) {
                const u32 bits = drop_bits(drop_rk, pair0 + (u32)(8 * hh + e2) * 0x85EBCA77u);
                const float dp0 = (bits & 0xffffu) >= p.drop_thresh ? dpb[e] * p.drop_scale : 0.f;
                const float dp1 = bits >= (p.drop_thresh << 16) ? dpb[e + 1] * p.drop_scale : 0.f;
                dsp[hh][e2] = pack2<BF16>(p0 * (dp0 - dvc), p1 * (dp1 - dvc));
              } else {
                dsp[hh][e2] = pack2<BF16>(p0 * (dpb[e] - dvc), p1 * (dpb[e + 1] - dvc));
              }
            }
          // dQ^T += K^T dS^T (K^T through the transposing read of the K tile).
#pragma unroll
          for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
              const int sl = 2 * nb + hh;
              const u32x2 lo = lds_read_tr16(Kt + ad.tr[db][0] + 16 * sl * D);
              const u32x2 hi = lds_read_tr16(Kt + ad.tr[db][1] + 16 * sl * D);
              dq[db] = mfma32x32x16<BF16>((u32x4){lo[0], lo[1], hi[0], hi[1]}, dsp[hh], dq[db]);
            }
        }
      }
      wait_all();
      stage_barrier();
    }
    // (the stages are free: the last step ended with every wave past its reads
    // and no DMA in flight)
    store_rows_lds<NDB, BF16>((unsigned char*)lds + wave * 64 * D,
                              (uint16_t*)p.dq + b * p.dq_sb + h * p.dq_sh, p.dq_ss, wq0, p.Sq,
                              dq, p.scale);
    stage_barrier();  // every wave's rows read before the next pass stages tiles
  }
}

// ---------------------------------------------------------------------------
// dK, dV: a workgroup owns keys [128 * kt, +128) of one (batch, K/V head);
// wave w keys +32w. Per Q tile (of every query head in the K/V head's group):
// S = Q K^T and dP = dO V^T (Q, dO rows from LDS, the wave's K and V rows in
// registers; lane = key, elements = query rows), P = exp2(S c - lse),
// dS = P * (dP - Dvec), dV^T += dO^T P, dK^T += Q^T dS.
// MODE selects the outputs: kBoth (dK and dV), kOnlyK, kOnlyV. At D = 128
// both accumulator sets take 128 registers and would leave one wave per SIMD,
// so dK and dV run as two kernels of two waves per SIMD each (the dV kernel
// recomputes S, and needs neither dP nor V); at D = 64 one kernel holds both.
// ---------------------------------------------------------------------------
constexpr int kBoth = 0, kOnlyK = 1, kOnlyV = 2;

template <int D, bool BF16, int MODE, bool DROP = false>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(D > 128 ? 1 : 2, D > 128 ? 1 : 2)))
void fa_bwd_dkdv_kernel(BwdParams p) {
  constexpr bool WANT_K = MODE != kOnlyV, WANT_V = MODE != kOnlyK;
  // Streamed Q / dO rows per step: 64, or 32 at D = 256 (four 64-row tiles of
  // 512-byte rows would fill 128 KB of LDS). NBLK 32-row blocks per step.
  constexpr int ROWS = D > 128 ? 32 : kBwdTile, NBLK = ROWS / 32;
  constexpr int NKS = D / 16, NDB = D / 32, TILE = ROWS * D;
  // Stage s: Q tile at [2s], dO tile at [2s + 1].
  __shared__ __align__(1024) uint16_t lds[4 * TILE];
  __shared__ __align__(16) float lse_lds[2][ROWS];
  __shared__ __align__(16) float dvc_lds[2][ROWS];

  const int n_kt = (p.Sk + kBwdOwn - 1) / kBwdOwn;
  int kt, bhk;  // key tile (first, under a causal mask the longest, first), (batch, K/V head)
  grid_tile(p.B * p.H_kv, n_kt, kt, bhk);
  const int b = bhk / p.H_kv, hk = bhk % p.H_kv;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 31, g = lane >> 5;
  const int k0 = kt * kBwdOwn, wk0 = k0 + wave * 32, mykey = wk0 + j;
  const int krow = min(mykey, p.Sk - 1);
  // Queries that see this key: [q_first, q_last] (keys past Sk are never
  // stored, and queries past Sq have lse = +inf).
  const int q_first = p.win_right >= 0 ? mykey - p.win_right : -(1 << 30);
  const int q_last = p.win_left >= 0 ? mykey + p.win_left : (1 << 30);
  // Dropout: this key's pair key of the forward's keep-mask hash and the half
  // of the hash that decides it.
  const u32 drop_pk = DROP ? drop_pair_key((u32)mykey >> 1, p.seed1) : 0u;
  const u32 drop_hm = (mykey & 1) ? 0xffff0000u : 0xffffu;
  const u32 drop_ht = (mykey & 1) ? p.drop_thresh << 16 : p.drop_thresh;

  const uint16_t* K = (const uint16_t*)p.k + b * p.k_sb + hk * p.k_sh;
  const uint16_t* V = (const uint16_t*)p.v + b * p.v_sb + hk * p.v_sh;
  u32x4 kf[NKS], vf[NKS];
  load_row_frags<NKS>(K + (int64_t)krow * p.k_ss, g, kf);
  if constexpr (WANT_K) load_row_frags<NKS>(V + (int64_t)krow * p.v_ss, g, vf);

  // Query range that sees this workgroup's keys; steps run over the query
  // heads of the K/V head's group (outer) and the query tiles (inner).
  const int k_last = min(k0 + kBwdOwn, p.Sk) - 1;
  const int q_lo = p.win_right >= 0 ? max(0, k0 - p.win_right) : 0;
  const int q_hi = p.win_left >= 0 ? min(p.Sq, k_last + p.win_left + 1) : p.Sq;
  const int t0 = q_lo / ROWS;
  const int n_t = q_hi > q_lo ? (q_hi - 1) / ROWS - t0 + 1 : 0;
  const int n_steps = n_t * p.kv_group;

  Addr<D> ad;
  ad.init(lane);
  TileDma<D, ROWS> qd, dd;
  qd.init(p.q_ss, wave, lane);
  dd.init(p.do_ss, wave, lane);
  const u32 lbase = lds_addr(lds);
  f32x16 dk[NDB], dv[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    dk[db] = (f32x16){};
    dv[db] = (f32x16){};
  }

  float lse_r = 0.f, dvc_r = 0.f;  // row threadIdx.x of the tile in flight (first 64 threads)
  // Step u's Q and dO tiles into stage S by DMA, its lse and Dvec rows into registers.
  auto load = [&](int u, int S) __attribute__((always_inline)) {
    const int h = hk * p.kv_group + u / n_t;
    const int row0 = (t0 + u % n_t) * ROWS;
    qd.load((const uint16_t*)p.q + b * p.q_sb + h * p.q_sh, lbase + (2 * S) * TILE * 2, row0,
            p.Sq);
    dd.load((const uint16_t*)p.dout + b * p.do_sb + h * p.do_sh,
            lbase + (2 * S + 1) * TILE * 2, row0, p.Sq);
    if (threadIdx.x < ROWS) {
      const int r = row0 + threadIdx.x;
      const int64_t rix = ((int64_t)b * p.H + h) * p.Sq + r;
      lse_r = r < p.Sq ? p.lse[rix] : INFINITY;
      dvc_r = r < p.Sq ? p.dvec[rix] : 0.f;
    }
  };
  auto store_vec = [&](int S) __attribute__((always_inline)) {
    if (threadIdx.x < ROWS) {
      lse_lds[S][threadIdx.x] = lse_r;
      dvc_lds[S][threadIdx.x] = dvc_r;
    }
  };
  if (n_steps > 0) {
    wait_all();  // K, V fragments landed before the first DMA
    load(0, 0);
    wait_all();
    store_vec(0);
    stage_barrier();
  }
  // Step u computes stage u % 2 while step u + 1's tiles land in the other
  // stage (whose previous tiles every wave finished before the last barrier).
  for (int u = 0; u < n_steps; ++u) {
    const int S = u & 1;
    if (u + 1 < n_steps) load(u + 1, S ^ 1);
    const int qr0 = (t0 + u % n_t) * ROWS;
    // (dropout: row key of query qr0 + 8 g of this step's head)
    const u32 drop_rk =
        DROP ? drop_row_key((u32)(((int64_t)b * p.H + hk * p.kv_group + u / n_t) * p.Sq + qr0 +
                                  8 * g),
                            p.seed0)
             : 0u;
    const bool skip = wk0 >= p.Sk ||
                      (p.win_right >= 0 && wk0 > qr0 + ROWS - 1 + p.win_right) ||
                      (p.win_left >= 0 && wk0 + 31 < qr0 - p.win_left);
    const bool full = (p.win_right < 0 || wk0 + 31 <= qr0 + p.win_right) &&
                      (p.win_left < 0 || wk0 >= qr0 + ROWS - 1 - p.win_left);
    if (!skip) {
      const uint16_t* Qt = lds + 2 * S * TILE;
      const uint16_t* Dt = Qt + TILE;
      const float* lsv = lse_lds[S];
      const float* dvv = dvc_lds[S];
      // One 32-query block at a time (element 8h + i of a block: query row
      // qr0 + 32nb + 16h + 8g + i): S and dP, then P and dS packed as the B
      // operands of k-steps 2nb, 2nb + 1, then their dV^T and dK^T terms.
#pragma unroll
      for (int nb = 0; nb < NBLK; ++nb) {
        f32x16 sb = {}, dpb = {};
#pragma unroll
        for (int kk = 0; kk < NKS; ++kk) {
          const u32x4 qa = *(const u32x4*)(Qt + nb * 32 * D + ad.row[kk]);
          const u32x4 da = *(const u32x4*)(Dt + nb * 32 * D + ad.row[kk]);
          sb = mfma32x32x16<BF16>(qa, kf[kk], sb);
          if constexpr (WANT_K) dpb = mfma32x32x16<BF16>(da, vf[kk], dpb);
        }
        if (!full) {
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int q = qr0 + nb * 32 + 16 * (e >> 3) + 8 * g + (e & 7);
            sb[e] = (q >= q_first) & (q <= q_last) ? sb[e] : -INFINITY;
          }
        }
        u32x4 pp[2], dsp[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int r8 = nb * 32 + 16 * hh + 8 * g;
          const f32x4 l0 = *(const f32x4*)(lsv + r8);
          const f32x4 l1 = *(const f32x4*)(lsv + r8 + 4);
          const f32x4 d0 = *(const f32x4*)(dvv + r8);
          const f32x4 d1 = *(const f32x4*)(dvv + r8 + 4);
#pragma unroll
          for (int e2 = 0; e2 < 4; ++e2) {
            const int e = 8 * hh + 2 * e2;
            const float lv0 = e2 < 2 ? l0[2 * e2] : l1[2 * e2 - 4];
            const float lv1 = e2 < 2 ? l0[2 * e2 + 1] : l1[2 * e2 - 3];
            const float dv0 = e2 < 2 ? d0[2 * e2] : d1[2 * e2 - 4];
            const float dv1 = e2 < 2 ? d0[2 * e2 + 1] : d1[2 * e2 - 3];
            const float p0 = fast_exp2(sb[e] * p.c - lv0);
            const float p1 = fast_exp2(sb[e + 1] * p.c - lv1);
            if constexpr (DROP) {
              // Rows qr0 + r8 + 2 e2 + {0, 1}: row keys drop_rk + (32 nb + 16 hh + 2 e2 + {0, 1}) G.
              const u32 rk0 = drop_rk + (u32)(32 * nb + 16 * hh + 2 * e2) * 0x9E3779B1u;
              const bool k0 = drop_keep(drop_bits(rk0, drop_pk), drop_hm, drop_ht);
              const bool k1 = drop_keep(drop_bits(rk0 + 0x9E3779B1u, drop_pk), drop_hm, drop_ht);
              if constexpr (WANT_V) pp[hh][e2] = pack2<BF16>(k0 ? p0 : 0.f, k1 ? p1 : 0.f);
              if constexpr (WANT_K)
                dsp[hh][e2] = pack2<BF16>(p0 * ((k0 ? dpb[e] * p.drop_scale : 0.f) - dv0),
                                          p1 * ((k1 ? dpb[e + 1] * p.drop_scale : 0.f) - dv1));
            } else {
              if constexpr (WANT_V) pp[hh][e2] = pack2<BF16>(p0, p1);
              if constexpr (WANT_K)
                dsp[hh][e2] = pack2<BF16>(p0 * (dpb[e] - dv0), p1 * (dpb[e + 1] - dv1));
            }
          }
        }
        // dV^T += dO^T P and dK^T += Q^T dS (transposing reads of the tiles).
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const int sl = 2 * nb + hh;
            if constexpr (WANT_V) {
              const u32x2 dlo = lds_read_tr16(Dt + ad.tr[db][0] + 16 * sl * D);
              const u32x2 dhi = lds_read_tr16(Dt + ad.tr[db][1] + 16 * sl * D);
              dv[db] =
                  mfma32x32x16<BF16>((u32x4){dlo[0], dlo[1], dhi[0], dhi[1]}, pp[hh], dv[db]);
            }
            if constexpr (WANT_K) {
              const u32x2 qlo = lds_read_tr16(Qt + ad.tr[db][0] + 16 * sl * D);
              const u32x2 qhi = lds_read_tr16(Qt + ad.tr[db][1] + 16 * sl * D);
              dk[db] =
                  mfma32x32x16<BF16>((u32x4){qlo[0], qlo[1], qhi[0], qhi[1]}, dsp[hh], dk[db]);
            }
          }
      }
    }
    wait_all();
    if (u + 1 < n_steps) store_vec(S ^ 1);
    stage_barrier();
  }
  if (mykey < p.Sk) {
    if constexpr (WANT_K)
      store_row<NDB, BF16>(
          (uint16_t*)p.dk + b * p.dk_sb + hk * p.dk_sh + (int64_t)mykey * p.dk_ss, g, dk,
          p.scale);
    if constexpr (WANT_V)
      store_row<NDB, BF16>(
          (uint16_t*)p.dv + b * p.dv_sb + hk * p.dv_sh + (int64_t)mykey * p.dv_ss, g, dv,
          DROP ? p.drop_scale : 1.f);
  }
}

// ---------------------------------------------------------------------------
// dK and dV in one pass at D = 128. fa_bwd_dkdv_kernel holds both accumulator
// sets next to the wave's K and V rows only at D = 64; here the workgroup's
// 128 K rows sit in LDS (read as the B operand of S = Q K^T), the wave's V
// rows stay in registers, and Q / dO stream in 32-row tiles, two stages:
// 32 KB of K + 32 KB of stages (two workgroups per CU) and two waves per SIMD.
// Per tile: S and dP once, P and dS packed as B operands, then dV^T += dO^T P
// and dK^T += Q^T dS (S is computed twice per backward instead of three times).
// ---------------------------------------------------------------------------
// With DS the kernel also stores each step's dS (the wave's 32 keys x the
// tile's 32 query rows, one 2 KB block) for fa_bwd_dq_ds_kernel; in the block,
// query half hh (rows 16 hh ..) is 1 KB, and the 16 bytes of key k, rows
// 16 hh + 8 g' .. + 7 sit at chunk 32 g' + (k ^ 4 (2 hh + g')) of it: each
// store instruction writes 1 KB contiguously, and the dQ kernel's transposing
// reads of the block are conflict-free.
constexpr int kFusedTile = 32;

template <bool BF16, bool DROP = false, bool DS = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void fa_bwd_dkdv_fused_kernel(BwdParams p) {
  constexpr int D = 128, NKS = D / 16, NDB = D / 32, TILE = kFusedTile * D;
  __shared__ __align__(1024) uint16_t ktile[kBwdOwn * D];
  // Stage s: Q tile at [2s], dO tile at [2s + 1].
  __shared__ __align__(1024) uint16_t lds[4 * TILE];
  // Stage s: lse of the tile's rows at [s][0], Dvec at [s][1], one 64-lane DMA
  // each (the second half holds the 32 rows after the tile, unused).
  __shared__ __align__(16) float vec_lds[2][2][64];
  static_assert(sizeof(ktile) + sizeof(lds) + sizeof(vec_lds) <= 80 * 1024,
                "two workgroups per CU");

  const int n_kt = (p.Sk + kBwdOwn - 1) / kBwdOwn;
  // A workgroup runs key tiles pt and n_kt - 1 - pt, the longer (under a
  // causal mask, the first) first: their step counts add up to the same total
  // for every pair, so all workgroups carry equal work and the launch ends
  // without a tail of long tiles that started late.
  int pt, bhk, single;  // tile pair, (batch, K/V head), single tile rank
  grid_pair(p.B * p.H_kv, n_kt, DS || MPX_BWD_TAIL_DKDV, pt, bhk, single);
  // (scalar: the lse / Dvec DMA descriptors are built from them)
  const int b = __builtin_amdgcn_readfirstlane(bhk / p.H_kv);
  const int hk = __builtin_amdgcn_readfirstlane(bhk % p.H_kv);
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 31, g = lane >> 5;

  const uint16_t* K = (const uint16_t*)p.k + b * p.k_sb + hk * p.k_sh;
  const uint16_t* V = (const uint16_t*)p.v + b * p.v_sb + hk * p.v_sh;
  // B operand of S: K row r = 32 wave + j (the wave's key j), k-group g of
  // step ks, at chunk (2 ks + g) ^ swz(r) = (2 ks ^ km) + kodd (computed per
  // read: an address array would push the kernel past 256 registers).
  const int kswz = swz<D>(32 * wave + j);
  const int kbase = (32 * wave + j) * D + 8 * ((g ^ kswz) & 1), km = kswz & 14;

  // Row operands (A of S and dP): query row perm(j) of the tile, k-group g of
  // step kk, at element rbase + ((16 kk) ^ rx). Transposing reads (A of dV^T
  // and dK^T) for 32-dim block db and row half hf at trb[hf] + ((32 db) ^ tx).
  // Two bases and a mask per family instead of an address per step keep the
  // registers free for operands in flight.
  const int perm = (j & ~12) | ((j & 4) << 1) | ((j & 8) >> 1);
  const int rsw = swz<D>(perm);
  const int rbase = perm * D + 8 * ((g ^ rsw) & 1), rx = 16 * (rsw >> 1);
  const int ts = lane & 15, thalf = (lane >> 4) & 1;
  const int tx = 32 * (ts >> 2);
  int trb[2];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
    trb[hf] = (8 * g + 4 * hf + (ts >> 2)) * D +
              8 * ((2 * thalf + ((ts & 3) >> 1)) ^ (2 * g + hf)) + 4 * (ts & 1);
  TileDma<D, kBwdOwn> kd;
  kd.init(p.k_ss, wave, lane);
  TileDma<D, kFusedTile> qd, dd;
  qd.init(p.q_ss, wave, lane);
  dd.init(p.do_ss, wave, lane);
  const u32 lbase = lds_addr(lds);

  for (int pass = 0; pass < 2; ++pass) {
    const int kt = single >= 0 ? single : (pass == 0 ? pt : n_kt - 1 - pt);
    // odd n_kt: the middle tile runs alone
    if (pass == 1 && (single >= 0 || kt == pt)) break;
    const int k0 = kt * kBwdOwn, wk0 = k0 + wave * 32, mykey = wk0 + j;
    const int krow = min(mykey, p.Sk - 1);
    // Visible query rows of this key, cut at Sq (rows past it are clamped
    // copies with a real row's lse): q - q_first <= span as unsigned (no row
    // at all: q_first = 2^30, span 0).
    // (DS: keys past Sk see no row either, so that their stored dS is zero.)
    const int q_lo_key = p.win_right >= 0 ? mykey - p.win_right : -(1 << 30);
    const int q_last = min(p.win_left >= 0 ? mykey + p.win_left : (1 << 30), p.Sq - 1);
    const bool no_row = q_last < q_lo_key || (DS && mykey >= p.Sk);
    const int q_first = no_row ? (1 << 30) : q_lo_key;
    const unsigned span = no_row ? 0u : (unsigned)q_last - (unsigned)q_first;
    // Dropout: this key's pair key of the forward's keep-mask hash and the
    // half of the hash that decides it.
    const u32 drop_pk = DROP ? drop_pair_key((u32)mykey >> 1, p.seed1) : 0u;
    const u32 drop_hm = (mykey & 1) ? 0xffff0000u : 0xffffu;
    const u32 drop_ht = (mykey & 1) ? p.drop_thresh << 16 : p.drop_thresh;
    u32x4 vf[NKS];
    load_row_frags<NKS>(V + (int64_t)krow * p.v_ss, g, vf);

    const int k_last = min(k0 + kBwdOwn, p.Sk) - 1;
    const int q_lo = p.win_right >= 0 ? max(0, k0 - p.win_right) : 0;
    const int q_hi = p.win_left >= 0 ? min(p.Sq, k_last + p.win_left + 1) : p.Sq;
    const int t0 = q_lo / kFusedTile;
    const int n_t = q_hi > q_lo ? (q_hi - 1) / kFusedTile - t0 + 1 : 0;
    const int n_steps = n_t * p.kv_group;

    f32x16 dk[NDB], dv[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      dk[db] = (f32x16){};
      dv[db] = (f32x16){};
    }

    // (DS) The wave's block of the step being computed: the key tile's first
    // block, query block t0 of head hk * kv_group, key block `wave`; 4 blocks
    // per step, and a head's blocks ds_tot apart.
    char* ds_cur = nullptr;
    if constexpr (DS) {
      int64_t off = 0;
      for (int t = 0; t < kt; ++t) {
        int a, n;
        ds_key_tile(p.Sq, p.Sk, p.win_left, p.win_right, t, a, n);
        off += 4 * n;
      }
      ds_cur = (char*)p.ds +
               (((int64_t)(b * p.H + hk * p.kv_group) * p.ds_tot + off + wave) * kDsBlockBytes);
    }

    // Step u covers query tile t0 + u % n_t of head hk * kv_group + u / n_t; the
    // pair is stepped, not divided, for the tile being loaded (lt, lh) and the
    // tile being computed (ct). Waves 0 and 1 also bring the tile's lse and
    // Dvec rows (clamped at Sq) into LDS.
    int lt = 0, lh = hk * p.kv_group, ct = 0, ch = hk * p.kv_group;
    auto load = [&](int S) __attribute__((always_inline)) {
      const int row0 = (t0 + lt) * kFusedTile;
      if (wave < 2) {
        const float* src = (wave == 0 ? p.lse : p.dvec) + ((int64_t)b * p.H + lh) * p.Sq;
        dma4(buffer_desc(src), lds_addr(vec_lds[S][wave]), min(row0 + lane, p.Sq - 1) * 4);
      }
      qd.load((const uint16_t*)p.q + b * p.q_sb + lh * p.q_sh, lbase + (2 * S) * TILE * 2, row0,
              p.Sq);
      dd.load((const uint16_t*)p.dout + b * p.do_sb + lh * p.do_sh,
              lbase + (2 * S + 1) * TILE * 2, row0, p.Sq);
      if (++lt == n_t) {
        lt = 0;
        ++lh;
      }
    };
    if (n_steps > 0) {
      wait_all();  // V fragments landed before the first DMA
      kd.load(K, lds_addr(ktile), k0, p.Sk);
      load(0);
      wait_all();
      stage_barrier();
    }
    for (int u = 0; u < n_steps; ++u) {
      const int S = u & 1;
      if (u + 1 < n_steps) load(S ^ 1);
      const int qr0 = (t0 + ct) * kFusedTile;
      // (dropout: row key of query qr0 + 8 g of this step's head ch)
      const u32 drop_rk =
          DROP ? drop_row_key((u32)(((int64_t)b * p.H + ch) * p.Sq + qr0 + 8 * g), p.seed0) : 0u;
      char* const ds_blk = ds_cur;
      if constexpr (DS) ds_cur += 4 * kDsBlockBytes;
      if (++ct == n_t) {
        ct = 0;
        ++ch;
        if constexpr (DS) ds_cur += (p.ds_tot - 4 * n_t) * kDsBlockBytes;
      }
      const bool skip = wk0 >= p.Sk ||
                        (p.win_right >= 0 && wk0 > qr0 + kFusedTile - 1 + p.win_right) ||
                        (p.win_left >= 0 && wk0 + 31 < qr0 - p.win_left);
      const bool full = qr0 + kFusedTile <= p.Sq && (!DS || wk0 + 32 <= p.Sk) &&
                        (p.win_right < 0 || wk0 + 31 <= qr0 + p.win_right) &&
                        (p.win_left < 0 || wk0 >= qr0 + kFusedTile - 1 - p.win_left);
      u32x4 dsp[2];
      if (!skip) {
        const float* lsv = vec_lds[S][0];
        const float* dvv = vec_lds[S][1];
        // (opaque copies: the addresses are recomputed every step instead of
        // being hoisted into loop-long registers)
        int kb = kbase, kx = km, rb = rbase + 2 * S * TILE, rxs = rx, t0b = trb[0] + 2 * S * TILE,
            t1b = trb[1] + 2 * S * TILE, txs = tx;
        asm volatile("" : "+v"(kb), "+v"(kx), "+v"(rb), "+v"(rxs), "+v"(t0b), "+v"(t1b), "+v"(txs));
        // S and dP of the tile's 32 query rows (element 8h + i: query qr0 + 16h + 8g + i).
        // The runs of products go at raised wave priority so that the other
        // wave on the SIMD fills the gaps between them rather than the runs.
        __builtin_amdgcn_s_setprio(1);
        f32x16 sb = {}, dpb = {};
#pragma unroll
        for (int kk = 0; kk < NKS; ++kk) {
          const int ro = rb + ((16 * kk) ^ rxs);
          const u32x4 qa = *(const u32x4*)(lds + ro);
          const u32x4 ka = *(const u32x4*)(ktile + kb + 8 * ((2 * kk) ^ kx));
          sb = mfma32x32x16<BF16>(qa, ka, sb);
          const u32x4 da = *(const u32x4*)(lds + ro + TILE);
          dpb = mfma32x32x16<BF16>(da, vf[kk], dpb);
        }
        __builtin_amdgcn_s_setprio(0);
        if (!full) {
          const int qd0 = qr0 + 8 * g - q_first;
#pragma unroll
          for (int e = 0; e < 16; ++e)
            sb[e] = (unsigned)(qd0 + 16 * (e >> 3) + (e & 7)) <= span ? sb[e] : -INFINITY;
        }
        u32x4 pp[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int r8 = 16 * hh + 8 * g;
          const f32x4 l0 = *(const f32x4*)(lsv + r8);
          const f32x4 l1 = *(const f32x4*)(lsv + r8 + 4);
          const f32x4 d0 = *(const f32x4*)(dvv + r8);
          const f32x4 d1 = *(const f32x4*)(dvv + r8 + 4);
#pragma unroll
          for (int e2 = 0; e2 < 4; ++e2) {
            const int e = 8 * hh + 2 * e2;
            const float lv0 = e2 < 2 ? l0[2 * e2] : l1[2 * e2 - 4];
            const float lv1 = e2 < 2 ? l0[2 * e2 + 1] : l1[2 * e2 - 3];
            const float dv0 = e2 < 2 ? d0[2 * e2] : d1[2 * e2 - 4];
            const float dv1 = e2 < 2 ? d0[2 * e2 + 1] : d1[2 * e2 - 3];
            const float p0 = fast_exp2(sb[e] * p.c - lv0);
            const float p1 = fast_exp2(sb[e + 1] * p.c - lv1);
            if constexpr (DROP) {
              // Rows qr0 + r8 + 2 e2 + {0, 1}: row keys drop_rk + (16 hh + 2 e2 + {0, 1}) G.
              const u32 rk0 = drop_rk + (u32)(16 * hh + 2 * e2) * 0x9E3779B1u;
              const bool k0 = drop_keep(drop_bits(rk0, drop_pk), drop_hm, drop_ht);
              const bool k1 = drop_keep(drop_bits(rk0 + 0x9E3779B1u, drop_pk), drop_hm, drop_ht);
              pp[hh][e2] = pack2<BF16>(k0 ? p0 : 0.f, k1 ? p1 : 0.f);
              dsp[hh][e2] = pack2<BF16>(p0 * ((k0 ? dpb[e] * p.drop_scale : 0.f) - dv0),
                                        p1 * ((k1 ? dpb[e + 1] * p.drop_scale : 0.f) - dv1));
            } else {
              pp[hh][e2] = pack2<BF16>(p0, p1);
              dsp[hh][e2] = pack2<BF16>(p0 * (dpb[e] - dv0), p1 * (dpb[e + 1] - dv1));
            }
          }
        }
        // dV^T += dO^T P and dK^T += Q^T dS (transposing reads of the tiles).
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const int o0 = t0b + ((32 * db) ^ txs) + 16 * hh * D;
            const int o1 = t1b + ((32 * db) ^ txs) + 16 * hh * D;
            const u32x2 dlo = lds_read_tr16(lds + o0 + TILE);
            const u32x2 dhi = lds_read_tr16(lds + o1 + TILE);
            dv[db] = mfma32x32x16<BF16>((u32x4){dlo[0], dlo[1], dhi[0], dhi[1]}, pp[hh], dv[db]);
            const u32x2 qlo = lds_read_tr16(lds + o0);
            const u32x2 qhi = lds_read_tr16(lds + o1);
            dk[db] = mfma32x32x16<BF16>((u32x4){qlo[0], qlo[1], qhi[0], qhi[1]}, dsp[hh], dk[db]);
          }
        __builtin_amdgcn_s_setprio(0);
      }
      wait_all();
      stage_barrier();
      // (DS) The step's dS goes out after the wait, so that the next step's
      // wait (vmcnt counts stores too) finds it long written.
      if (DS && !skip) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
          __builtin_nontemporal_store(
              dsp[hh], (u32x4*)(ds_blk + hh * 1024 + (32 * g + (j ^ (4 * (2 * hh + g)))) * 16));
      }
    }
    if (mykey < p.Sk) {
      store_row<NDB, BF16>((uint16_t*)p.dk + b * p.dk_sb + hk * p.dk_sh + (int64_t)mykey * p.dk_ss,
                           g, dk, p.scale);
      store_row<NDB, BF16>((uint16_t*)p.dv + b * p.dv_sb + hk * p.dv_sh + (int64_t)mykey * p.dv_ss,
                           g, dv, DROP ? p.drop_scale : 1.f);
    }
  }
}

// ---------------------------------------------------------------------------
// Dvec = rowsum(dO * O) in float32 for the stored-dS schedule (whose dK/dV
// kernel runs first): one 16-byte chunk of a row per lane, D / 8 lanes per row.
// ---------------------------------------------------------------------------
template <int D, bool BF16>
__global__ __launch_bounds__(256) void fa_bwd_dvec_kernel(BwdParams p) {
  constexpr int CPR = D / 8, RPB = 256 / CPR;
  const int64_t rows = (int64_t)p.B * p.H * p.Sq;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / CPR;
  const int c = threadIdx.x % CPR;
  float part = 0.f;
  if (row < rows) {
    const int64_t bh = row / p.Sq;
    const int s = (int)(row - bh * p.Sq), b = (int)(bh / p.H), h = (int)(bh % p.H);
    const u32x4 o = *(const u32x4*)((const uint16_t*)p.o + b * p.o_sb + h * p.o_sh +
                                    (int64_t)s * p.o_ss + 8 * c);
    const u32x4 d = *(const u32x4*)((const uint16_t*)p.dout + b * p.do_sb + h * p.do_sh +
                                    (int64_t)s * p.do_ss + 8 * c);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      part += h2f<BF16>((uint16_t)(o[w] & 0xffffu)) * h2f<BF16>((uint16_t)(d[w] & 0xffffu));
      part += h2f<BF16>((uint16_t)(o[w] >> 16)) * h2f<BF16>((uint16_t)(d[w] >> 16));
    }
  }
#pragma unroll
  for (int m = CPR / 2; m >= 1; m >>= 1) part += __shfl_xor(part, m);
  if (row < rows && c == 0) p.dvec[row] = part;
}

// ---------------------------------------------------------------------------
// dQ from the stored dS^T: a workgroup owns query rows [128 QB qt, +128 QB) of
// one (batch, head) (wave w: the QB query blocks from 4 QB qt + QB w) and
// streams 64-key steps: the K tile into LDS (shared by the four waves) and
// each wave's dS^T blocks (two key blocks per query block) into its own LDS,
// both by DMA. dQ^T += K^T dS^T with both operands from transposing reads
// (B: column j = query j of the block, k-group = 8 keys); each K^T fragment
// serves the wave's QB query blocks. The dS^T stream bounds the kernel (one
// 2 KB block per 32 x 32 products): NST stages, NST - 1 steps in flight, one
// workgroup per CU.
// ---------------------------------------------------------------------------
template <int QB>
struct DqDsShape {
  static constexpr int kDsBytes = QB * 4096;                 // a wave's dS^T per step
  static constexpr int kStage = kBwdTile * 128 * 2 + kBwdWaves * kDsBytes;  // bytes (D = 128)
  static constexpr int NST = (160 * 1024) / kStage > 4 ? 4 : (160 * 1024) / kStage;
};

template <int D, bool BF16, int QB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void fa_bwd_dq_ds_kernel(BwdParams p) {
  constexpr int NDB = D / 32, TILE = kBwdTile * D;
  constexpr int NST = DqDsShape<QB>::NST, DSB = DqDsShape<QB>::kDsBytes;
  constexpr int OWN = kBwdOwn * QB;                      // query rows per workgroup
  constexpr int NPER = TileDma<D>::NDMA + DSB / 1024;    // DMAs per wave per step
  static_assert(NST >= 2 && NPER * (NST - 2) <= 63, "stages and vmcnt range");
  __shared__ __align__(1024) uint16_t kl[NST * TILE];
  // Stage s, wave w: the wave's blocks at byte (kBwdWaves s + w) * DSB, query
  // block k's two key blocks at + 4096 k.
  __shared__ __align__(1024) uint16_t dsl[NST * kBwdWaves * DSB / 2];

  const int n_qt = (p.Sq + OWN - 1) / OWN;
  // Query tiles n_qt - 1 - pt and pt, as fa_bwd_dq_kernel.
  int pt, bh, single;
  grid_pair(p.B * p.H, n_qt, true, pt, bh, single);
  const int b = bh / p.H, h = bh % p.H;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 5;
  const uint16_t* K = (const uint16_t*)p.k + b * p.k_sb + (h / p.kv_group) * p.k_sh;
  const char* dsh = (const char*)p.ds + (int64_t)bh * p.ds_tot * kDsBlockBytes;
  Addr<D> ad;
  ad.init(lane);
  TileDma<D> kd;
  kd.init(p.k_ss, wave, lane);
  const u32 kbase = lds_addr(kl);
  const u32 dbase = lds_addr(dsl) + (u32)(wave * DSB);
  const char* dsw = (const char*)dsl + wave * DSB;
  // Transposing read of a block (k-step ks of the step: block ks / 2, keys
  // 16 (ks % 2) + 8 g + 4 hf + s / 4, rows 16 gq + 4 (s % 4) .. + 3, s = lane
  // % 16, gq = (lane / 16) % 2) at byte (ks / 2) * 2048 + (ks % 2) * 256 +
  // dtr[hf]: chunk 32 g' + (key ^ 4 (2 gq + g')) of half gq, g' = (s % 4) / 2.
  const int s = lane & 15, gq = (lane >> 4) & 1, gh = (s & 3) >> 1;
  int dtr[2];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const int kq = 8 * g + 4 * hf + (s >> 2);
    dtr[hf] = gq * 1024 + (32 * gh + (kq ^ (4 * (2 * gq + gh)))) * 16 + (s & 1) * 8;
  }

  for (int pass = 0; pass < 2; ++pass) {
    const int qt = single >= 0 ? n_qt - 1 - single : (pass == 0 ? n_qt - 1 - pt : pt);
    // odd n_qt: the middle tile runs alone
    if (pass == 1 && (single >= 0 || qt == n_qt - 1 - pt)) break;
    const int q0 = qt * OWN, wq0 = q0 + wave * 32 * QB;
    const int qb0 = wq0 / 32;  // the wave's first query block
    const int q_last = min(q0 + OWN, p.Sq) - 1;
    const int kv_lo = p.win_left >= 0 ? max(0, q0 - p.win_left) : 0;
    const int kv_hi = p.win_right >= 0 ? min(p.Sk, q_last + p.win_right + 1) : p.Sk;
    const int t0 = kv_lo / kBwdTile;
    const int n_t = kv_hi > kv_lo ? (kv_hi - 1) / kBwdTile - t0 + 1 : 0;

    f32x16 dq[QB][NDB];
#pragma unroll
    for (int k = 0; k < QB; ++k)
#pragma unroll
      for (int db = 0; db < NDB; ++db) dq[k][db] = (f32x16){};

    // Load cursor: key tile lkt of the step being loaded, its first block and
    // query block range (steps are consecutive 64-key halves of key tiles).
    int lkt = t0 / 2, lt0, lnt;
    int64_t loff = 0;
    for (int t = 0; t < lkt; ++t) {
      int a, n;
      ds_key_tile(p.Sq, p.Sk, p.win_left, p.win_right, t, a, n);
      loff += 4 * n;
    }
    ds_key_tile(p.Sq, p.Sk, p.win_left, p.win_right, lkt, lt0, lnt);
    auto load = [&](int t) __attribute__((always_inline)) {
      const int kv0 = (t0 + t) * kBwdTile, kt = kv0 / kBwdOwn, S = t % NST;
      if (kt != lkt) {
        loff += 4 * lnt;
        lkt = kt;
        ds_key_tile(p.Sq, p.Sk, p.win_left, p.win_right, kt, lt0, lnt);
      }
      kd.load(K, kbase + S * TILE * 2, kv0, p.Sk);
      // A query block the key tile has no blocks for reads (and ignores) the
      // buffer's first 4 KB, so that every step issues the same DMAs.
#pragma unroll
      for (int k = 0; k < QB; ++k) {
        const int qb = qb0 + k;
        const bool have = qb >= lt0 && qb < lt0 + lnt;
        const char* src =
            have ? dsh + (loff + 4 * (qb - lt0) + ((kv0 / 32) & 3)) * kDsBlockBytes
                 : (const char*)p.ds;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          dma16_global_s(dbase + (u32)(S * kBwdWaves * DSB + k * 4096 + r * 1024), src + r * 1024,
                         (u32)lane * 16u);
      }
    };
    if (n_t > 0) {
      wait_all();
      for (int t = 0; t < min(n_t, NST - 1); ++t) load(t);
    }
    // Step t: wait for its DMAs, barrier (every wave's part of the K tile has
    // landed, and every wave finished step t - 1, whose stage the load of step
    // t + NST - 1 then overwrites), then compute.
    for (int t = 0; t < n_t; ++t) {
      const int ahead = min(n_t - 1 - t, NST - 2);
      if (NST > 3 && ahead >= 2)
        __builtin_amdgcn_s_waitcnt(0x0F70 | ((2 * NPER) & 15) | (((2 * NPER) >> 4) << 14));
      else if (ahead >= 1)
        __builtin_amdgcn_s_waitcnt(0x0F70 | (NPER & 15) | ((NPER >> 4) << 14));
      else
        __builtin_amdgcn_s_waitcnt(0x0F70);
      stage_barrier();
      if (t + NST - 1 < n_t) load(t + NST - 1);
      const int S = t % NST;
      const int kv0 = (t0 + t) * kBwdTile, kt = kv0 / kBwdOwn;
      int ct0, cnt;
      ds_key_tile(p.Sq, p.Sk, p.win_left, p.win_right, kt, ct0, cnt);
      const uint16_t* Kt = kl + S * TILE;
      const char* Dt = dsw + S * kBwdWaves * DSB;
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
        // Query block k uses the key block's dS^T unless the dK/dV kernel
        // skipped it (no block for the pair, or outside the mask's reach).
        const int kb0 = kv0 + 32 * blk;
        bool use[QB];
        bool any = false;
#pragma unroll
        for (int k = 0; k < QB; ++k) {
          const int qb = qb0 + k, qr = 32 * qb;
          use[k] = qb >= ct0 && qb < ct0 + cnt && kb0 < p.Sk &&
                   !(p.win_right >= 0 && kb0 > qr + 31 + p.win_right) &&
                   !(p.win_left >= 0 && kb0 + 31 < qr - p.win_left);
          any |= use[k];
        }
        if (!any) continue;
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
          const int ks = 2 * blk + k2;
          u32x4 dsb[QB];
#pragma unroll
          for (int k = 0; k < QB; ++k) {
            const char* a = Dt + k * 4096 + blk * kDsBlockBytes + k2 * 256;
            const u32x2 dlo = lds_read_tr16(a + dtr[0]);
            const u32x2 dhi = lds_read_tr16(a + dtr[1]);
            // (a block the pair does not use contributes zero)
            dsb[k] = use[k] ? (u32x4){dlo[0], dlo[1], dhi[0], dhi[1]} : (u32x4){0u, 0u, 0u, 0u};
          }
#pragma unroll
          for (int db = 0; db < NDB; ++db) {
            const u32x2 lo = lds_read_tr16(Kt + ad.tr[db][0] + 16 * ks * D);
            const u32x2 hi = lds_read_tr16(Kt + ad.tr[db][1] + 16 * ks * D);
            const u32x4 ka = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
            for (int k = 0; k < QB; ++k) dq[k][db] = mfma32x32x16<BF16>(ka, dsb[k], dq[k][db]);
          }
        }
      }
    }
    stage_barrier();  // every wave done with the stages (the last step waited for every DMA)
    // The wave's query blocks go out through its own 64 D bytes of the K tile
    // stages, one block after the other.
    static_assert(kBwdWaves * 64 * D <= sizeof(kl), "a region per wave");
#pragma unroll
    for (int k = 0; k < QB; ++k)
      store_rows_lds<NDB, BF16>((unsigned char*)kl + wave * 64 * D,
                                (uint16_t*)p.dq + b * p.dq_sb + h * p.dq_sh, p.dq_ss,
                                wq0 + 32 * k, p.Sq, dq[k], p.scale);
    stage_barrier();  // every wave's rows read before the next pass loads
  }
}

constexpr int kDqDsQB = 2;  // query blocks per wave of fa_bwd_dq_ds_kernel

template <int D, bool BF16, bool DROP>
hipError_t launch_bwd(const BwdParams& p, hipStream_t st) {
  const int n_qt = (p.Sq + kBwdOwn - 1) / kBwdOwn, n_kt = (p.Sk + kBwdOwn - 1) / kBwdOwn;
  if constexpr (D == 128) {
    if (p.ds != nullptr) {
      // Stored dS: Dvec, then dK / dV (which stores dS), then dQ = scale dS K.
      const long rows = (long)p.B * p.H * p.Sq;
      hipLaunchKernelGGL((fa_bwd_dvec_kernel<D, BF16>), dim3((rows + 15) / 16), dim3(256), 0, st,
                         p);
      hipLaunchKernelGGL((fa_bwd_dkdv_fused_kernel<BF16, DROP, true>),
                         dim3(bwd_pair_grid(p.B * p.H_kv, n_kt, true)), dim3(256), 0, st, p);
      const int n_qt2 = (p.Sq + kBwdOwn * kDqDsQB - 1) / (kBwdOwn * kDqDsQB);
      hipLaunchKernelGGL((fa_bwd_dq_ds_kernel<D, BF16, kDqDsQB>),
                         dim3(bwd_pair_grid(p.B * p.H, n_qt2, true)), dim3(256), 0, st, p);
      return hipGetLastError();
    }
  }
  // dQ (which also writes Dvec) before dK / dV, which reads it.
  hipLaunchKernelGGL((fa_bwd_dq_kernel<D, BF16, DROP>),
                     dim3(bwd_pair_grid(p.B * p.H, n_qt, MPX_BWD_TAIL_DQ)), dim3(256), 0, st, p);
  const dim3 grid_kv(p.B * p.H_kv * n_kt);
  if constexpr (D == 128) {
    const dim3 grid_pairs(bwd_pair_grid(p.B * p.H_kv, n_kt, MPX_BWD_TAIL_DKDV));
    hipLaunchKernelGGL((fa_bwd_dkdv_fused_kernel<BF16, DROP>), grid_pairs, dim3(256), 0, st, p);
  } else {  // D = 64, and D = 256 (one wave per SIMD)
    hipLaunchKernelGGL((fa_bwd_dkdv_kernel<D, BF16, kBoth, DROP>), grid_kv, dim3(256), 0, st, p);
  }
  return hipGetLastError();
}

template <bool BF16, bool DROP>
hipError_t launch_bwd_d(const BwdParams& p, int D, hipStream_t st) {
  if (D == 64) return launch_bwd<64, BF16, DROP>(p, st);
  if (D == 256) return launch_bwd<256, BF16, DROP>(p, st);
  return launch_bwd<128, BF16, DROP>(p, st);
}

}  // namespace mpx

using namespace mpx;

extern "C" size_t mpx_attn_bwd_workspace_bytes(int B, int H, int Sq) {
  if (B <= 0 || H <= 0 || Sq <= 0) return 0;
  return (size_t)B * H * Sq * sizeof(float);
}

// Stored dS^T blocks per query head (the key tiles' block counts summed).
static int64_t ds_blocks_per_head(int Sq, int Sk, int win_left, int win_right) {
  const int n_kt = (Sk + kBwdOwn - 1) / kBwdOwn;
  int64_t tot = 0;
  for (int kt = 0; kt < n_kt; ++kt) {
    int t0, nt;
    ds_key_tile(Sq, Sk, win_left, win_right, kt, t0, nt);
    tot += 4 * nt;
  }
  return tot;
}

// Bytes of Dvec rounded up to 256: the stored dS^T starts there.
static size_t dvec_region_bytes(int B, int H, int Sq) {
  return (mpx_attn_bwd_workspace_bytes(B, H, Sq) + 255) & ~(size_t)255;
}

extern "C" size_t mpx_attn_bwd_ds_workspace_bytes(int B, int H, int Sq, int Sk, int D, int dtype,
                                                  int causal, int window_left,
                                                  int window_right) {
  if (B <= 0 || H <= 0 || Sq <= 0 || Sk <= 0 || D != 128 ||
      (dtype != MPX_F16 && dtype != MPX_BF16))
    return 0;
  const int wl = window_left < 0 ? -1 : window_left;
  const int wr = causal ? 0 : (window_right < 0 ? -1 : window_right);
  const int64_t blocks = (int64_t)B * H * ds_blocks_per_head(Sq, Sk, wl, wr);
  // (at least 4 KB: the dQ kernel's placeholder reads)
  return dvec_region_bytes(B, H, Sq) + (size_t)std::max<int64_t>(blocks, 2) * kDsBlockBytes;
}

static int attn_bwd_entry(const void* q, const void* k, const void* v, const void* o,
                          const void* dout, const float* lse, void* dq, void* dk, void* dv,
                          const int64_t* q_strides, const int64_t* k_strides,
                          const int64_t* v_strides, const int64_t* o_strides,
                          const int64_t* do_strides, const int64_t* dq_strides,
                          const int64_t* dk_strides, const int64_t* dv_strides, int B, int H,
                          int H_kv, int Sq, int Sk, int D, float scale, int causal,
                          int window_left, int window_right, int dtype, float dropout_p,
                          uint64_t seed, void* workspace, size_t workspace_bytes, void* stream) {
  MPX_CHECK_ARG(dropout_p >= 0.f && dropout_p < 1.f,
                "mpx_attn_bwd_dropout: dropout_p must be in [0, 1), got %g", (double)dropout_p);
  MPX_CHECK_ARG(dtype == MPX_F32 || dtype == MPX_F16 || dtype == MPX_BF16,
                "mpx_attn_bwd: unknown dtype code %d", dtype);
  MPX_CHECK_ARG(B >= 0 && H >= 0 && Sq >= 0 && Sk >= 0, "mpx_attn_bwd: negative size");
  MPX_CHECK_ARG(H_kv > 0 ? H % H_kv == 0 : H == 0,
                "mpx_attn_bwd: %d query heads are not a multiple of %d K/V heads", H, H_kv);
  if (D != 64 && D != 128 && D != 256) {
    set_error("mpx_attn_bwd: head_dim %d not supported (backward kernels exist for 64, 128, "
              "256)", D);
    return MPX_EUNSUPPORTED;
  }
  MPX_CHECK_ARG(std::isfinite(scale) && scale > 0.f, "mpx_attn_bwd: scale must be positive");
  if ((long)B * H == 0 || (Sq == 0 && Sk == 0)) return MPX_OK;
  MPX_CHECK_ARG(Sq > 0 && Sk > 0, "mpx_attn_bwd: empty query or key sequence");
  const void* ptrs[9] = {q, k, v, o, dout, lse, dq, dk, dv};
  for (int i = 0; i < 9; ++i) MPX_CHECK_ARG(ptrs[i] != nullptr, "mpx_attn_bwd: null pointer");
  for (int i = 0; i < 9; ++i)
    MPX_CHECK_ARG(((uintptr_t)ptrs[i] & 15u) == 0, "mpx_attn_bwd: tensors must be 16-byte aligned");
  const int64_t* all[8] = {q_strides, k_strides, v_strides, o_strides,
                           do_strides, dq_strides, dk_strides, dv_strides};
  const int vec = dtype == MPX_F32 ? 4 : 8;
  for (int t = 0; t < 8; ++t) {
    MPX_CHECK_ARG(all[t] != nullptr, "mpx_attn_bwd: null strides");
    for (int i = 0; i < 3; ++i)
      MPX_CHECK_ARG(all[t][i] >= 0 && all[t][i] % vec == 0,
                    "mpx_attn_bwd: strides must be non-negative multiples of %d elements", vec);
  }
  const size_t need = mpx_attn_bwd_workspace_bytes(B, H, Sq);
  MPX_CHECK_ARG(workspace != nullptr && workspace_bytes >= need &&
                    ((uintptr_t)workspace & 15u) == 0,
                "mpx_attn_bwd: 16-byte aligned workspace of %zu bytes required, %zu given", need,
                workspace_bytes);
  // The kernels address one (batch, head) of q, dout, k, v with 32-bit byte offsets.
  const int64_t span = std::max((int64_t)Sq + kBwdTile, (int64_t)Sk + kBwdTile) * 2 *
                       std::max(std::max(q_strides[2], do_strides[2]),
                                std::max(k_strides[2], v_strides[2]));
  if (dtype != MPX_F32 && span >= (1LL << 31)) {
    set_error("mpx_attn_bwd: seq_len * seq_stride exceeds the 2 GiB addressing range of one head");
    return MPX_EUNSUPPORTED;
  }
  const long tiles = (long)B * H * (((Sq > Sk ? Sq : Sk) + kBwdOwn - 1) / kBwdOwn);
  MPX_CHECK_ARG(tiles < (1L << 31) && (long)B * H * Sq < (1L << 35),
                "mpx_attn_bwd: problem too large");

  BwdParams p = {};
  p.q = q; p.k = k; p.v = v; p.o = o; p.dout = dout; p.lse = lse;
  p.dvec = (float*)workspace; p.dq = dq; p.dk = dk; p.dv = dv;
  p.q_sb = q_strides[0]; p.q_sh = q_strides[1]; p.q_ss = q_strides[2];
  p.k_sb = k_strides[0]; p.k_sh = k_strides[1]; p.k_ss = k_strides[2];
  p.v_sb = v_strides[0]; p.v_sh = v_strides[1]; p.v_ss = v_strides[2];
  p.o_sb = o_strides[0]; p.o_sh = o_strides[1]; p.o_ss = o_strides[2];
  p.do_sb = do_strides[0]; p.do_sh = do_strides[1]; p.do_ss = do_strides[2];
  p.dq_sb = dq_strides[0]; p.dq_sh = dq_strides[1]; p.dq_ss = dq_strides[2];
  p.dk_sb = dk_strides[0]; p.dk_sh = dk_strides[1]; p.dk_ss = dk_strides[2];
  p.dv_sb = dv_strides[0]; p.dv_sh = dv_strides[1]; p.dv_ss = dv_strides[2];
  p.B = B; p.H = H; p.H_kv = H_kv; p.kv_group = H / H_kv; p.Sq = Sq; p.Sk = Sk;
  p.win_left = window_left < 0 ? -1 : window_left;
  p.win_right = causal ? 0 : (window_right < 0 ? -1 : window_right);
  p.scale = scale;
  p.c = scale * kLog2e;
  const bool drop = dropout_p > 0.f;
  if (drop) {
    p.drop_thresh = drop_threshold(dropout_p);
    p.seed0 = (uint32_t)seed;
    p.seed1 = (uint32_t)(seed >> 32);
    p.drop_scale = 1.f / (1.f - dropout_p);
  }
  // The stored-dS schedule when the workspace holds it.
  const size_t ds_need = mpx_attn_bwd_ds_workspace_bytes(B, H, Sq, Sk, D, dtype, causal,
                                                         window_left, window_right);
  if (ds_need > 0 && workspace_bytes >= ds_need) {
    p.ds = (char*)workspace + dvec_region_bytes(B, H, Sq);
    p.ds_tot = ds_blocks_per_head(Sq, Sk, p.win_left, p.win_right);
  }
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (dtype == MPX_F32)
    e = launch_bwd32(p, D, drop, st);
  else if (dtype == MPX_BF16)
    e = drop ? launch_bwd_d<true, true>(p, D, st) : launch_bwd_d<true, false>(p, D, st);
  else
    e = drop ? launch_bwd_d<false, true>(p, D, st) : launch_bwd_d<false, false>(p, D, st);
  MPX_CHECK_HIP(e);
  return MPX_OK;
}

extern "C" int mpx_attn_bwd(const void* q, const void* k, const void* v, const void* o,
                            const void* dout, const float* lse, void* dq, void* dk, void* dv,
                            const int64_t* q_strides, const int64_t* k_strides,
                            const int64_t* v_strides, const int64_t* o_strides,
                            const int64_t* do_strides, const int64_t* dq_strides,
                            const int64_t* dk_strides, const int64_t* dv_strides, int B, int H,
                            int H_kv, int Sq, int Sk, int D, float scale, int causal,
                            int window_left, int window_right, int dtype, void* workspace,
                            size_t workspace_bytes, void* stream) {
  clear_error();
  return attn_bwd_entry(q, k, v, o, dout, lse, dq, dk, dv, q_strides, k_strides, v_strides,
                        o_strides, do_strides, dq_strides, dk_strides, dv_strides, B, H, H_kv, Sq,
                        Sk, D, scale, causal, window_left, window_right, dtype, 0.f, 0, workspace,
                        workspace_bytes, stream);
}

extern "C" int mpx_attn_bwd_dropout(const void* q, const void* k, const void* v, const void* o,
                                    const void* dout, const float* lse, void* dq, void* dk,
                                    void* dv, const int64_t* q_strides,
                                    const int64_t* k_strides, const int64_t* v_strides,
                                    const int64_t* o_strides, const int64_t* do_strides,
                                    const int64_t* dq_strides, const int64_t* dk_strides,
                                    const int64_t* dv_strides, int B, int H, int H_kv, int Sq,
                                    int Sk, int D, float scale, int causal, int window_left,
                                    int window_right, int dtype, float dropout_p, uint64_t seed,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  return attn_bwd_entry(q, k, v, o, dout, lse, dq, dk, dv, q_strides, k_strides, v_strides,
                        o_strides, do_strides, dq_strides, dk_strides, dv_strides, B, H, H_kv, Sq,
                        Sk, D, scale, causal, window_left, window_right, dtype, dropout_p, seed,
                        workspace, workspace_bytes, stream);
}
