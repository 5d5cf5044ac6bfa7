// Exact-softmax attention forward for gfx950 (MI355X): launches, split-KV
// planning and the C-ABI entry points of flash / sliding-window /
// chunked-cross attention and paged prefill. The kernels and their algorithm
// are in fa_fwd_kernels.h.
#include "fa_fwd_kernels.h"

namespace mpx {

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
// The dropout forward launches (fa_fwd_drop.hip).
hipError_t dispatch_fwd_drop(const FwdParams& p, int D, int dtype, int grid, hipStream_t st);

namespace {

constexpr int kNumCUs = 256;
constexpr int kNumXcds = 8;
#ifndef MPX_FA_TAIL_SLOTS
#define MPX_FA_TAIL_SLOTS 32
#endif
constexpr int kTailSlots = MPX_FA_TAIL_SLOTS;  // one XCD's CUs

// Workgroups a split launch aims for: one full wave of resident workgroups.
// The 16-bit kernels at D >= 64 hold 96-128 KB of LDS (one workgroup per CU);
// the others fit two per CU.
int target_workgroups(int D, int dtype) {
  return dtype != MPX_F32 && D >= 64 ? kNumCUs : 2 * kNumCUs;
}

struct Plan {
  int BM, BN, n_qtiles, splits, tiles_per_split, win_left, win_right;
  int n_slots, paired, win_first;
  int tail_bh;  // paired: (batch, head)s per XCD run as single q-tiles at the end
  int var_split;  // splits per (batch, head) when each q-tile has its own count, else 0
  size_t ws_bytes;
};

// Paged 16-bit kernels at D = 128 take 128-key tiles (page ids read from the
// table a step ahead) when pages are a power of two of at least the 4 rows one
// DMA instruction of a wave stages, and no ALiBi bias is given.
bool paged_wide_tiles(int D, int dtype, int bs_log2, bool alibi) {
  // Page sizes 4 .. 128 divide the tile: every tile starts on a page boundary.
  return MPX_FA_DIRECT && dtype != MPX_F32 && D == 128 && bs_log2 >= 2 && bs_log2 <= 7 &&
         !alibi;
}

// Keys per KV tile (the D = 32 16-bit kernels, and the paged ones at other
// page sizes, take 64).
int tile_n(int D, int dtype, bool paged = false, int bs_log2 = -1, bool alibi = false) {
  if (dtype == MPX_F32) return D > 64 ? 32 : 64;
  if (D > 128) return paged ? 32 : 64;
  if (paged) return paged_wide_tiles(D, dtype, bs_log2, alibi) ? 128 : 64;
  return D < 64 || !MPX_FA_DIRECT ? 64 : MPX_FA_BN16;
}

Plan make_plan(int B, int H, int Sq, int Sk, int D, int causal, int window_left,
               int window_right, int dtype, int max_tiles_per_split = 1 << 30,
               bool paged = false, int bs_log2 = -1, bool alibi = false) {
  Plan pl;
  pl.BM = 32 * (dtype == MPX_F32 ? kNumWaves32 : (D > 128 ? kNumWavesWide : kNumWaves16));
  pl.BN = tile_n(D, dtype, paged, bs_log2, alibi);
  pl.win_left = window_left < 0 ? -1 : window_left;
  pl.win_right = causal ? 0 : (window_right < 0 ? -1 : window_right);
  pl.n_qtiles = (Sq + pl.BM - 1) / pl.BM;
  // Widest KV range over all q-tiles.
  int max_tiles = 0;
  for (int qt = 0; qt < pl.n_qtiles; ++qt)
    max_tiles = std::max(max_tiles, qtile_kv_tiles(qt, pl.BM, pl.BN, Sq, Sk, pl.win_left,
                                                   pl.win_right));
  const long base = (long)B * H * pl.n_qtiles;
  int splits = 1;
  const long target = target_workgroups(D, dtype);
  if (base > 0 && base < target && max_tiles >= 8) {
    splits = (int)std::min<long>((target + base - 1) / base, max_tiles / 4);
    splits = std::max(splits, 1);
  }
  pl.tiles_per_split = splits > 1 ? (max_tiles + splits - 1) / splits : std::max(max_tiles, 1);
  pl.tiles_per_split = std::min(pl.tiles_per_split, std::max(max_tiles_per_split, 1));
  splits = std::max(1, (max_tiles + pl.tiles_per_split - 1) / pl.tiles_per_split);
  pl.splits = splits;
  pl.ws_bytes = splits > 1 ? (size_t)splits * B * H * Sq * (D + 2) * sizeof(float) : 0;
  // Causal-shaped launches (KV range growing with the q-tile) of the 16-bit
  // kernel pair q-tiles into equal-work slots while that still leaves a full
  // wave of workgroups for the CUs.
  const int half = (pl.n_qtiles + 1) / 2;
  pl.paired = dtype != MPX_F32 && splits == 1 && pl.win_left < 0 && pl.win_right >= 0 &&
              pl.n_qtiles >= 2 && (long)B * H * half >= kNumCUs;
  pl.n_slots = pl.paired ? half : pl.n_qtiles;
  // One-workgroup-per-CU paired launches end with single q-tiles, longest
  // first, in place of the last ~round of pairs on each XCD (kTailSlots
  // pairs' worth of (batch, head)s): the XCD's CUs then finish within about
  // one short q-tile of each other. (Measured at B=4, H=32, S=4096, D=128
  // causal bf16: +2.2% with 32 slots, less with 16 or 64; the head-dim-256
  // kernel, 128-row q-tiles, -1.3%.)
  pl.tail_bh = 0;
  if (pl.paired && kTailSlots > 0 && (long)B * H % kNumXcds == 0 && D <= 128 &&
      target_workgroups(D, dtype) == kNumCUs) {
    const long bpx = (long)B * H / kNumXcds;
    const long t = (kTailSlots + pl.n_slots - 1) / pl.n_slots;
    if (t < bpx) pl.tail_bh = (int)t;
  }
  pl.win_first = -1;
  if (!pl.paired && pl.win_left >= 0) {
    pl.win_first = 0;
    while (pl.win_first < pl.n_qtiles - 1 &&
           qtile_kv_tiles(pl.win_first, pl.BM, pl.BN, Sq, Sk, pl.win_left, pl.win_right) <
               max_tiles)
      ++pl.win_first;
  }
  // Ranges of unequal length (causal, windows) split by one tile count leave
  // short q-tiles with empty splits and long ones with many: instead, each
  // q-tile gets ceil(its tiles / T) splits of T tiles, with the smallest T (at
  // least 4) whose launch fits one resident wave of workgroups.
  pl.var_split = 0;
  if (splits > 1 && !pl.paired && pl.n_qtiles <= 64) {
    const int cap = std::max(max_tiles_per_split, 1);
    for (int T = 4; T <= std::min(max_tiles, cap); ++T) {
      long per_bh = 0;
      for (int qt = 0; qt < pl.n_qtiles; ++qt)
        per_bh += qtile_splits(qt, pl.BM, pl.BN, Sq, Sk, pl.win_left, pl.win_right, T);
      if ((long)B * H * per_bh > target) continue;
      if (per_bh < (long)pl.n_qtiles * splits) {
        pl.var_split = (int)per_bh;
        pl.tiles_per_split = T;
        pl.splits = (max_tiles + T - 1) / T;
        pl.ws_bytes = (size_t)pl.splits * B * H * Sq * (D + 2) * sizeof(float);
      }
      break;
    }
  }
  return pl;
}

// BIG: 16-bit paged pools of 4 GiB and more (p.pool_bytes == 0).
template <int D, int BN, bool F32, bool BF16, bool PAGED, bool BIG = false>
hipError_t launch_fwd(const FwdParams& p, int grid, hipStream_t stream) {
  if constexpr (F32) {
    hipLaunchKernelGGL((fa_fwd32_kernel<D, BN, kNumWaves32, PAGED>), dim3(grid),
                       dim3(64 * kNumWaves32), 0, stream, p);
  } else {
    hipLaunchKernelGGL((fa_fwd16_kernel<D, BN, kNumWaves16, BF16, PAGED, BIG>), dim3(grid),
                       dim3(64 * kNumWaves16), 0, stream, p);
  }
  return hipGetLastError();
}

template <bool PAGED, bool BIG = false>
hipError_t dispatch_fwd(const FwdParams& p, int D, int dtype, int grid, hipStream_t st) {
  if constexpr (PAGED && !BIG) {
    // 16-bit pools of 4 GiB and more: the 64-bit address forms
    if (dtype != MPX_F32 && p.pool_bytes == 0) return dispatch_fwd<true, true>(p, D, dtype, grid, st);
  }
  if (D == 256) {
    // (16-bit: 64-key DMA-staged tiles dense, 32-key register-staged paged)
    constexpr int kBNw = PAGED ? 32 : 64;
    if (dtype == MPX_F32) return launch_fwd<256, 32, true, false, PAGED>(p, grid, st);
    if (dtype == MPX_BF16)
      hipLaunchKernelGGL((fa_fwd16_wide_kernel<256, kBNw, kNumWavesWide, true, PAGED, false, BIG>),
                         dim3(grid), dim3(64 * kNumWavesWide), 0, st, p);
    else
      hipLaunchKernelGGL((fa_fwd16_wide_kernel<256, kBNw, kNumWavesWide, false, PAGED, false, BIG>),
                         dim3(grid), dim3(64 * kNumWavesWide), 0, st, p);
    return hipGetLastError();
  }
  if constexpr (PAGED) {
    if (paged_wide_tiles(D, dtype, p.bs_log2, p.slopes != nullptr)) {
      return dtype == MPX_BF16 ? launch_fwd<128, 128, false, true, true, BIG>(p, grid, st)
                               : launch_fwd<128, 128, false, false, true, BIG>(p, grid, st);
    }
  }
  if (dtype == MPX_F32) {
    switch (D) {
      case 32: return launch_fwd<32, 64, true, false, PAGED>(p, grid, st);
      case 64: return launch_fwd<64, 64, true, false, PAGED>(p, grid, st);
      default: return launch_fwd<128, 32, true, false, PAGED>(p, grid, st);
    }
  } else if (dtype == MPX_BF16) {
    switch (D) {
      case 32: return launch_fwd<32, kBN16<PAGED, 32>, false, true, PAGED, BIG>(p, grid, st);
      case 64: return launch_fwd<64, kBN16<PAGED, 64>, false, true, PAGED, BIG>(p, grid, st);
      default: return launch_fwd<128, kBN16<PAGED, 128>, false, true, PAGED, BIG>(p, grid, st);
    }
  } else {
    switch (D) {
      case 32: return launch_fwd<32, kBN16<PAGED, 32>, false, false, PAGED, BIG>(p, grid, st);
      case 64: return launch_fwd<64, kBN16<PAGED, 64>, false, false, PAGED, BIG>(p, grid, st);
      default: return launch_fwd<128, kBN16<PAGED, 128>, false, false, PAGED, BIG>(p, grid, st);
    }
  }
}

// Attention kernel(s) for a prepared FwdParams: the forward launch (with
// dropout: the dropout kernels), then the split merge when the plan splits
// the KV range.
template <bool PAGED>
int run_fwd(FwdParams& p, const Plan& pl, int D, int dtype, void* workspace, hipStream_t st,
            bool drop = false) {
  p.ws_o = pl.splits > 1 ? (float*)workspace : nullptr;
  p.ws_ml = pl.splits > 1 ? (float*)workspace + (size_t)pl.splits * p.B * p.H * p.Sq * D : nullptr;
  p.win_left = pl.win_left; p.win_right = pl.win_right;
  p.n_qtiles = pl.n_qtiles; p.num_splits = pl.splits; p.tiles_per_split = pl.tiles_per_split;
  p.n_slots = pl.n_slots; p.paired = pl.paired; p.tail_bh = pl.tail_bh;
  p.var_split = pl.var_split; p.bm = pl.BM; p.bn = pl.BN; p.win_first = pl.win_first;
  const long grid_l =
      pl.tail_bh > 0
          ? (long)p.B * p.H * pl.n_slots + (long)kNumXcds * pl.tail_bh * (pl.n_qtiles - pl.n_slots)
          : (long)p.B * p.H * (pl.var_split > 0 ? pl.var_split : (long)pl.n_slots * pl.splits);
  MPX_CHECK_ARG(grid_l < (1L << 31), "attention: problem too large");
  if (!PAGED && drop)
    MPX_CHECK_HIP(dispatch_fwd_drop(p, D, dtype, (int)grid_l, st));
  else
    MPX_CHECK_HIP(dispatch_fwd<PAGED>(p, D, dtype, (int)grid_l, st));
  if (pl.splits > 1) {
    const MergeShape ms = {pl.var_split, pl.BM, pl.BN, p.Sk, pl.win_left, pl.win_right,
                           pl.tiles_per_split};
    const long threads = (long)p.B * p.H * p.Sq * (D / 4);
    const int blocks = (int)((threads + 255) / 256);
#define MPX_MERGE(DT)                                                                         \
  hipLaunchKernelGGL(fa_split_merge_kernel<DT>, dim3(blocks), dim3(256), 0, st, p.ws_o, p.ws_ml, \
                     p.o, p.o_sb, p.o_sh, p.o_ss, p.B, p.H, p.Sq, D, pl.splits, p.eps,         \
                     p.nan_empty, p.lse, ms)
    if (dtype == MPX_F32)
      MPX_MERGE(MPX_F32);
    else if (dtype == MPX_BF16)
      MPX_MERGE(MPX_BF16);
    else
      MPX_MERGE(MPX_F16);
#undef MPX_MERGE
    MPX_CHECK_HIP(hipGetLastError());
  }
  return MPX_OK;
}

// Output rows of a query that can see no key at all (empty pool): NaN, as the
// reference's softmax over an all -inf row.
template <int DT>
__global__ void fill_nan_kernel(void* o, int64_t o_sb, int64_t o_sh, int64_t o_ss, int B, int H,
                                int Sq, int D) {
  const int64_t n = (int64_t)B * H * Sq * D;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int d = (int)(i % D);
    const int64_t r = i / D;
    const int q = (int)(r % Sq);
    const int64_t bh = r / Sq;
    const int b = (int)(bh / H), h = (int)(bh % H);
    const int64_t off = b * o_sb + h * o_sh + q * o_ss + d;
    if constexpr (DT == MPX_F32)
      ((float*)o)[off] = __builtin_nanf("");
    else
      ((uint16_t*)o)[off] = DT == MPX_BF16 ? 0x7FC0 : 0x7E00;
  }
}

// Tiles per split so that one work item's pages fit the LDS page table.
// Tiles per split item of a paged launch: the 64-key kernels stage the item's
// page ids in LDS (at most kMaxItemPages); the 128-key ones read them from the
// table and take any number.
int paged_tile_cap(int block_size, int BN) {
  if (BN == 128) return 1 << 30;
  return std::max(1, (int)std::min<long>(1L << 30, (long)(kMaxItemPages - 2) * block_size / BN));
}

int log2_if_pow2(int x) { return x > 0 && (x & (x - 1)) == 0 ? __builtin_ctz((unsigned)x) : -1; }

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

}  // namespace
}  // namespace mpx

using namespace mpx;

extern "C" size_t mpx_attn_fwd_workspace_bytes(int B, int H, int Sq, int Sk, int D, int causal,
                                               int window_left, int window_right, int dtype) {
  if (B <= 0 || H <= 0 || Sq <= 0 || Sk <= 0 || D <= 0) return 0;
  return make_plan(B, H, Sq, Sk, D, causal, window_left, window_right, dtype).ws_bytes;
}

namespace {
// Optional extras of the dense forward entries.
struct FwdExtras {
  float* lse = nullptr;
  const void* rope_cos = nullptr;
  const void* rope_sin = nullptr;
  int rope_offset = 0, rope_cdt = 0;
  bool drop = false;  // dropout on the weights (the fields below)
  uint32_t drop_thresh = 0, seed0 = 0, seed1 = 0;
  float drop_scale = 1.f;
};
}  // namespace

static int attn_fwd_entry(const void* q, const void* k, const void* v, void* o,
                          const int64_t* q_strides, const int64_t* k_strides,
                          const int64_t* v_strides, const int64_t* o_strides, int B, int H,
                          int H_kv, int Sq, int Sk, int D, float scale, int causal,
                          int window_left, int window_right, int dtype, void* workspace,
                          size_t workspace_bytes, void* stream, const FwdExtras& ex) {
  MPX_CHECK_ARG(dtype == MPX_F32 || dtype == MPX_F16 || dtype == MPX_BF16,
                "mpx_attn_fwd: unknown dtype code %d", dtype);
  MPX_CHECK_ARG(B >= 0 && H >= 0 && Sq >= 0 && Sk >= 0, "mpx_attn_fwd: negative size");
  MPX_CHECK_ARG(H_kv > 0 ? H % H_kv == 0 : H == 0,
                "mpx_attn_fwd: %d query heads are not a multiple of %d K/V heads", H, H_kv);
  if (D != 32 && D != 64 && D != 128 && D != 256) {
    set_error("mpx_attn_fwd: head_dim %d not supported (kernels exist for 32, 64, 128, 256)", D);
    return MPX_EUNSUPPORTED;
  }
  MPX_CHECK_ARG(std::isfinite(scale), "mpx_attn_fwd: scale must be finite");
  if ((long)B * H * Sq == 0) return MPX_OK;
  MPX_CHECK_ARG(q && k && v && o && q_strides && k_strides && v_strides && o_strides,
                "mpx_attn_fwd: null pointer argument");
  MPX_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o),
                "mpx_attn_fwd: tensors must be 16-byte aligned");
  const int vec = dtype == MPX_F32 ? 4 : 8;
  const int64_t* all[4] = {q_strides, k_strides, v_strides, o_strides};
  for (int t = 0; t < 4; ++t)
    for (int i = 0; i < 3; ++i)
      MPX_CHECK_ARG(all[t][i] >= 0 && all[t][i] % vec == 0,
                    "mpx_attn_fwd: strides must be non-negative multiples of %d elements", vec);

  const Plan pl = make_plan(B, H, Sq, Sk, D, causal, window_left, window_right, dtype);
  if (pl.splits > 1) {
    MPX_CHECK_ARG(workspace != nullptr && workspace_bytes >= pl.ws_bytes,
                  "mpx_attn_fwd: workspace of %zu bytes required, %zu given", pl.ws_bytes,
                  workspace_bytes);
    MPX_CHECK_ARG(aligned16(workspace), "mpx_attn_fwd: workspace must be 16-byte aligned");
  }
  if (dtype != MPX_F32) {
    // The 16-bit kernel addresses one (batch, head) of K/V with 32-bit byte offsets.
    const int64_t span_k = ((int64_t)Sk + 64) * k_strides[2] * 2 + (int64_t)D * 2;
    const int64_t span_v = ((int64_t)Sk + 64) * v_strides[2] * 2 + (int64_t)D * 2;
    if (span_k >= (1LL << 31) || span_v >= (1LL << 31)) {
      set_error("mpx_attn_fwd: Sk * seq_stride exceeds the 2 GiB addressing range of one head");
      return MPX_EUNSUPPORTED;
    }
  }

  FwdParams p = {};
  p.q = q; p.k = k; p.v = v; p.o = o;
  p.q_sb = q_strides[0]; p.q_sh = q_strides[1]; p.q_ss = q_strides[2];
  p.k_sb = k_strides[0]; p.k_sh = k_strides[1]; p.k_ss = k_strides[2];
  p.v_sb = v_strides[0]; p.v_sh = v_strides[1]; p.v_ss = v_strides[2];
  p.o_sb = o_strides[0]; p.o_sh = o_strides[1]; p.o_ss = o_strides[2];
  p.B = B; p.H = H; p.Sq = Sq; p.Sk = Sk;
  p.kv_group = H / H_kv;
  p.c = std::fabs(scale) * kLog2e;
  p.neg = scale < 0.f ? 1 : 0;
  p.eps = kSoftmaxEps;
  p.nan_empty = 0;
  p.lse = ex.lse;
  p.rope_cos = ex.rope_cos;
  p.rope_sin = ex.rope_sin;
  p.rope_offset = ex.rope_offset;
  p.rope_cdt = ex.rope_cdt;
  p.drop_thresh = ex.drop_thresh;
  p.seed0 = ex.seed0;
  p.seed1 = ex.seed1;
  p.drop_scale = ex.drop_scale;
  return run_fwd<false>(p, pl, D, dtype, workspace, (hipStream_t)stream, ex.drop);
}

extern "C" int mpx_attn_fwd_lse(const void* q, const void* k, const void* v, void* o,
                                float* lse, const int64_t* q_strides, const int64_t* k_strides,
                                const int64_t* v_strides, const int64_t* o_strides, int B, int H,
                                int H_kv, int Sq, int Sk, int D, float scale, int causal,
                                int window_left, int window_right, int dtype, void* workspace,
                                size_t workspace_bytes, void* stream) {
  clear_error();
  FwdExtras ex;
  ex.lse = lse;
  return attn_fwd_entry(q, k, v, o, q_strides, k_strides, v_strides, o_strides, B, H, H_kv, Sq,
                        Sk, D, scale, causal, window_left, window_right, dtype, workspace,
                        workspace_bytes, stream, ex);
}

extern "C" int mpx_attn_fwd_dropout(const void* q, const void* k, const void* v, void* o,
                                    float* lse, const int64_t* q_strides,
                                    const int64_t* k_strides, const int64_t* v_strides,
                                    const int64_t* o_strides, int B, int H, int H_kv, int Sq,
                                    int Sk, int D, float scale, int causal, int window_left,
                                    int window_right, int dtype, float dropout_p, uint64_t seed,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  MPX_CHECK_ARG(dropout_p >= 0.f && dropout_p < 1.f,
                "mpx_attn_fwd_dropout: dropout_p must be in [0, 1), got %g", (double)dropout_p);
  FwdExtras ex;
  ex.lse = lse;
  if (dropout_p > 0.f) {
    if (D != 64 && D != 128 && D != 256) {
      set_error("mpx_attn_fwd_dropout: head_dim %d not supported (dropout kernels exist for 64, "
                "128, 256)", D);
      return MPX_EUNSUPPORTED;
    }
    ex.drop = true;
    ex.drop_thresh = drop_threshold(dropout_p);
    ex.seed0 = (uint32_t)seed;
    ex.seed1 = (uint32_t)(seed >> 32);
    ex.drop_scale = 1.f / (1.f - dropout_p);
  }
  return attn_fwd_entry(q, k, v, o, q_strides, k_strides, v_strides, o_strides, B, H, H_kv, Sq,
                        Sk, D, scale, causal, window_left, window_right, dtype, workspace,
                        workspace_bytes, stream, ex);
}

extern "C" int mpx_attn_fwd_rope(const void* q, const void* k, const void* v, void* o,
                                 const int64_t* q_strides, const int64_t* k_strides,
                                 const int64_t* v_strides, const int64_t* o_strides, int B,
                                 int H, int H_kv, int Sq, int Sk, int D, float scale, int causal,
                                 int window_left, int window_right, int dtype,
                                 const void* cos_cache, const void* sin_cache, int q_offset,
                                 int n_pos, int cache_dtype, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  clear_error();
  if (dtype == MPX_F32) {
    set_error("mpx_attn_fwd_rope: Q is rotated on load by the 16-bit kernels only");
    return MPX_EUNSUPPORTED;
  }
  if (D > 128) {
    set_error("mpx_attn_fwd_rope: head_dim %d not supported (32, 64, 128)", D);
    return MPX_EUNSUPPORTED;
  }
  MPX_CHECK_ARG(cache_dtype == MPX_F32 || cache_dtype == MPX_F16 || cache_dtype == MPX_BF16,
                "mpx_attn_fwd_rope: unknown cache dtype code %d", cache_dtype);
  MPX_CHECK_ARG(q_offset >= 0 && (Sq == 0 || (long)q_offset + Sq <= n_pos),
                "mpx_attn_fwd_rope: positions %d..%d exceed the %d-row cos/sin caches",
                q_offset, q_offset + Sq - 1, n_pos);
  MPX_CHECK_ARG((long)B * H * Sq == 0 || (cos_cache && sin_cache),
                "mpx_attn_fwd_rope: null cos/sin cache");
  MPX_CHECK_ARG(aligned16(cos_cache) && aligned16(sin_cache),
                "mpx_attn_fwd_rope: cos/sin caches must be 16-byte aligned");
  FwdExtras ex;
  ex.rope_cos = cos_cache;
  ex.rope_sin = sin_cache;
  ex.rope_offset = q_offset;
  ex.rope_cdt = cache_dtype;
  return attn_fwd_entry(q, k, v, o, q_strides, k_strides, v_strides, o_strides, B, H, H_kv, Sq,
                        Sk, D, scale, causal, window_left, window_right, dtype, workspace,
                        workspace_bytes, stream, ex);
}

extern "C" int mpx_attn_fwd_gqa(const void* q, const void* k, const void* v, void* o,
                                const int64_t* q_strides, const int64_t* k_strides,
                                const int64_t* v_strides, const int64_t* o_strides, int B, int H,
                                int H_kv, int Sq, int Sk, int D, float scale, int causal,
                                int window_left, int window_right, int dtype, void* workspace,
                                size_t workspace_bytes, void* stream) {
  clear_error();
  return attn_fwd_entry(q, k, v, o, q_strides, k_strides, v_strides, o_strides, B, H, H_kv, Sq,
                        Sk, D, scale, causal, window_left, window_right, dtype, workspace,
                        workspace_bytes, stream, FwdExtras());
}

extern "C" int mpx_attn_fwd(const void* q, const void* k, const void* v, void* o,
                            const int64_t* q_strides, const int64_t* k_strides,
                            const int64_t* v_strides, const int64_t* o_strides, int B, int H,
                            int Sq, int Sk, int D, float scale, int causal, int window_left,
                            int window_right, int dtype, void* workspace, size_t workspace_bytes,
                            void* stream) {
  return mpx_attn_fwd_gqa(q, k, v, o, q_strides, k_strides, v_strides, o_strides, B, H,
                          H > 0 ? H : 1, Sq, Sk, D, scale, causal, window_left, window_right,
                          dtype, workspace, workspace_bytes, stream);
}

extern "C" size_t mpx_paged_prefill_workspace_bytes(int B, int Sq, int H, int D, int block_size,
                                                    int max_blocks, int causal, int dtype) {
  if (B <= 0 || H <= 0 || Sq <= 0 || D <= 0 || block_size <= 0 || max_blocks <= 0) return 0;
  // The size covers both tile widths (the width also depends on whether an
  // ALiBi bias is given, which this query does not name).
  size_t bytes = 0;
  for (int alibi = 0; alibi < 2; ++alibi) {
    const int bl = log2_if_pow2(block_size);
    const int BN = tile_n(D, dtype, true, bl, alibi);
    bytes = std::max(bytes, make_plan(B, H, Sq, max_blocks * block_size, D, causal, -1, -1,
                                      dtype, paged_tile_cap(block_size, BN), true, bl, alibi)
                                .ws_bytes);
  }
  return bytes;
}

extern "C" int mpx_paged_prefill_gqa(const void* q, const void* k_pool, const void* v_pool,
                                     const int32_t* block_tables, const int32_t* context_lens,
                                     const float* alibi_slopes, void* o,
                                     const int64_t* q_strides, const int64_t* o_strides, int B,
                                     int Sq, int H, int H_kv, int D, int num_blocks,
                                     int block_size, int max_blocks, float scale, int causal,
                                     int dtype, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  clear_error();
  MPX_CHECK_ARG(dtype == MPX_F32 || dtype == MPX_F16 || dtype == MPX_BF16,
                "mpx_paged_prefill: unknown dtype code %d", dtype);
  MPX_CHECK_ARG(B >= 0 && Sq >= 0 && H >= 0 && num_blocks >= 0 && max_blocks >= 0,
                "mpx_paged_prefill: negative size");
  MPX_CHECK_ARG(block_size > 0, "mpx_paged_prefill: block_size must be positive");
  MPX_CHECK_ARG(H_kv > 0 ? H % H_kv == 0 : H == 0,
                "mpx_paged_prefill: %d query heads are not a multiple of %d K/V heads", H, H_kv);
  if (D != 32 && D != 64 && D != 128 && D != 256) {
    set_error("mpx_paged_prefill: head_dim %d not supported (kernels exist for 32, 64, 128, "
              "256)", D);
    return MPX_EUNSUPPORTED;
  }
  MPX_CHECK_ARG(std::isfinite(scale), "mpx_paged_prefill: scale must be finite");
  if ((long)B * H * Sq == 0) return MPX_OK;
  MPX_CHECK_ARG(q && o && context_lens && q_strides && o_strides,
                "mpx_paged_prefill: null pointer argument");
  MPX_CHECK_ARG(max_blocks == 0 || num_blocks == 0 || (k_pool && v_pool && block_tables),
                "mpx_paged_prefill: null pool/table pointer");
  MPX_CHECK_ARG(aligned16(q) && aligned16(o) && aligned16(k_pool) && aligned16(v_pool),
                "mpx_paged_prefill: tensors must be 16-byte aligned");
  const int vec = dtype == MPX_F32 ? 4 : 8;
  for (int i = 0; i < 3; ++i)
    MPX_CHECK_ARG(q_strides[i] >= 0 && q_strides[i] % vec == 0 && o_strides[i] >= 0 &&
                      o_strides[i] % vec == 0,
                  "mpx_paged_prefill: strides must be non-negative multiples of %d elements", vec);
  const long max_tokens = (long)max_blocks * block_size;
  MPX_CHECK_ARG(max_tokens < (1L << 30), "mpx_paged_prefill: block table too large");
  const int es = dtype == MPX_F32 ? 4 : 2;
  const uint64_t pool_bytes = (uint64_t)num_blocks * block_size * H_kv * D * es;
  hipStream_t st = (hipStream_t)stream;
  if (num_blocks == 0 || max_blocks == 0) {
    // No key exists for any query: every output row is NaN.
    const long n = (long)B * H * Sq * D;
    const int blocks = (int)std::min<long>((n + 255) / 256, 4096);
    if (dtype == MPX_F32)
      hipLaunchKernelGGL(fill_nan_kernel<MPX_F32>, dim3(blocks), dim3(256), 0, st, o,
                         o_strides[0], o_strides[1], o_strides[2], B, H, Sq, D);
    else if (dtype == MPX_BF16)
      hipLaunchKernelGGL(fill_nan_kernel<MPX_BF16>, dim3(blocks), dim3(256), 0, st, o,
                         o_strides[0], o_strides[1], o_strides[2], B, H, Sq, D);
    else
      hipLaunchKernelGGL(fill_nan_kernel<MPX_F16>, dim3(blocks), dim3(256), 0, st, o,
                         o_strides[0], o_strides[1], o_strides[2], B, H, Sq, D);
    MPX_CHECK_HIP(hipGetLastError());
    return MPX_OK;
  }
  const int BN = tile_n(D, dtype, true, log2_if_pow2(block_size), alibi_slopes != nullptr);
  const Plan pl = make_plan(B, H, Sq, (int)max_tokens, D, causal, -1, -1, dtype,
                            paged_tile_cap(block_size, BN), true, log2_if_pow2(block_size),
                            alibi_slopes != nullptr);
  if (pl.splits > 1) {
    MPX_CHECK_ARG(workspace != nullptr && workspace_bytes >= pl.ws_bytes,
                  "mpx_paged_prefill: workspace of %zu bytes required, %zu given", pl.ws_bytes,
                  workspace_bytes);
    MPX_CHECK_ARG(aligned16(workspace), "mpx_paged_prefill: workspace must be 16-byte aligned");
  }

  FwdParams p = {};
  p.q = q; p.k = k_pool; p.v = v_pool; p.o = o;
  p.q_sb = q_strides[0]; p.q_sh = q_strides[1]; p.q_ss = q_strides[2];
  p.k_sb = 0; p.k_sh = D; p.k_ss = (int64_t)H_kv * D;
  p.v_sb = 0; p.v_sh = D; p.v_ss = (int64_t)H_kv * D;
  p.o_sb = o_strides[0]; p.o_sh = o_strides[1]; p.o_ss = o_strides[2];
  p.B = B; p.H = H; p.Sq = Sq; p.Sk = (int)max_tokens;
  p.kv_group = H / H_kv;
  p.c = std::fabs(scale) * kLog2e;
  p.neg = scale < 0.f ? 1 : 0;
  p.eps = 0.f;
  p.nan_empty = 1;
  p.bt = block_tables; p.ctx = context_lens; p.slopes = alibi_slopes;
  p.bs = block_size;
  p.bs_log2 = log2_if_pow2(block_size);
  p.max_blocks = max_blocks; p.num_blocks = num_blocks;
  // 0: a pool of 4 GiB - 256 bytes or more, read through 64-bit addresses (the
  // 32-bit buffer offsets of the other kernels reach below that; fp32 kernels
  // always address pools in 64 bits).
  p.pool_bytes = pool_bytes < 0xFFFFFF00ull ? (uint32_t)pool_bytes : 0u;
  return run_fwd<true>(p, pl, D, dtype, workspace, st);
}

extern "C" int mpx_paged_prefill(const void* q, const void* k_pool, const void* v_pool,
                                 const int32_t* block_tables, const int32_t* context_lens,
                                 const float* alibi_slopes, void* o, const int64_t* q_strides,
                                 const int64_t* o_strides, int B, int Sq, int H, int D,
                                 int num_blocks, int block_size, int max_blocks, float scale,
                                 int causal, int dtype, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  return mpx_paged_prefill_gqa(q, k_pool, v_pool, block_tables, context_lens, alibi_slopes, o,
                               q_strides, o_strides, B, Sq, H, H > 0 ? H : 1, D, num_blocks,
                               block_size, max_blocks, scale, causal, dtype, workspace,
                               workspace_bytes, stream);
}
