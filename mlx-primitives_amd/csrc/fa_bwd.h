// Shared declarations of the attention backward kernels (fa_bwd.hip: 16-bit,
// fa_bwd32.hip: float32).
#pragma once

#include "mpx_common.h"

namespace mpx {

struct BwdParams {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  const float* lse;   // (B, H, Sq) log2 units, +inf for rows without keys
  float* dvec;        // (B, H, Sq) workspace
  void* dq;
  void* dk;
  void* dv;
  int64_t q_sb, q_sh, q_ss, k_sb, k_sh, k_ss, v_sb, v_sh, v_ss, o_sb, o_sh, o_ss;
  int64_t do_sb, do_sh, do_ss, dq_sb, dq_sh, dq_ss, dk_sb, dk_sh, dk_ss, dv_sb, dv_sh, dv_ss;
  int B, H, H_kv, kv_group, Sq, Sk;  // K/V (and dK/dV) carry H_kv = H / kv_group heads
  int win_left, win_right;  // -1 = unbounded (causal: win_right = 0)
  float scale, c;           // c = scale * log2(e)
  // Dropout of the forward (the DROP kernels only): keep threshold and seed
  // words of the keep-mask hash, and the 1 / (1 - p) of the kept weights.
  uint32_t drop_thresh, seed0, seed1;
  float drop_scale;
};

constexpr int kBwdWaves = 4;    // waves per workgroup (one per SIMD)
constexpr int kBwdOwn = 32 * kBwdWaves;  // rows (or keys) a workgroup owns
constexpr int kBwdTile = 64;    // streamed rows per step

// The float32 backward (rowsum, dQ, dK/dV kernels) for D in {64, 128}, with
// the forward's dropout when drop is set, enqueued on st; defined in
// fa_bwd32.hip.
hipError_t launch_bwd32(const BwdParams& p, int D, bool drop, hipStream_t st);

}  // namespace mpx
