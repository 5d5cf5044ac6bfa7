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
  // Stored dS^T (the stored-dS schedule only): ds_tot blocks per query head.
  void* ds;
  int64_t ds_tot;
};

constexpr int kBwdWaves = 4;    // waves per workgroup (one per SIMD)
constexpr int kBwdOwn = 32 * kBwdWaves;  // rows (or keys) a workgroup owns
constexpr int kBwdTile = 64;    // streamed rows per step

// Stored dS^T: per query head, 2 KB blocks of 32 keys x 32 queries (16-bit).
// Key tile kt (kBwdOwn keys, four key blocks) owns the blocks of the 32-row
// query blocks t0 .. t0 + nt - 1 that its keys' masks reach, query block
// major, key block minor; its first block is 4 * (sum of nt over the key
// tiles before it). Blocks that a key block and a query block do not share
// (outside both window edges, keys past Sk) are never written or read.
constexpr int kDsBlockBytes = 2048;

__host__ __device__ inline void ds_key_tile(int Sq, int Sk, int win_left, int win_right, int kt,
                                            int& t0, int& nt) {
  const int k0 = kt * kBwdOwn;
  const int k_last = (k0 + kBwdOwn < Sk ? k0 + kBwdOwn : Sk) - 1;
  const int q_lo = win_right >= 0 ? (k0 - win_right > 0 ? k0 - win_right : 0) : 0;
  const int q_hi = win_left >= 0 ? (k_last + win_left + 1 < Sq ? k_last + win_left + 1 : Sq) : Sq;
  t0 = q_lo / 32;
  nt = q_hi > q_lo ? (q_hi - 1) / 32 - t0 + 1 : 0;
}

// The float32 backward (rowsum, dQ, dK/dV kernels) for D in {64, 128}, with
// the forward's dropout when drop is set, enqueued on st; defined in
// fa_bwd32.hip.
hipError_t launch_bwd32(const BwdParams& p, int D, bool drop, hipStream_t st);

}  // namespace mpx
