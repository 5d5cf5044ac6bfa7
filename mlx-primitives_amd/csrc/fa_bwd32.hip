// Attention backward in float32 for gfx950: v_mfma_f32_32x32x2f32 (true fp32
// products), head_dim 64 or 128. Same gradients and decomposition as the
// 16-bit kernels (fa_bwd.hip): Dvec = rowsum(dO * O); a query-parallel dQ
// kernel and a key-parallel dK/dV kernel that recompute S and dP from the
// forward's row log-sum-exp. The reference differentiates its float32 tiled
// path with mx.grad (mlx_primitives/attention/flash.py:257-316;
// tests/attention/test_flash.py:338-362, tests/parity/pytorch/
// test_attention_parity.py:107-163 run float32).
//
// 32x32x2 f32 layouts (lane = j + 32 g): A lane holds element (row j, k = g),
// B (k = g, column j), C element e of the lane holds row 8 (e/4) + 4 g + e%4,
// column j. Products over head dims take their two k values from one 16-byte
// read (dims 8 jj + 4 g + t4, t4 < 4). Products over a C block's rows (dQ^T +=
// K^T dS^T, dV^T += dO^T P, dK^T += Q^T dS) step through the 16 C elements:
// element e is the B operand of its step directly (k = g <-> row 8 (e/4) + 4 g
// + e%4), and the A operand is one scalar LDS read of that row. Tiles of 32
// rows are staged through registers into LDS rows padded to D + 4 floats
// (16-byte row reads conflict-free).
#include "fa_bwd.h"

#include <algorithm>
#include <cmath>

namespace mpx {

constexpr int kB32Tile = 32;  // streamed rows per step

template <int D>
__global__ __launch_bounds__(256) void fa_bwd32_dvec_kernel(BwdParams p) {
  constexpr int LPR = D / 4;  // lanes per row, 4 floats each
  const int64_t rows = (int64_t)p.B * p.H * p.Sq;
  const int64_t row = ((int64_t)blockIdx.x * 256 + threadIdx.x) / LPR;
  const int l = threadIdx.x % LPR;
  float acc = 0.f;
  if (row < rows) {
    const int i = (int)(row % p.Sq);
    const int64_t bh = row / p.Sq;
    const int b = (int)(bh / p.H), h = (int)(bh % p.H);
    const float* o = (const float*)p.o + b * p.o_sb + h * p.o_sh + (int64_t)i * p.o_ss;
    const float* d = (const float*)p.dout + b * p.do_sb + h * p.do_sh + (int64_t)i * p.do_ss;
    const f32x4 ov = *(const f32x4*)(o + 4 * l);
    const f32x4 dv = *(const f32x4*)(d + 4 * l);
    acc = ov[0] * dv[0] + ov[1] * dv[1] + ov[2] * dv[2] + ov[3] * dv[3];
  }
#pragma unroll
  for (int off = LPR / 2; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (row < rows && l == 0) p.dvec[row] = acc;
}

// 32 rows of a float32 (rows, D) slice through 256 threads: global ->
// registers (rows past `rows` re-read the last one) -> LDS rows of stride D + 4.
template <int D>
struct Stage32 {
  static constexpr int CPR = D / 4, PER_T = kB32Tile * CPR / 256, RS = D + 4;
  f32x4 r[PER_T];
  __device__ __forceinline__ void load(const float* base, int64_t row_stride, int row0,
                                       int rows) {
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int c = threadIdx.x + 256 * i;
      const int row = min(row0 + c / CPR, rows - 1);
      r[i] = *(const f32x4*)(base + (int64_t)row * row_stride + (c % CPR) * 4);
    }
  }
  __device__ __forceinline__ void store(float* lds) const {
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int c = threadIdx.x + 256 * i;
      *(f32x4*)(lds + (c / CPR) * RS + (c % CPR) * 4) = r[i];
    }
  }
};

// Row of a float32 tensor as B-operand fragments: f[jj] = dims 8 jj + 4 g .. +3.
template <int D>
__device__ __forceinline__ void load_row32(const float* row, int g, f32x4 (&f)[D / 8]) {
#pragma unroll
  for (int jj = 0; jj < D / 8; ++jj) f[jj] = *(const f32x4*)(row + 8 * jj + 4 * g);
}

// Accumulator set (lane = output row, C rows = dims) times mul, stored as one
// float32 row.
template <int NDB>
__device__ __forceinline__ void store_row32(float* row, int g, const f32x16 (&acc)[NDB],
                                            float mul) {
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4)
      *(f32x4*)(row + db * 32 + 8 * e4 + 4 * g) =
          (f32x4){acc[db][4 * e4] * mul, acc[db][4 * e4 + 1] * mul, acc[db][4 * e4 + 2] * mul,
                  acc[db][4 * e4 + 3] * mul};
}

// Row (within a 32-row tile) that C element e of a lane in half g stands for.
__device__ __forceinline__ constexpr int crow(int e, int g) {
  return 8 * (e >> 2) + 4 * g + (e & 3);
}

// ---------------------------------------------------------------------------
// dQ: a workgroup owns 128 query rows of one (batch, head), wave w rows +32w;
// per 32-key tile: S^T = K Q^T, dP^T = V dO^T, dS^T = P^T (dP^T - Dvec),
// dQ^T += K^T dS^T.
// ---------------------------------------------------------------------------
template <int D, bool DROP = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void fa_bwd32_dq_kernel(BwdParams p) {
  constexpr int NQ4 = D / 8, NDB = D / 32, RS = D + 4, TILE = kB32Tile * RS;
  // D = 256: one LDS stage (two would be 133 KB); the next tile is loaded
  // after the barrier that ends the current one.
  constexpr int NSTG = D > 128 ? 1 : 2;
  __shared__ __align__(16) float lds[NSTG][2][TILE];  // [stage][K, V]

  const int n_qt = (p.Sq + kBwdOwn - 1) / kBwdOwn;
  const int qt = n_qt - 1 - (int)(blockIdx.x / (p.B * p.H));
  const int bh = blockIdx.x % (p.B * p.H);
  const int b = bh / p.H, h = bh % p.H;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 31, g = lane >> 5;
  const int q0 = qt * kBwdOwn, wq0 = q0 + wave * 32, myq = wq0 + j;
  const int qrow = min(myq, p.Sq - 1);

  const int kvh = h / p.kv_group;
  const float* Q = (const float*)p.q + b * p.q_sb + h * p.q_sh;
  const float* K = (const float*)p.k + b * p.k_sb + kvh * p.k_sh;
  const float* V = (const float*)p.v + b * p.v_sb + kvh * p.v_sh;
  const float* dO = (const float*)p.dout + b * p.do_sb + h * p.do_sh;
  f32x4 qf[NQ4], df[NQ4];
  load_row32<D>(Q + (int64_t)qrow * p.q_ss, g, qf);
  load_row32<D>(dO + (int64_t)qrow * p.do_ss, g, df);
  const int64_t rix = (int64_t)bh * p.Sq + qrow;
  const float lse = myq < p.Sq ? p.lse[rix] : INFINITY;
  const float dvc = p.dvec[rix];
  // Dropout: this row's key of the forward's keep-mask hash.
  const u32 drop_rk = DROP ? drop_row_key((u32)((int64_t)bh * p.Sq + myq), p.seed0) : 0u;
  const int kv_first = p.win_left >= 0 ? myq - p.win_left : -(1 << 30);
  const int kv_last = min(p.win_right >= 0 ? myq + p.win_right : (1 << 30), p.Sk - 1);

  const int q_last = min(q0 + kBwdOwn, p.Sq) - 1;
  const int kv_lo = p.win_left >= 0 ? max(0, q0 - p.win_left) : 0;
  const int kv_hi = p.win_right >= 0 ? min(p.Sk, q_last + p.win_right + 1) : p.Sk;
  const int t0 = kv_lo / kB32Tile;
  const int n_t = kv_hi > kv_lo ? (kv_hi - 1) / kB32Tile - t0 + 1 : 0;

  f32x16 dq[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) dq[db] = (f32x16){};

  Stage32<D> kst, vst;
  if (n_t > 0) {
    kst.load(K, p.k_ss, t0 * kB32Tile, p.Sk);
    vst.load(V, p.v_ss, t0 * kB32Tile, p.Sk);
    kst.store(lds[0][0]);
    vst.store(lds[0][1]);
  }
  __syncthreads();
  for (int t = 0; t < n_t; ++t) {
    const int S = NSTG == 1 ? 0 : t & 1;
    const int kv0 = (t0 + t) * kB32Tile;
    if (NSTG == 2 && t + 1 < n_t) {
      kst.load(K, p.k_ss, kv0 + kB32Tile, p.Sk);
      vst.load(V, p.v_ss, kv0 + kB32Tile, p.Sk);
    }
    const bool skip = wq0 >= p.Sq ||
                      (p.win_right >= 0 && kv0 > wq0 + 31 + p.win_right) ||
                      (p.win_left >= 0 && kv0 + kB32Tile - 1 < wq0 - p.win_left);
    const bool full = kv0 + kB32Tile <= p.Sk &&
                      (p.win_right < 0 || kv0 + kB32Tile - 1 <= wq0 + p.win_right) &&
                      (p.win_left < 0 || kv0 >= wq0 + 31 - p.win_left);
    if (!skip) {
      const float* Kt = lds[S][0];
      const float* Vt = lds[S][1];
      f32x16 sb = {}, dpb = {};
      const f32x4* kp = (const f32x4*)(Kt + j * RS) + g;
      const f32x4* vp = (const f32x4*)(Vt + j * RS) + g;
#pragma unroll
      for (int jj = 0; jj < NQ4; ++jj) {
        const f32x4 ka = kp[2 * jj], va = vp[2 * jj];
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) {
          sb = mfma32x32x2f32(ka[t4], qf[jj][t4], sb);
          dpb = mfma32x32x2f32(va[t4], df[jj][t4], dpb);
        }
      }
      if (!full) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = kv0 + crow(e, g);
          sb[e] = (key >= kv_first) & (key <= kv_last) ? sb[e] : -INFINITY;
        }
      }
      if constexpr (DROP) {
        // dS = P (dP keep / (1 - p) - Dvec); elements 2 e2, 2 e2 + 1 hold keys
        // kv0 + crow(2 e2, g) + {0, 1}, the hash's key pair
        // kv0 / 2 + 4 (e2 / 2) + 2 g + e2 % 2.
        const u32 pair0 = drop_pair_key((u32)(kv0 >> 1) + 2u * g, p.seed1);
#pragma unroll
        for (int e2 = 0; e2 < 8; ++e2) {
          const u32 bits = drop_bits(drop_rk, pair0 + (u32)(4 * (e2 >> 1) + (e2 & 1)) * 0x85EBCA77u);
          dpb[2 * e2] = (bits & 0xffffu) >= p.drop_thresh ? dpb[2 * e2] * p.drop_scale : 0.f;
          dpb[2 * e2 + 1] = bits >= (p.drop_thresh << 16) ? dpb[2 * e2 + 1] * p.drop_scale : 0.f;
        }
      }
      f32x16 ds;
#pragma unroll
      for (int e = 0; e < 16; ++e) ds[e] = fast_exp2(sb[e] * p.c - lse) * (dpb[e] - dvc);
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          dq[db] = mfma32x32x2f32(Kt[crow(e, g) * RS + db * 32 + j], ds[e], dq[db]);
    }
    if (t + 1 < n_t) {
      if constexpr (NSTG == 1) {
        __syncthreads();
        kst.load(K, p.k_ss, kv0 + kB32Tile, p.Sk);
        vst.load(V, p.v_ss, kv0 + kB32Tile, p.Sk);
      }
      kst.store(lds[NSTG == 1 ? 0 : S ^ 1][0]);
      vst.store(lds[NSTG == 1 ? 0 : S ^ 1][1]);
    }
    __syncthreads();
  }
  if (myq < p.Sq)
    store_row32<NDB>((float*)p.dq + b * p.dq_sb + h * p.dq_sh + (int64_t)myq * p.dq_ss, g, dq,
                     p.scale);
}

// ---------------------------------------------------------------------------
// dK, dV: a workgroup owns 128 keys of one (batch, K/V head), wave w keys
// +32w; per 32-row Q tile (every query head of the group): S = Q K^T,
// dP = dO V^T, P = exp2(S c - lse), dS = P (dP - Dvec), dV^T += dO^T P,
// dK^T += Q^T dS. WANT_K / WANT_V select the outputs: at D = 128 K, V and both
// accumulator sets do not fit one wave's registers, so dK and dV run as two
// kernels (the dV one recomputes S and needs neither dP nor V).
// ---------------------------------------------------------------------------
template <int D, bool WANT_K, bool WANT_V, bool DROP = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void fa_bwd32_dkdv_kernel(BwdParams p) {
  constexpr int NQ4 = D / 8, NDB = D / 32, RS = D + 4, TILE = kB32Tile * RS;
  // D = 256: one LDS stage, as in the dQ kernel.
  constexpr int NSTG = D > 128 ? 1 : 2;
  __shared__ __align__(16) float lds[NSTG][2][TILE];  // [stage][Q, dO]
  __shared__ __align__(16) float lse_lds[2][kB32Tile];
  __shared__ __align__(16) float dvc_lds[2][kB32Tile];

  const int kt = (int)(blockIdx.x / (p.B * p.H_kv));
  const int bhk = blockIdx.x % (p.B * p.H_kv);
  const int b = bhk / p.H_kv, hk = bhk % p.H_kv;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 31, g = lane >> 5;
  const int k0 = kt * kBwdOwn, wk0 = k0 + wave * 32, mykey = wk0 + j;
  const int krow = min(mykey, p.Sk - 1);
  const int q_first = p.win_right >= 0 ? mykey - p.win_right : -(1 << 30);
  const int q_last = p.win_left >= 0 ? mykey + p.win_left : (1 << 30);
  // Dropout: this key's pair key of the forward's keep-mask hash and the half
  // of the hash that decides it.
  const u32 drop_pk = DROP ? drop_pair_key((u32)mykey >> 1, p.seed1) : 0u;
  const u32 drop_hm = (mykey & 1) ? 0xffff0000u : 0xffffu;
  const u32 drop_ht = (mykey & 1) ? p.drop_thresh << 16 : p.drop_thresh;

  const float* K = (const float*)p.k + b * p.k_sb + hk * p.k_sh;
  const float* V = (const float*)p.v + b * p.v_sb + hk * p.v_sh;
  f32x4 kf[NQ4], vf[NQ4];
  load_row32<D>(K + (int64_t)krow * p.k_ss, g, kf);
  if constexpr (WANT_K) load_row32<D>(V + (int64_t)krow * p.v_ss, g, vf);

  const int k_last = min(k0 + kBwdOwn, p.Sk) - 1;
  const int q_lo = p.win_right >= 0 ? max(0, k0 - p.win_right) : 0;
  const int q_hi = p.win_left >= 0 ? min(p.Sq, k_last + p.win_left + 1) : p.Sq;
  const int t0 = q_lo / kB32Tile;
  const int n_t = q_hi > q_lo ? (q_hi - 1) / kB32Tile - t0 + 1 : 0;
  const int n_steps = n_t * p.kv_group;

  f32x16 dk[NDB], dv[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    dk[db] = (f32x16){};
    dv[db] = (f32x16){};
  }

  Stage32<D> qst, dst;
  float lse_r = 0.f, dvc_r = 0.f;
  auto load = [&](int u) __attribute__((always_inline)) {
    const int h = hk * p.kv_group + u / n_t;
    const int row0 = (t0 + u % n_t) * kB32Tile;
    qst.load((const float*)p.q + b * p.q_sb + h * p.q_sh, p.q_ss, row0, p.Sq);
    dst.load((const float*)p.dout + b * p.do_sb + h * p.do_sh, p.do_ss, row0, p.Sq);
    if (threadIdx.x < kB32Tile) {
      const int r = row0 + threadIdx.x;
      const int64_t rix = ((int64_t)b * p.H + h) * p.Sq + r;
      lse_r = r < p.Sq ? p.lse[rix] : INFINITY;
      dvc_r = r < p.Sq ? p.dvec[rix] : 0.f;
    }
  };
  auto store = [&](int S) __attribute__((always_inline)) {
    qst.store(lds[S][0]);
    dst.store(lds[S][1]);
    if (threadIdx.x < kB32Tile) {
      lse_lds[S][threadIdx.x] = lse_r;
      dvc_lds[S][threadIdx.x] = dvc_r;
    }
  };
  if (n_steps > 0) {
    load(0);
    store(0);
  }
  __syncthreads();
  for (int u = 0; u < n_steps; ++u) {
    const int S = NSTG == 1 ? 0 : u & 1;
    if (NSTG == 2 && u + 1 < n_steps) load(u + 1);
    const int qr0 = (t0 + u % n_t) * kB32Tile;
    const bool skip = wk0 >= p.Sk ||
                      (p.win_right >= 0 && wk0 > qr0 + kB32Tile - 1 + p.win_right) ||
                      (p.win_left >= 0 && wk0 + 31 < qr0 - p.win_left);
    const bool full = (p.win_right < 0 || wk0 + 31 <= qr0 + p.win_right) &&
                      (p.win_left < 0 || wk0 >= qr0 + kB32Tile - 1 - p.win_left);
    if (!skip) {
      const float* Qt = lds[S][0];
      const float* Dt = lds[S][1];
      f32x16 sb = {}, dpb = {};
      const f32x4* qp = (const f32x4*)(Qt + j * RS) + g;
      const f32x4* dp = (const f32x4*)(Dt + j * RS) + g;
#pragma unroll
      for (int jj = 0; jj < NQ4; ++jj) {
        const f32x4 qa = qp[2 * jj], da = dp[2 * jj];
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) {
          sb = mfma32x32x2f32(qa[t4], kf[jj][t4], sb);
          if constexpr (WANT_K) dpb = mfma32x32x2f32(da[t4], vf[jj][t4], dpb);
        }
      }
      if (!full) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int q = qr0 + crow(e, g);
          sb[e] = (q >= q_first) & (q <= q_last) ? sb[e] : -INFINITY;
        }
      }
      f32x16 pr, ds;
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const f32x4 lv = *(const f32x4*)(&lse_lds[S][8 * e4 + 4 * g]);
        const f32x4 dv4 = *(const f32x4*)(&dvc_lds[S][8 * e4 + 4 * g]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e = 4 * e4 + i;
          pr[e] = fast_exp2(sb[e] * p.c - lv[i]);
          if constexpr (DROP) {
            // Row qr0 + crow(e, g) of this step's head (u / n_t of the group).
            const u32 rk = drop_row_key(
                (u32)(((int64_t)b * p.H + hk * p.kv_group + u / n_t) * p.Sq + qr0 + crow(e, g)),
                p.seed0);
            const bool keep = drop_keep(drop_bits(rk, drop_pk), drop_hm, drop_ht);
            if constexpr (WANT_K) ds[e] = pr[e] * ((keep ? dpb[e] * p.drop_scale : 0.f) - dv4[i]);
            pr[e] = keep ? pr[e] : 0.f;
          } else {
            if constexpr (WANT_K) ds[e] = pr[e] * (dpb[e] - dv4[i]);
          }
        }
      }
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = crow(e, g) * RS + db * 32 + j;
          if constexpr (WANT_V) dv[db] = mfma32x32x2f32(Dt[r], pr[e], dv[db]);
          if constexpr (WANT_K) dk[db] = mfma32x32x2f32(Qt[r], ds[e], dk[db]);
        }
    }
    if (u + 1 < n_steps) {
      if constexpr (NSTG == 1) {
        __syncthreads();
        load(u + 1);
      }
      store(NSTG == 1 ? 0 : S ^ 1);
    }
    __syncthreads();
  }
  if (mykey < p.Sk) {
    if constexpr (WANT_K)
      store_row32<NDB>((float*)p.dk + b * p.dk_sb + hk * p.dk_sh + (int64_t)mykey * p.dk_ss, g,
                       dk, p.scale);
    if constexpr (WANT_V)
      store_row32<NDB>((float*)p.dv + b * p.dv_sb + hk * p.dv_sh + (int64_t)mykey * p.dv_ss, g,
                       dv, DROP ? p.drop_scale : 1.f);
  }
}

template <int D, bool DROP>
hipError_t launch_bwd32_d(const BwdParams& p, hipStream_t st) {
  const int64_t rows = (int64_t)p.B * p.H * p.Sq;
  hipLaunchKernelGGL((fa_bwd32_dvec_kernel<D>), dim3((unsigned)((rows * (D / 4) + 255) / 256)),
                     dim3(256), 0, st, p);
  const int n_qt = (p.Sq + kBwdOwn - 1) / kBwdOwn, n_kt = (p.Sk + kBwdOwn - 1) / kBwdOwn;
  hipLaunchKernelGGL((fa_bwd32_dq_kernel<D, DROP>), dim3(p.B * p.H * n_qt), dim3(256), 0, st, p);
  const dim3 grid_kv(p.B * p.H_kv * n_kt);
  if constexpr (D >= 128) {
    hipLaunchKernelGGL((fa_bwd32_dkdv_kernel<D, true, false, DROP>), grid_kv, dim3(256), 0, st, p);
    hipLaunchKernelGGL((fa_bwd32_dkdv_kernel<D, false, true, DROP>), grid_kv, dim3(256), 0, st, p);
  } else {
    hipLaunchKernelGGL((fa_bwd32_dkdv_kernel<D, true, true, DROP>), grid_kv, dim3(256), 0, st, p);
  }
  return hipGetLastError();
}

template <bool DROP>
hipError_t launch_bwd32_drop(const BwdParams& p, int D, hipStream_t st) {
  if (D == 64) return launch_bwd32_d<64, DROP>(p, st);
  if (D == 256) return launch_bwd32_d<256, DROP>(p, st);
  return launch_bwd32_d<128, DROP>(p, st);
}

hipError_t launch_bwd32(const BwdParams& p, int D, bool drop, hipStream_t st) {
  return drop ? launch_bwd32_drop<true>(p, D, st) : launch_bwd32_drop<false>(p, D, st);
}

}  // namespace mpx
