// Dropout forward launches for gfx950: fa_fwd16_drop_kernel and the DROP forms
// of the head-dim-256 and float32 kernels (fa_fwd_kernels.h). They sit in a
// translation unit of their own so that they keep the compiler's default
// machine scheduler while fa_fwd.hip is built for maximum ILP.
#include "fa_fwd_kernels.h"

namespace mpx {

// The dropout kernels (dense K/V, D = 64, 128 or 256).
hipError_t dispatch_fwd_drop(const FwdParams& p, int D, int dtype, int grid, hipStream_t st) {
#define MPX_DROP16(DD, BF)                                                                  \
  hipLaunchKernelGGL((fa_fwd16_drop_kernel<DD, kBN16<false, DD>, kNumWaves16, BF>), dim3(grid), \
                     dim3(64 * kNumWaves16), 0, st, p)
  if (D == 256) {
    if (dtype == MPX_F32)
      hipLaunchKernelGGL((fa_fwd32_kernel<256, 32, kNumWaves32, false, true>), dim3(grid),
                         dim3(64 * kNumWaves32), 0, st, p);
    else if (dtype == MPX_BF16)
      hipLaunchKernelGGL((fa_fwd16_wide_kernel<256, 64, kNumWavesWide, true, false, true>),
                         dim3(grid), dim3(64 * kNumWavesWide), 0, st, p);
    else
      hipLaunchKernelGGL((fa_fwd16_wide_kernel<256, 64, kNumWavesWide, false, false, true>),
                         dim3(grid), dim3(64 * kNumWavesWide), 0, st, p);
    return hipGetLastError();
  }
  if (dtype == MPX_F32) {
    if (D == 64)
      hipLaunchKernelGGL((fa_fwd32_kernel<64, 64, kNumWaves32, false, true>), dim3(grid),
                         dim3(64 * kNumWaves32), 0, st, p);
    else
      hipLaunchKernelGGL((fa_fwd32_kernel<128, 32, kNumWaves32, false, true>), dim3(grid),
                         dim3(64 * kNumWaves32), 0, st, p);
  } else if (dtype == MPX_BF16) {
    if (D == 64) MPX_DROP16(64, true); else MPX_DROP16(128, true);
  } else {
    if (D == 64) MPX_DROP16(64, false); else MPX_DROP16(128, false);
  }
#undef MPX_DROP16
  return hipGetLastError();
}

}  // namespace mpx
