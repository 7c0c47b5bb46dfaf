// Instantiations and launches of the fp8 forward and the e4m3 quantiser.
#include "fwd_fp8.h"
#include "launch.h"

namespace fa {

int launch_fwd_fp8(const Fp8FwdArgs& a, int D, bool mods, hipStream_t s) {
  constexpr int NW = 4;
  const dim3 grid((unsigned)fwd_items(a.p, 0, 32 * NW)), block(64 * NW);
  if (D == 128) {
    if (mods) hipLaunchKernelGGL((fwd_fp8_kernel<128, NW, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((fwd_fp8_kernel<128, NW, false>), grid, block, 0, s, a);
  } else if (D == 64) {
    if (mods) hipLaunchKernelGGL((fwd_fp8_kernel<64, NW, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((fwd_fp8_kernel<64, NW, false>), grid, block, 0, s, a);
  } else {
    return FA_ERR_UNSUPPORTED;
  }
  return launch_status();
}

int launch_quant_fp8(const QuantArgs& a, hipStream_t s) {
  const unsigned grid = (unsigned)(a.heads * cdiv(a.S, kFp8ScaleRows));
  switch (a.D) {
    case 32: hipLaunchKernelGGL((quant_fp8_kernel<32>), dim3(grid), dim3(256), 0, s, a); break;
    case 64: hipLaunchKernelGGL((quant_fp8_kernel<64>), dim3(grid), dim3(256), 0, s, a); break;
    case 128: hipLaunchKernelGGL((quant_fp8_kernel<128>), dim3(grid), dim3(256), 0, s, a); break;
    default: return FA_ERR_UNSUPPORTED;
  }
  return launch_status();
}

}  // namespace fa
