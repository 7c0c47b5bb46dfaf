// Launchers of the tile kernels: the C ABI (capi.hip) validates a call and
// picks its tiles, these pick the instantiation and launch it.  Defined in
// kernels.hip, which is compiled once per head dim and direction (the objects
// build in parallel).
#pragma once
#include <hip/hip_runtime.h>

#include "../../include/flexattn.h"
#include "bwd.h"
#include "fwd.h"
#include "fwd_fp8.h"
#include "problem.h"

namespace fa {

inline int launch_status() { return hipGetLastError() == hipSuccess ? FA_OK : FA_ERR_LAUNCH; }

// Element type T (uint16_t: bf16, float), head dim D, with (M) or without
// the built-in score mods (ALiBi, soft-cap); tiles as chosen by the C ABI.
// A tile with no instantiation returns FA_ERR_UNSUPPORTED.
template <typename T, int D, bool M>
int launch_fwd(const FwdArgs& a, const Tiles& t, hipStream_t s);  // forward (+ split-KV merge)
template <typename T, int D, bool M>
int launch_dq(const BwdArgs& a, const Tiles& t, hipStream_t s);
template <typename T, int D, bool M>
int launch_dkdv(const BwdArgs& a, const Tiles& t, hipStream_t s);
template <typename T, int D>
int launch_delta(const BwdArgs& a, hipStream_t s);  // Delta = rowsum(dO * O)

// fp8 forward (D = 64 or 128, 128 x 64 tiles) and the bf16 -> e4m3 block
// quantiser (kernels_fp8.hip)
int launch_fwd_fp8(const Fp8FwdArgs& a, int D, bool mods, hipStream_t s);
int launch_quant_fp8(const QuantArgs& a, hipStream_t s);

}  // namespace fa
