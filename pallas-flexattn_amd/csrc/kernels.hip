// The kernel instantiations and their launches for one head dim
// (FA_KERNELS_D) and one direction (FA_KERNELS_BWD = 0: forward, 1:
// backward); build.py compiles this file once per pair.
#include "bwd_bf16.h"
#include "fwd_bf16.h"
#include "launch.h"

#if !defined(FA_KERNELS_D) || !defined(FA_KERNELS_BWD)
#error "compile with -DFA_KERNELS_D=32|64|128 -DFA_KERNELS_BWD=0|1"
#endif

namespace fa {

// (BN, NW) of the generic kernels: one key tile per dtype, up to 4 waves
template <typename T, int BN, int NW>
constexpr bool generic_tile() {
  return BN == (sizeof(T) == 2 ? 64 : 32) && NW <= 4;
}

template <typename T, int D, int BN, int NW, bool M, int NS = 2>
int run_fwd(const FwdArgs& a, hipStream_t s) {
  const int grid = fwd_items(a.p, a.pack, 32 * NW);
  if constexpr (sizeof(T) == 2) {
    if (interval_masks(a.p)) {  // bf16: LDS-DMA + transposing-read kernel
      const bool cache = a.pack > 1 || a.page_table || a.kv_lens;
      if constexpr (NW == 4 && BN == 64) {
        // split-KV decode (every packed row in one 32-row block): one wave
        // per workgroup and 32-key tiles, 4x less MFMA work on dead rows and
        // half the LDS per workgroup; measured 5.72 against 5.40 TB/s of KV
        // reads at B8 Hq32 Hkv8 Skv32768 (a plain streaming read reaches
        // ~5.8).  Unsplit, its grid of one-wave workgroups is too small.
        if (cache && a.pack > 1 && a.pack * a.p.Sq <= 32 && a.n_splits > 1 && D >= 64)
          hipLaunchKernelGGL((fa::fwd_bf16_kernel<D, 32, 1, M, fa::BuiltinMod, true>), dim3(grid * a.n_splits),
                             dim3(64), 0, s, a);
        else if (cache)
          hipLaunchKernelGGL((fa::fwd_bf16_kernel<D, BN, NW, M, fa::BuiltinMod, true>), dim3(grid * a.n_splits),
                             dim3(NW * 64), 0, s, a);
        else
          hipLaunchKernelGGL((fa::fwd_bf16_kernel<D, BN, NW, M>), dim3(grid * a.n_splits), dim3(NW * 64), 0, s, a);
      } else {
        if (cache) return FA_ERR_UNSUPPORTED;  // the KV-cache variant has 128 x 64 tiles
        hipLaunchKernelGGL((fa::fwd_bf16_kernel<D, BN, NW, M, fa::BuiltinMod, false, NS>), dim3(grid * a.n_splits),
                           dim3(NW * 64), 0, s, a);
      }
      if (a.n_splits > 1) {
        const size_t n = (size_t)a.p.B * a.p.Hq * a.p.Sq * D;
        hipLaunchKernelGGL((fa::fwd_split_merge<D>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a);
      }
      return launch_status();
    }
  }
  if constexpr (generic_tile<T, BN, NW>() && NS == 2) {
    FwdArgs g = a;  // the generic kernel has no split-KV, packed or paged form
    g.n_splits = 1;
    g.pack = 0;
    hipLaunchKernelGGL((fa::fwd_kernel<T, D, BN, NW, M>), dim3(fwd_items(a.p, 0, 32 * NW)), dim3(NW * 64), 0, s, g);
    return launch_status();
  }
  return FA_ERR_UNSUPPORTED;  // default_tiles gives generic calls generic tiles
}

template <typename T, int D, bool M>
int launch_fwd(const FwdArgs& a, const Tiles& t, hipStream_t s) {
  if constexpr (sizeof(T) == 2) {
    if constexpr (D >= 64) {
      // LDS stages: 3 with 32-key tiles, 1 with 128-key tiles, else 2
      if (t.bn == 32) return t.ns == 3 ? run_fwd<T, D, 32, 4, M, 3>(a, s) : run_fwd<T, D, 32, 4, M>(a, s);
      if (t.bn == 128) return t.ns == 1 ? run_fwd<T, D, 128, 4, M, 1>(a, s) : run_fwd<T, D, 128, 4, M>(a, s);
      if (t.bm == 256) return run_fwd<T, D, 64, 8, M>(a, s);
    }
    return t.bm == 64 ? run_fwd<T, D, 64, 2, M>(a, s) : run_fwd<T, D, 64, 4, M>(a, s);
  } else {
    return t.bm == 64 ? run_fwd<T, D, 32, 2, M>(a, s) : run_fwd<T, D, 32, 4, M>(a, s);
  }
}

template <typename T, int D, int BN, int NW, bool M>
int run_dq(const BwdArgs& a, hipStream_t s) {
  const int grid = dq_grid(a.p, 32 * NW);
  if constexpr (sizeof(T) == 2) {
    if (interval_masks(a.p)) {
      hipLaunchKernelGGL((fa::dq_bf16_kernel<D, BN, NW, M>), dim3(grid), dim3(NW * 64), 0, s, a);
      return launch_status();
    }
  }
  if constexpr (generic_tile<T, BN, NW>()) {
    hipLaunchKernelGGL((fa::dq_kernel<T, D, BN, NW, M>), dim3(grid), dim3(NW * 64), 0, s, a);
    return launch_status();
  }
  return FA_ERR_UNSUPPORTED;
}

template <typename T, int D, int BQ, int NW, bool M>
int run_dkdv(const BwdArgs& a, hipStream_t s) {
  const int grid = dkdv_grid(a.p, 32 * NW);
  if constexpr (sizeof(T) == 2) {
    if (interval_masks(a.p)) {
      hipLaunchKernelGGL((fa::dkdv_bf16_kernel<D, BQ, NW, M>), dim3(grid), dim3(NW * 64), 0, s, a);
      return launch_status();
    }
  }
  if constexpr (NW == 4 && BQ <= 64) {
    hipLaunchKernelGGL((fa::dkdv_kernel<T, D, BQ, NW, M>), dim3(grid), dim3(NW * 64), 0, s, a);
    return launch_status();
  }
  return FA_ERR_UNSUPPORTED;
}

template <typename T, int D, bool M>
int launch_dq(const BwdArgs& a, const Tiles& t, hipStream_t s) {
  if constexpr (sizeof(T) == 2) {
    if constexpr (D >= 64) {
      if (t.bn == 32) return run_dq<T, D, 32, 4, M>(a, s);
      if (t.bn == 128) return run_dq<T, D, 128, 4, M>(a, s);
      if (t.bm == 256) return run_dq<T, D, 64, 8, M>(a, s);
    }
    return t.bm == 64 ? run_dq<T, D, 64, 2, M>(a, s) : run_dq<T, D, 64, 4, M>(a, s);
  } else {
    return t.bm == 64 ? run_dq<T, D, 32, 2, M>(a, s) : run_dq<T, D, 32, 4, M>(a, s);
  }
}

template <typename T, int D, bool M>
int launch_dkdv(const BwdArgs& a, const Tiles& t, hipStream_t s) {
  constexpr int BQ = sizeof(T) == 2 ? 64 : 32;
  if constexpr (sizeof(T) == 2 && D >= 64) {
    if (t.bkv == 64) return run_dkdv<T, D, BQ, 2, M>(a, s);
    // 128-query tiles (bf16 tile kernel only: the C ABI picks them for
    // interval masks and tables at a multiple of 128)
    if (t.bq == 128) return run_dkdv<T, D, 128, 4, M>(a, s);
  }
  return run_dkdv<T, D, BQ, 4, M>(a, s);
}

template <typename T, int D>
int launch_delta(const BwdArgs& a, hipStream_t s) {
  const int nrows = a.p.B * a.p.Hq * a.p.Sq;
  const int rpb = 256 / (D * (int)sizeof(T) / 16);
  hipLaunchKernelGGL((fa::delta_kernel<T, D>), dim3(cdiv(nrows, rpb)), dim3(256), 0, s, a, nrows);
  return launch_status();
}

#if FA_KERNELS_BWD
template int launch_dq<uint16_t, FA_KERNELS_D, false>(const BwdArgs&, const Tiles&, hipStream_t);
template int launch_dq<uint16_t, FA_KERNELS_D, true>(const BwdArgs&, const Tiles&, hipStream_t);
template int launch_dq<float, FA_KERNELS_D, false>(const BwdArgs&, const Tiles&, hipStream_t);
template int launch_dq<float, FA_KERNELS_D, true>(const BwdArgs&, const Tiles&, hipStream_t);
template int launch_dkdv<uint16_t, FA_KERNELS_D, false>(const BwdArgs&, const Tiles&, hipStream_t);
template int launch_dkdv<uint16_t, FA_KERNELS_D, true>(const BwdArgs&, const Tiles&, hipStream_t);
template int launch_dkdv<float, FA_KERNELS_D, false>(const BwdArgs&, const Tiles&, hipStream_t);
template int launch_dkdv<float, FA_KERNELS_D, true>(const BwdArgs&, const Tiles&, hipStream_t);
template int launch_delta<uint16_t, FA_KERNELS_D>(const BwdArgs&, hipStream_t);
template int launch_delta<float, FA_KERNELS_D>(const BwdArgs&, hipStream_t);
#else
template int launch_fwd<uint16_t, FA_KERNELS_D, false>(const FwdArgs&, const Tiles&, hipStream_t);
template int launch_fwd<uint16_t, FA_KERNELS_D, true>(const FwdArgs&, const Tiles&, hipStream_t);
template int launch_fwd<float, FA_KERNELS_D, false>(const FwdArgs&, const Tiles&, hipStream_t);
template int launch_fwd<float, FA_KERNELS_D, true>(const FwdArgs&, const Tiles&, hipStream_t);
#endif

}  // namespace fa
