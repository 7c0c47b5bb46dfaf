// Kernel argument blocks (passed by value) and the device-side mask /
// score-modification epilogues shared by the forward and backward kernels.
#pragma once
#include "common.h"

namespace fa {

// Element policy of the kernels.  BuiltinMod: the element mask is the window
// / document terms of the Problem and the score epilogue its ALiBi + soft-cap.
// A policy compiled at run time from user mods (fa_mods_build) has the same
// members with kMask / kScore set and
//   static bool  mask(const Problem&, int b, int h, int q, int kv)
//   static float score(const Problem&, float s, int b, int h, int q, int kv, float* dsds)
// where s = scale * q.k, the result is the modified score (natural units)
// and *dsds its derivative with respect to s.
struct BuiltinMod {
  static constexpr bool kMask = false;
  static constexpr bool kScore = false;
  __device__ static bool mask(const Problem&, int, int, int, int) { return true; }
  __device__ static float score(const Problem&, float s, int, int, int, int, float* dsds) {
    *dsds = 1.0f;
    return s;
  }
};

// Window part of the element mask (q, kv inside the sequence bounds).
__device__ __forceinline__ bool window_ok(const Problem& p, int q, int k) {
  const int delta = q - k;
  bool ok = true;
  if (p.win_left >= 0) ok = ok && (delta <= p.win_left);
  if (p.win_right >= 0) ok = ok && (-delta <= p.win_right);
  return ok;
}

// Full element mask given the two document ids (ignored without documents).
__device__ __forceinline__ bool mask_ok(const Problem& p, int q, int k, int qdoc, int kdoc) {
  return window_ok(p, q, k) && (p.q_doc == nullptr || qdoc == kdoc);
}

// True when every mask term is an interval on the other sequence (window
// and/or contiguous documents); false for arbitrary document labels.
__device__ __forceinline__ bool interval_mask(const Problem& p) {
  return p.q_doc == nullptr || p.doc_start != nullptr;
}

__device__ __forceinline__ int kv_doc_of(const Problem& p, int b, int k) {
  return p.q_doc ? p.kv_doc[(size_t)b * p.Skv + k] : 0;
}
__device__ __forceinline__ int q_doc_of(const Problem& p, int b, int q) {
  return p.q_doc ? p.q_doc[(size_t)b * p.Sq + q] : 0;
}

// Score epilogue: raw q.k -> log2-domain logit t = s * log2(e), where
// s = softcap(alibi(scale * raw)).  Also returns d s / d(scale*raw) for the
// backward (1 without soft-cap).
template <bool kMods>
__device__ __forceinline__ float score_t(const Problem& p, float raw, float slope, int q, int k,
                                         float* dsdx) {
  if constexpr (!kMods) {
    if (dsdx) *dsdx = 1.0f;
    return raw * p.scale_log2;
  } else {
    float s = raw * p.scale;
    if (p.alibi) s += slope * (float)(k - q);
    if (p.softcap > 0.f) {
      const float th = tanh_fast(s * (1.0f / p.softcap));
      s = p.softcap * th;
      if (dsdx) *dsdx = 1.0f - th * th;
    } else if (dsdx) {
      *dsdx = 1.0f;
    }
    return s * kLog2e;
  }
}

// score_t<true> without branches, for straight-line tile schedules: the
// soft-cap's tanh is always evaluated and selected (cap_inv = 1 / softcap, or
// 0 without a soft-cap; slope 0 without ALiBi).
__device__ __forceinline__ float score_mods_flat(float raw, float scale, float slope, int q, int k, float softcap,
                                                 float cap_inv, float* dsdx) {
  float s = fmaf(slope, (float)(k - q), raw * scale);
  const float th = tanh_fast(s * cap_inv);
  const bool capped = softcap > 0.f;
  *dsdx = capped ? fmaf(-th, th, 1.0f) : 1.0f;
  s = capped ? softcap * th : s;
  return s * kLog2e;
}

// Log2-domain logit of raw q.k under the policy: a user score mod, or the
// built-in ALiBi + soft-cap epilogue (score_mods_flat).
template <class Mod>
__device__ __forceinline__ float mod_score_flat(const Problem& P, float raw, float slope, int b, int h, int q, int k,
                                                float cap_inv, float* dsdx) {
  if constexpr (Mod::kScore) return Mod::score(P, raw * P.scale, b, h, q, k, dsdx) * kLog2e;
  else return score_mods_flat(raw, P.scale, slope, q, k, P.softcap, cap_inv, dsdx);
}

// score_t under the policy (generic kernels).
template <class Mod, bool kMods>
__device__ __forceinline__ float mod_score_t(const Problem& P, float raw, float slope, int b, int h, int q, int k,
                                             float* dsdx) {
  if constexpr (Mod::kScore) {
    float d;
    const float t = Mod::score(P, raw * P.scale, b, h, q, k, &d) * kLog2e;
    if (dsdx) *dsdx = d;
    return t;
  } else {
    return score_t<kMods>(P, raw, slope, q, k, dsdx);
  }
}

// Element (q, k) of a partial tile is kept: inside [lo, hi] (the interval
// of keys the window / contiguous documents leave to query q, which also
// bounds k below Skv) and, with a user mask, where the mask holds.
template <class Mod>
__device__ __forceinline__ bool mod_keep(const Problem& P, int b, int h, int q, int k, int lo, int hi) {
  if constexpr (Mod::kMask) return k >= lo && k <= hi && Mod::mask(P, b, h, q, k);
  else return k >= lo && k <= hi;
}

// mask_ok under the policy (generic kernels).
template <class Mod>
__device__ __forceinline__ bool mod_mask_ok(const Problem& P, int b, int h, int q, int k, int qdoc, int kdoc) {
  if constexpr (Mod::kMask) return mask_ok(P, q, k, qdoc, kdoc) && Mod::mask(P, b, h, q, k);
  else return mask_ok(P, q, k, qdoc, kdoc);
}

}  // namespace fa
