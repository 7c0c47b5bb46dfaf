// Kernel argument blocks (passed by value) and the device-side mask /
// score-modification epilogues shared by the forward and backward kernels.
#pragma once
#include "common.h"

namespace fa {

// Everything a kernel needs to know about the attention problem except the
// tensor pointers.  Built on the host from fa_params.
struct Problem {
  int B, Hq, Hkv, Sq, Skv;
  float scale;       // softmax scale applied to q.k
  float scale_log2;  // scale * log2(e)
  // mask: window on delta = q - kv (left/right < 0: unlimited) and documents
  int win_left, win_right;
  const int* q_doc;   // (B, Sq) or null
  const int* kv_doc;  // (B, Skv) or null
  // contiguous documents (self-attention): token t's document is
  // [doc_start[b][t], doc_end[b][t]); when set, masks are key/query intervals
  const int* doc_start;
  const int* doc_end;
  // score modification: s += alibi[h] * (kv - q); then s = cap * tanh(s / cap)
  const float* alibi;  // (Hq) or null
  float softcap;       // <= 0: off
  // block tables at mask-block granularity (PyTorch BlockMask convention:
  // kv_* lists the partial blocks, full_kv_* the fully-live ones)
  const int *kv_num, *kv_idx, *full_kv_num, *full_kv_idx;  // rows = q mask blocks
  const int *q_num, *q_idx, *full_q_num, *full_q_idx;      // rows = kv mask blocks
  int tab_b, tab_h;      // 1 or B, 1 or Hq
  int n_qblk, n_kvblk;   // table rows (q side / kv side)
  int kv_width, q_width;
  int mblk_q, mblk_kv;   // mask block sizes
  int has_tables;        // 0: dense iteration over all blocks
  int has_mask;          // any window / doc term active
  int xcd_remap;         // group work of a head onto one XCD
  int head_group_q;      // heads per level-major group, q-tile walks (forward, dQ)
  int head_group_kv;     // the same for kv-tile walks (dK/dV)
  // tensors read by user score / mask mods compiled at run time (see Mod below)
  const void* mod_buf[8];
};

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

// Keys visible to query q: [lo, hi] (empty when lo > hi).  With delta = q - k,
// delta <= left gives k >= q - left and -delta <= right gives k <= q + right.
__device__ __forceinline__ void key_interval(const Problem& p, int b, int q, int* lo, int* hi) {
  int l = p.win_left >= 0 ? q - p.win_left : 0;
  int h = p.win_right >= 0 ? q + p.win_right : p.Skv - 1;
  if (p.doc_start != nullptr && q < p.Sq) {
    l = max(l, p.doc_start[(size_t)b * p.Sq + q]);
    h = min(h, p.doc_end[(size_t)b * p.Sq + q] - 1);
  }
  *lo = max(l, 0);
  *hi = q < p.Sq ? min(h, p.Skv - 1) : -1;
}

// Queries that see key k: [lo, hi] (q <= k + left, q >= k - right).
__device__ __forceinline__ void query_interval(const Problem& p, int b, int k, int* lo, int* hi) {
  int l = p.win_right >= 0 ? k - p.win_right : 0;
  int h = p.win_left >= 0 ? k + p.win_left : p.Sq - 1;
  if (p.doc_start != nullptr && k < p.Skv) {
    l = max(l, p.doc_start[(size_t)b * p.Skv + k]);
    h = min(h, p.doc_end[(size_t)b * p.Skv + k] - 1);
  }
  *lo = max(l, 0);
  *hi = k < p.Skv ? min(h, p.Sq - 1) : -1;
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

// Tile start used for out-of-range table entries: beyond any sequence, so the
// tile is skipped and its loads are predicated off.
constexpr int kPastEnd = 0x40000000;

__device__ __forceinline__ int clamp_count(int n, int width) { return n < 0 ? 0 : (n > width ? width : n); }

// Row of the block tables for (b, h, row).
__device__ __forceinline__ int tab_row(const Problem& p, int b, int h, int row, int nrows) {
  const int tb = p.tab_b == 1 ? 0 : b;
  const int th = p.tab_h == 1 ? 0 : h;
  return (tb * p.tab_h + th) * nrows + row;
}

// Work-item order: blockIdx.x is dispatched round-robin over the 8 XCDs.  With
// remapping, XCD x processes heads [x*H/8, (x+1)*H/8) in groups of `group`
// heads, one group after another, so the K/V (or Q/dO) of a group stay in
// that XCD's L2 while its tiles run (the host sizes groups to the L2).  Inside
// a group the tiles go level by level across its heads, the longest walks
// first (causal: the last q tiles, or with low_first the first kv tiles), so
// the short tiles fill the end of the grid.
__device__ __forceinline__ void work_item(int bid, int nheads, int ntiles, bool remap, int group, bool low_first,
                                          int* head, int* tile) {
  int t;
  if (remap && (nheads % 8) == 0) {
    const int xcd = bid & 7, slot = bid >> 3;
    const int hpx = nheads >> 3;
    const int per_group = group * ntiles;
    const int gi = slot / per_group, r = slot - gi * per_group;
    *head = xcd * hpx + gi * group + r % group;
    t = r / group;
  } else {
    *head = bid / ntiles;
    t = bid % ntiles;
  }
  *tile = low_first ? t : ntiles - 1 - t;
}

}  // namespace fa
