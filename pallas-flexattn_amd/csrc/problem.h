// Host-side problem set-up of the C ABI, plain C++ (no HIP): the checks of
// fa_params, the Problem the kernels get (masks, tables, work order), the
// kernel tiles of a call and the launch geometry.  Shared by the library
// (capi.hip, kernels.hip) and the CPU bounds-check driver
// (tests/native/kernel_index_check.cpp), which feeds every launch it models
// through these same functions.
#pragma once
#include <math.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/flexattn.h"
#include "index.h"

namespace fa {

struct Tiles {
  int bm, bn;    // forward / dQ: query tile, key tile
  int bkv, bq;   // dK/dV: key tile, query tile
  int ns;        // forward: K / V tiles held in LDS (stages)
};

inline int cdiv(int a, int b) { return (a + b - 1) / b; }

// The bf16 LDS-DMA kernels evaluate masks as per-lane intervals (windows and
// contiguous documents); arbitrary document labels go to the generic kernels.
inline bool interval_masks(const Problem& p) { return p.q_doc == nullptr || p.doc_start != nullptr; }

// Work items of the forward: (batch, q head, query tile), or with GQA row
// packing (batch, kv head, tile of the group's g * Sq rows).
inline int fwd_items(const Problem& p, int pack, int bm) {
  return pack > 1 ? p.B * p.Hkv * cdiv(pack * p.Sq, bm) : p.B * p.Hq * cdiv(p.Sq, bm);
}

// Workgroups of the dQ and dK/dV launches.
inline int dq_grid(const Problem& p, int bm) { return p.B * p.Hq * cdiv(p.Sq, bm); }
inline int dkdv_grid(const Problem& p, int bkv) { return p.B * p.Hkv * cdiv(p.Skv, bkv); }

// The tiles of a call: the requested ones (0 = default) where an
// instantiation exists.  bf16 interval kernels: (bm, bn) in {(128, 64),
// (64, 64)} and, for D >= 64, {(128, 32), (128, 128), (256, 64)}; dK/dV key
// tile bkv 128, or 64 for D >= 64; forward LDS stages 2, or 3 with bn 32 and
// 1 with bn 128.  The generic kernels (document labels compared per
// element; every fp32 call) keep their own tiles: bm at most 128, bn, bkv and
// the stages at the defaults.  The dK/dV query tile (bq) is settled by the
// backward (dkdv_query_tile): 0 here means automatic.
inline int default_tiles(const fa_params* p, Tiles* t) {
  t->bm = p->block_m ? p->block_m : 128;
  t->bkv = p->block_kv ? p->block_kv : 128;
  t->bq = p->block_q;
  t->ns = p->lds_stages ? p->lds_stages : 2;
  if (p->dtype == FA_DTYPE_BF16) {
    t->bn = p->block_n ? p->block_n : 64;
    if (p->q_doc_ids && !p->doc_start) {  // generic kernel
      if (t->bm == 256) t->bm = 128;
      t->bn = 64;
      t->bkv = 128;
      t->ns = 2;
    }
    const bool base = (t->bm == 128 || t->bm == 64) && t->bn == 64;
    const bool wide = (t->bm == 128 && (t->bn == 32 || t->bn == 128)) || (t->bm == 256 && t->bn == 64);
    if (!(base || (wide && p->D >= 64))) return FA_ERR_UNSUPPORTED;
    if (!(t->bkv == 128 || (t->bkv == 64 && p->D >= 64))) return FA_ERR_UNSUPPORTED;
    const bool stages = t->ns == 2 || (t->ns == 3 && t->bn == 32) || (t->ns == 1 && t->bn == 128);
    if (!stages) return FA_ERR_UNSUPPORTED;
    if (!(t->bq == 0 || t->bq == 64 || t->bq == 128)) return FA_ERR_UNSUPPORTED;
  } else if (p->dtype == FA_DTYPE_FP8_E4M3) {  // forward only: 128 x 64
    t->bn = p->block_n ? p->block_n : 64;
    if (!(t->bm == 128 && t->bn == 64 && t->bkv == 128 && t->ns == 2 && t->bq == 0)) return FA_ERR_UNSUPPORTED;
    t->bq = 64;
  } else {
    t->bn = p->block_n ? p->block_n : 32;
    if (!((t->bm == 128 || t->bm == 64) && t->bn == 32 && t->bkv == 128 && t->ns == 2)) return FA_ERR_UNSUPPORTED;
    if (!(t->bq == 0 || t->bq == 32)) return FA_ERR_UNSUPPORTED;
    t->bq = 32;
  }
  return FA_OK;
}

// The dK/dV query tile of a bf16 backward.  128 rows (four 32-row sub-tiles,
// half the tile boundaries of 64) run with the interval-mask kernel, D >= 64,
// 128-key workgroups and q-side tables at a multiple of 128 rows; the
// automatic choice takes them for D = 128 (step 9.10-9.14 against 9.33-9.36 ms
// at causal B4 H32 S8192 D128) and 64 rows otherwise (D = 64: the 64-row tile
// is 6 % faster at causal B4 H32 S4096, tuner measurement).  A requested tile
// (fa_params.block_q) that the call cannot run is refused.
inline int dkdv_query_tile(const fa_params* p, const Problem& pr, Tiles* t) {
  if (p->dtype != FA_DTYPE_BF16) return FA_OK;  // fp32: 32 (default_tiles)
  const bool q128 = p->D >= 64 && t->bkv == 128 && interval_masks(pr) && (!pr.has_tables || pr.mblk_q % 128 == 0);
  if (t->bq == 0) t->bq = (q128 && p->D >= 128) ? 128 : 64;
  return (t->bq == 128 && !q128) ? FA_ERR_UNSUPPORTED : FA_OK;
}

// Byte budgets of a head group: the L2 of one XCD is 4 MiB; q-tile walks
// (forward, dQ) measured best at twice that (the misses hit the MALL and the
// wider level-major groups balance the grid's tail), kv-tile walks (dK/dV) at
// the L2 size.
constexpr size_t kGroupBytesQ = 8u << 20;
constexpr size_t kGroupBytesKV = 4u << 20;
// largest power of two g dividing the heads of one XCD with g * bytes <= budget
inline int head_group(int nheads, size_t bytes_per_head, size_t budget) {
  const int hpx = nheads % 8 == 0 ? nheads / 8 : 1;
  int g = 1;
  while (hpx % (2 * g) == 0 && (size_t)(2 * g) * bytes_per_head <= budget) g *= 2;
  return g;
}

inline int build_problem(const fa_params* p, const Tiles& t, Problem* pr) {
  if (!p) return FA_ERR_NULL;
  if (p->abi_version != FA_ABI_VERSION) return FA_ERR_VERSION;
  if (p->dtype != FA_DTYPE_BF16 && p->dtype != FA_DTYPE_F32 && p->dtype != FA_DTYPE_FP8_E4M3) return FA_ERR_DTYPE;
  if (p->B < 1 || p->Hq < 1 || p->Hkv < 1 || p->Sq < 1 || p->Skv < 1) return FA_ERR_SHAPE;
  if (p->Hq % p->Hkv != 0) return FA_ERR_SHAPE;
  if (p->D != 32 && p->D != 64 && p->D != 128) return FA_ERR_UNSUPPORTED;
  if (!(p->softcap >= 0.f) || !(p->scale >= 0.f)) return FA_ERR_SHAPE;
  if ((p->q_doc_ids == nullptr) != (p->kv_doc_ids == nullptr)) return FA_ERR_NULL;
  Problem& r = *pr;
  r.B = p->B;
  r.Hq = p->Hq;
  r.Hkv = p->Hkv;
  r.Sq = p->Sq;
  r.Skv = p->Skv;
  r.scale = p->scale > 0.f ? p->scale : 1.0f / sqrtf((float)p->D);
  r.scale_log2 = r.scale * 1.4426950408889634f;  // log2(e)
  r.win_left = p->window_left < 0 ? -1 : p->window_left;
  r.win_right = p->window_right < 0 ? -1 : p->window_right;
  r.q_doc = p->q_doc_ids;
  r.kv_doc = p->kv_doc_ids;
  if ((p->doc_start == nullptr) != (p->doc_end == nullptr)) return FA_ERR_NULL;
  if (p->doc_start && (!p->q_doc_ids || p->Sq != p->Skv)) return FA_ERR_SHAPE;
  r.doc_start = p->doc_start;
  r.doc_end = p->doc_end;
  r.alibi = p->alibi_slopes;
  r.softcap = p->softcap;
  r.has_mask = (r.win_left >= 0 || r.win_right >= 0 || r.q_doc != nullptr) ? 1 : 0;
  r.xcd_remap = 1;
  // heads per level-major group: as many as keep their K/V (forward, dQ) or
  // Q/dO (dK/dV, all q heads of a kv head) within the group budget
  {
    const size_t es = p->dtype == FA_DTYPE_BF16 ? 2 : p->dtype == FA_DTYPE_F32 ? 4 : 1;
    const size_t kv_head = 2 * (size_t)p->Skv * p->D * es / (size_t)(p->Hq / p->Hkv);
    const size_t q_heads = 2 * (size_t)p->Sq * p->D * es * (size_t)(p->Hq / p->Hkv);
    r.head_group_q = head_group(p->B * p->Hq, kv_head, kGroupBytesQ);
    r.head_group_kv = head_group(p->B * p->Hkv, q_heads, kGroupBytesKV);
  }
  r.kv_num = p->kv_num_blocks;
  r.kv_idx = p->kv_indices;
  r.full_kv_num = p->full_kv_num_blocks;
  r.full_kv_idx = p->full_kv_indices;
  r.q_num = p->q_num_blocks;
  r.q_idx = p->q_indices;
  r.full_q_num = p->full_q_num_blocks;
  r.full_q_idx = p->full_q_indices;
  r.has_tables = (r.kv_num || r.full_kv_num || r.q_num || r.full_q_num) ? 1 : 0;
  if (r.has_tables) {
    if ((r.kv_num == nullptr) != (r.kv_idx == nullptr)) return FA_ERR_TABLES;
    if ((r.full_kv_num == nullptr) != (r.full_kv_idx == nullptr)) return FA_ERR_TABLES;
    if ((r.q_num == nullptr) != (r.q_idx == nullptr)) return FA_ERR_TABLES;
    if ((r.full_q_num == nullptr) != (r.full_q_idx == nullptr)) return FA_ERR_TABLES;
    if (p->mask_block_q < 1 || p->mask_block_kv < 1) return FA_ERR_TABLES;
    if (p->table_b != 1 && p->table_b != p->B) return FA_ERR_TABLES;
    if (p->table_h != 1 && p->table_h != p->Hq) return FA_ERR_TABLES;
    if (p->kv_width < 0 || p->q_width < 0) return FA_ERR_TABLES;
    r.mblk_q = p->mask_block_q;
    r.mblk_kv = p->mask_block_kv;
  } else {
    r.mblk_q = t.bm;
    r.mblk_kv = t.bn;
  }
  r.tab_b = p->table_b < 1 ? 1 : p->table_b;
  r.tab_h = p->table_h < 1 ? 1 : p->table_h;
  r.kv_width = p->kv_width;
  r.q_width = p->q_width;
  r.n_qblk = cdiv(p->Sq, r.mblk_q);
  r.n_kvblk = cdiv(p->Skv, r.mblk_kv);
  return FA_OK;
}

// GQA row packing: for query blocks shorter than a tile, the g = Hq / Hkv
// heads sharing a kv head run as one work item, so each K / V tile is read
// once for the group instead of once per head (decode shapes).  Needs the
// bf16 interval kernel and block tables (if any) shared by all heads with Sq
// inside one mask block.
inline int choose_pack(const fa_params* p, const Tiles& t, const Problem& pr) {
  const int g = p->Hq / p->Hkv;
  if (p->dtype != FA_DTYPE_BF16 || !interval_masks(pr) || g < 2 || p->Sq >= t.bm || t.bm != 128 || t.bn != 64)
    return 0;
  if (pr.has_tables && (pr.tab_h != 1 || p->Sq > pr.mblk_q)) return 0;
  return g;
}

// Split-KV: the requested count (<= 0: about two workgroups per CU of the
// cus compute units, at least four key tiles per split), or 1 where the
// generic kernel runs.
inline int choose_splits(const fa_params* p, const Tiles& t, const Problem& pr, int requested, int cus) {
  if (p->dtype != FA_DTYPE_BF16 || !interval_masks(pr)) return 1;
  const int items = fwd_items(pr, choose_pack(p, t, pr), t.bm);
  const int max_by_keys = cdiv(p->Skv, 4 * t.bn);
  int n = requested;
  if (n <= 0) n = cdiv(2 * cus, items);
  if (n > max_by_keys) n = max_by_keys;
  if (n > 64) n = 64;
  return n < 1 ? 1 : n;
}

inline size_t split_bytes(const fa_params* p, int n) {
  return n > 1 ? (size_t)n * p->B * p->Hq * p->Sq * (p->D + 2) * sizeof(float) : 0;
}

}  // namespace fa
