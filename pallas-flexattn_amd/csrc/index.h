// Index arithmetic of the kernels, compiled for the device (hipcc, hipRTC)
// and for the host: the CPU bounds-check driver (tests/native/
// kernel_index_check.cpp, built with AddressSanitizer) walks every work item
// of a launch through these same functions and checks each address they
// produce against its buffer.  Work order, block-table rows, key / query
// intervals of the masks, LDS swizzles and per-lane LDS / DMA offsets, tile
// starts from table entries, the table walks and the page addressing of
// KV caches.
#pragma once
#if defined(__HIPCC__) || defined(__HIPCC_RTC__)
#define FA_HD __host__ __device__ __forceinline__
#else
#include <stddef.h>
#include <stdint.h>
#define FA_HD inline
#endif

namespace fa {

FA_HD int imin(int a, int b) { return a < b ? a : b; }
FA_HD int imax(int a, int b) { return a > b ? a : b; }

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
  // tensors read by user score / mask mods compiled at run time
  const void* mod_buf[8];
};

// Keys visible to query q: [lo, hi] (empty when lo > hi).  With delta = q - k,
// delta <= left gives k >= q - left and -delta <= right gives k <= q + right.
FA_HD void key_interval(const Problem& p, int b, int q, int* lo, int* hi) {
  int l = p.win_left >= 0 ? q - p.win_left : 0;
  int h = p.win_right >= 0 ? q + p.win_right : p.Skv - 1;
  if (p.doc_start != nullptr && q < p.Sq) {
    l = imax(l, p.doc_start[(size_t)b * p.Sq + q]);
    h = imin(h, p.doc_end[(size_t)b * p.Sq + q] - 1);
  }
  *lo = imax(l, 0);
  *hi = q < p.Sq ? imin(h, p.Skv - 1) : -1;
}

// Queries that see key k: [lo, hi] (q <= k + left, q >= k - right).
FA_HD void query_interval(const Problem& p, int b, int k, int* lo, int* hi) {
  int l = p.win_right >= 0 ? k - p.win_right : 0;
  int h = p.win_left >= 0 ? k + p.win_left : p.Sq - 1;
  if (p.doc_start != nullptr && k < p.Skv) {
    l = imax(l, p.doc_start[(size_t)b * p.Skv + k]);
    h = imin(h, p.doc_end[(size_t)b * p.Skv + k] - 1);
  }
  *lo = imax(l, 0);
  *hi = k < p.Skv ? imin(h, p.Sq - 1) : -1;
}

// Tile start used for out-of-range table entries: beyond any sequence, so the
// tile is skipped and its loads are predicated off.
constexpr int kPastEnd = 0x40000000;

FA_HD int clamp_count(int n, int width) { return n < 0 ? 0 : (n > width ? width : n); }

// Row of the block tables for (b, h, row).
FA_HD int tab_row(const Problem& p, int b, int h, int row, int nrows) {
  const int tb = p.tab_b == 1 ? 0 : b;
  const int th = p.tab_h == 1 ? 0 : h;
  return (tb * p.tab_h + th) * nrows + row;
}

// First row of the tile of a table entry (block `raw`, sub-tile s of bn rows
// in a mask block of mblk), or kPastEnd for an entry outside [0, nblk).
FA_HD int tile_start(int raw, int nblk, int mblk, int s, int bn) {
  return (raw < 0 || raw >= nblk) ? kPastEnd : raw * mblk + s * bn;
}

// Work-item order: blockIdx.x is dispatched round-robin over the 8 XCDs.  With
// remapping, XCD x processes heads [x*H/8, (x+1)*H/8) in groups of `group`
// heads, one group after another, so the K/V (or Q/dO) of a group stay in
// that XCD's L2 while its tiles run (the host sizes groups to the L2).  Inside
// a group the tiles go level by level across its heads, the longest walks
// first (causal: the last q tiles, or with low_first the first kv tiles), so
// the short tiles fill the end of the grid.
FA_HD void work_item(int bid, int nheads, int ntiles, bool remap, int group, bool low_first, int* head, int* tile) {
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

FA_HD int perm23(int r) { return (r & ~0xc) | ((r & 4) << 1) | ((r & 8) >> 1); }

// physical row (within a 32-row tile) of accumulator element e held by lane half h
FA_HD int acc_row(int e, int h) { return 16 * (e >> 3) + 8 * h + 4 * ((e >> 2) & 1) + (e & 3); }

// ---- LDS tile swizzle ------------------------------------------------------
// Row-major bf16 tiles with KCH 16-byte chunks per row store logical chunk c
// of row r in slot c ^ chunk_swz<KCH>(r).  gfx950's LDS serves 64 banks x 4 B
// per clock: a ds_read_b128 is conflict-free when each group of 16 lanes
// covers 16 distinct 16-byte bank slots, a ds_read_b64_tr_b16 when each group
// of 32 lanes (4 rows x 4 chunks) does.  With KCH = 16 (one row per 256-byte
// bank row) the swizzle maps
//   * the 16 rows an A-operand read takes (any 16-aligned row block, same
//     logical chunk) to 16 distinct slots: f is a bijection on r & 15;
//   * the 4 consecutive rows of a transposing read to 4 distinct quarter-rows:
//     bits 2-3 of f are r & 3.
// KCH = 8 and 4 (two / four rows per bank row) follow the same rules with the
// row's position in the bank row taking the place of the high bits.
template <int KCH>
FA_HD int chunk_swz(int r) {
  static_assert(KCH == 4 || KCH == 8 || KCH == 16, "chunks per row");
  if constexpr (KCH == 16) return ((r & 3) << 2) | ((r >> 2) & 3);
  else if constexpr (KCH == 8) return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
  else return (r >> 2) & 3;
}

// Swizzle for tiles read only by transposing reads (the forward's V): the 4
// rows of a read land in distinct quarter-rows and rows r, r + 4 share their
// swizzle, so a lane's addresses for rows +0..3 and +4..7 differ by a constant.
template <int KCH>
FA_HD int tr_swz(int r) {
  if constexpr (KCH == 16) return 4 * (r & 3);
  else if constexpr (KCH == 8) return 4 * ((r >> 1) & 1);
  else return 0;
}

FA_HD int div_pow2_or(int x, int d, int d_log2) { return d_log2 >= 0 ? x >> d_log2 : x / d; }
FA_HD int log2_if_pow2(int d) { return (d > 0 && (d & (d - 1)) == 0) ? __builtin_ctz(d) : -1; }

// ---- per-lane offsets ------------------------------------------------------
// Reads of a swizzled row-major bf16 tile (rows of D bf16, chunk c of row r
// in slot c ^ chunk_swz(r)): A operand rows perm23(lane % 32) (+32 j) at k
// step s, and transposing reads (two per fragment: rows +0..3 / +4..7) of
// column tile dt.
template <int D>
struct RowTileOffsets {
  static constexpr int RB = D * 2;
  static constexpr int KCH = D / 8;
  static constexpr int KSTEPS = D / 16;
  static constexpr int DT = D / 32;
  int aoff[KSTEPS];  // A operand, rows perm23(lane%32) (+32j), k step s
  int tr[2][DT];     // transposing read: [rows +0..3 / +4..7][d tile]
  FA_HD void init(int lane) {
    const int lr = lane & 31, hh = lane >> 5;
    const int r = perm23(lr);
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) aoff[s] = r * RB + (((2 * s + hh) ^ chunk_swz<KCH>(r)) * 16);
    const int s16 = lane & 15, g = lane >> 4;
    const int rowbase = 8 * (g >> 1) + (s16 >> 2);
    const int x = 2 * (g & 1) + ((s16 & 3) >> 1);
#pragma unroll
    for (int rd = 0; rd < 2; ++rd)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int row = 4 * rd + rowbase;
        tr[rd][dt] = row * RB + (((4 * dt + x) ^ chunk_swz<KCH>(row)) * 16) + (s16 & 1) * 8;
      }
  }
};

// Source offset (bytes from the tile's first row) of the u-th of a wave's
// copy instructions for an R-row tile copied by NW waves, 16 bytes per lane;
// the instruction writes LDS bytes [(w * IPW + u) * 1024, + 1024) of the
// tile, lane l at + 16 l, with chunks swizzled by SW (chunk_swz or tr_swz).
template <int D, int R, int NW, bool kTr = false>
FA_HD int tile_dma_offset(int lane, int w, int u) {
  constexpr int RB = D * 2, KCH = D / 8, IPW = R * RB / 1024 / NW;
  const int g = (w * IPW + u) * 64 + lane;
  const int r = g / KCH, p = g % KCH;
  return r * RB + ((p ^ (kTr ? tr_swz<KCH>(r) : chunk_swz<KCH>(r))) * 16);
}

// The forward's transposing reads of its V tile (tr_swz layout): rows row +
// 16 c (+4 for the upper half of a fragment), chunk 4 i + x of d tile i.
template <int D>
FA_HD int fwd_voff_t(int lane, int i) {
  constexpr int RB = D * 2, KCH = D / 8;
  const int s16 = lane & 15, g = lane >> 4;
  const int row = 8 * (g >> 1) + (s16 >> 2);
  const int x = 2 * (g & 1) + ((s16 & 3) >> 1);
  return row * RB + (((4 * i + x) ^ tr_swz<KCH>(row)) * 16) + (s16 & 1) * 8;
}

// Rows a tile copy reads: first row row0 clamped to the tensor's `rows` and
// the byte range of the buffer resource (rows past the end read as zero).
struct RowSpan {
  int row0;
  uint32_t bytes;
};
FA_HD RowSpan row_span(int row0, int rows, int row_bytes) {
  row0 = row0 < rows ? row0 : rows;
  return RowSpan{row0, (uint32_t)(rows - row0) * (uint32_t)row_bytes};
}

// Paged KV cache: the key tile starting at key kb (< skv) of batch row b lies
// in page pg = kb / page_size; `phys` is that page's table entry.  Returns
// the first cache row (a row = one key of one kv head) and the readable rows:
// to the page's end or the row's length; an entry outside [0, num_pages)
// reads nothing (zeros), never another page.
struct PageSpan {
  size_t row;
  int rows;
};
FA_HD PageSpan page_span(int kb, int pg, int skv, int page_size, int phys, int num_pages, int Hkv, int hk) {
  const int off = kb - pg * page_size;
  const bool ok = phys >= 0 && phys < num_pages;
  const size_t row = ((size_t)(ok ? phys : 0) * Hkv + hk) * page_size + off;
  return PageSpan{row, ok ? imin(page_size - off, skv - kb) : 0};
}

// A tile of a walk whose table entry may still be in flight: fetch() issues
// the load, the walk's resolve step turns the entry into a tile start (an
// iteration or two later, so the load latency is hidden).
struct TileRef {
  int raw;  // table entry, still in a VGPR (dense walks: the tile number)
  int s;    // sub-tile of the mask block
  int hq;   // q head (q-side walks)
};

// kv-tile iteration over block tables (or densely over all tiles).  L: how
// table words are read (the device's scalar / vector loads, or the host
// driver's checked reads): L::scalar(p, i), L::vector(p, i, n) (zero for i
// >= n), L::uniform(x).
template <class L>
struct KvWalkT {
  const int* full;
  const int* part;
  int nfull, npart, sub, bn, mblk, nblk, ntiles_dense;
  bool dense, dense_masked;
  FA_HD int count() const { return dense ? ntiles_dense : (nfull + npart) * sub; }
  // the full tiles come first in the iteration order
  FA_HD int count_full() const { return dense ? (dense_masked ? 0 : ntiles_dense) : nfull * sub; }
  FA_HD TileRef fetch(int it) const {
    TileRef r{it, 0, 0};
    if (!dense) {
      const int bi = div_pow2_or(it, sub, log2_if_pow2(sub));
      r.s = it - bi * sub;
      r.raw = bi < nfull ? L::vector(full, bi, nfull) : L::vector(part, bi - nfull, npart);
    }
    return r;
  }
  FA_HD int kbase(const TileRef& r) const {
    if (dense) return r.raw * bn;
    return tile_start(L::uniform(r.raw), nblk, mblk, r.s, bn);
  }
  FA_HD void get(int it, int* kb, bool* masked) const {
    if (dense) {
      *kb = it * bn;
      *masked = dense_masked;
      return;
    }
    const int bi = it / sub, s = it - bi * sub;
    const int idx = bi < nfull ? L::scalar(full, bi) : L::scalar(part, bi - nfull);
    *masked = bi >= nfull;
    // an out-of-range table entry becomes a tile past the end (skipped)
    *kb = tile_start(idx, nblk, mblk, s, bn);
  }
};

// q-tile walk of the dK/dV kernels over the q-side tables of all q heads in a
// GQA group (L as for KvWalkT)
template <class L>
struct QWalkT {
  const Problem* P;
  int b, hq0, g, kvrow, sub, bq, ntiles_dense;
  bool dense;
  int n_full, n_all;  // set by init()
  // lists of the first head (all heads when the tables do not depend on the head)
  int nf0, np0;
  const int *fl0, *pl0;
  FA_HD void head_lists(int hq, int* nf, const int** fl, int* np, const int** pl) const {
    const int row = tab_row(*P, b, hq, kvrow, P->n_kvblk);
    *nf = P->full_q_num ? clamp_count(L::scalar(P->full_q_num, row), P->q_width) : 0;
    *fl = P->full_q_num ? P->full_q_idx + (size_t)row * P->q_width : nullptr;
    *np = P->q_num ? clamp_count(L::scalar(P->q_num, row), P->q_width) : 0;
    *pl = P->q_num ? P->q_idx + (size_t)row * P->q_width : nullptr;
  }
  // tiles of head hq in the full (part = 0) or partial (part = 1) list
  FA_HD int per_head(int hq, int part) const {
    if (dense) return (part == (P->has_mask ? 1 : 0)) ? ntiles_dense : 0;
    int nf, np;
    const int *fl, *pl;
    head_lists(hq, &nf, &fl, &np, &pl);
    return (part ? np : nf) * sub;
  }
  FA_HD int count_part(int part) const {
    if (dense || P->tab_h == 1) return g * per_head(hq0, part);
    int n = 0;
    for (int i = 0; i < g; ++i) n += per_head(hq0 + i, part);
    return n;
  }
  // Iteration order: the full tiles of every head of the group, then the
  // partial ones, so a kernel can run the two kinds in separate loops.
  FA_HD void init() {
    n_full = count_part(0);
    n_all = n_full + count_part(1);
    nf0 = np0 = 0;
    fl0 = pl0 = nullptr;
    if (!dense) head_lists(hq0, &nf0, &fl0, &np0, &pl0);
  }
  FA_HD int count() const { return n_all; }
  FA_HD int count_full() const { return n_full; }
  // Table lookups stay off the scalar cache for the common layouts (one head,
  // or tables shared by all heads): counts come from init(), the entry
  // through a vector load that the caller consumes a tile later.
  FA_HD TileRef fetch(int it) const {
    const int part = it >= n_full ? 1 : 0;
    int gi = 0, rem = part ? it - n_full : it;
    if (g == 1 && sub == 1) {
      // one q head and one q tile per mask block (the common layout): the
      // entry is the list word itself.  Same result as the general path
      // below, without its head and sub-tile arithmetic, which the four
      // waves of a workgroup would run on the shared scalar unit at the same
      // moment at every tile boundary.
      TileRef r{rem, 0, hq0};
      if (!dense) r.raw = part ? L::vector(pl0, rem, np0) : L::vector(fl0, rem, nf0);
      return r;
    }
    int nf = nf0, np = np0;
    const int *fl = fl0, *pl = pl0;
    if (dense || P->tab_h == 1) {
      if (g > 1) {
        const int c = dense ? per_head(hq0, part) : (part ? np0 : nf0) * sub;
        gi = c > 0 ? rem / c : 0;
        rem -= gi * c;
      }
    } else {
      for (; gi < g - 1; ++gi) {
        const int c = per_head(hq0 + gi, part);
        if (rem < c) break;
        rem -= c;
      }
      if (gi > 0) head_lists(hq0 + gi, &nf, &fl, &np, &pl);
    }
    TileRef r{rem, 0, hq0 + gi};
    if (!dense) {
      const int bi = div_pow2_or(rem, sub, log2_if_pow2(sub));
      r.s = rem - bi * sub;
      r.raw = part ? L::vector(pl, bi, np) : L::vector(fl, bi, nf);
    }
    return r;
  }
  FA_HD int qbase(const TileRef& r) const {
    if (dense) return r.raw * bq;
    return tile_start(L::uniform(r.raw), P->n_qblk, P->mblk_q, r.s, bq);
  }
  // -> q head, first query of the tile, whether the element mask applies
  FA_HD void get(int it, int* hq, int* qb, bool* masked) const {
    const int part = it >= n_full ? 1 : 0;
    int gi = 0, rem = part ? it - n_full : it;
    if (dense || P->tab_h == 1) {
      const int c = per_head(hq0, part);
      gi = c > 0 ? rem / c : 0;
      rem -= gi * c;
    } else {
      for (; gi < g - 1; ++gi) {
        const int c = per_head(hq0 + gi, part);
        if (rem < c) break;
        rem -= c;
      }
    }
    *hq = hq0 + gi;
    *masked = part != 0;
    if (dense) {
      *qb = rem * bq;
      return;
    }
    int nf, np;
    const int *fl, *pl;
    head_lists(*hq, &nf, &fl, &np, &pl);
    const int bi = rem / sub, s = rem - bi * sub;
    const int idx = part ? L::scalar(pl, bi) : L::scalar(fl, bi);
    *qb = tile_start(idx, P->n_qblk, P->mblk_q, s, bq);
  }
};

}  // namespace fa
