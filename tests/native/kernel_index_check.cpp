// Bounds check of the bf16 tile kernels' index arithmetic on the CPU.
//
// The kernels' work order, block-table walks, mask intervals, per-lane LDS /
// DMA offsets, buffer-resource ranges and page addressing live in
// csrc/index.h, and the host set-up of a call (fa_params checks, the Problem
// the kernels get, tiles, launch geometry) in csrc/problem.h; both compile
// here unchanged.  For each problem read from a case file (tables built by the
// package's create_block_mask) this driver enumerates every workgroup of the
// forward (also split-KV, GQA-packed and paged), dQ and dK/dV launches at the
// given tiles, runs each through those functions in the kernels' order, and
// checks every address they produce:
//   * table and document reads go through exact-size heap arrays (so
//     AddressSanitizer sees any overread) and are also checked against the
//     array bounds;
//   * buffer resources (tile copies, register loads, statistics) must lie
//     inside their tensor's head, the per-lane offsets inside the tile;
//   * LDS offsets (copy destinations, operand reads, staging) inside the
//     kernel's LDS allocation, tile reads inside their tile;
//   * stores (O, LSE, Delta, dQ, dK, dV, split partials) inside their tensor.
// Prints "ok <cases> <checks>"; the first violation aborts with its location.
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "problem.h"

using namespace fa;

static long long g_checks = 0;
static const char* g_where = "";

[[noreturn]] static void fail(const char* fmt, ...) {
  std::fprintf(stderr, "bounds violation [%s]: ", g_where);
  va_list ap;
  va_start(ap, fmt);
  std::vfprintf(stderr, fmt, ap);
  va_end(ap);
  std::fprintf(stderr, "\n");
  std::abort();
}

// [off, off + len) inside [0, size)
static void inside(long long off, long long len, long long size, const char* what) {
  ++g_checks;
  if (off < 0 || len < 0 || off + len > size) fail("%s: [%lld, %lld) outside [0, %lld)", what, off, off + len, size);
}

// ---- table arrays: exact-size heap copies, every read checked -------------
struct IntArray {
  const int* p;
  long long n;
};
static std::vector<IntArray> g_arrays;

static const IntArray& owner(const int* p, const char* what) {
  for (const auto& a : g_arrays)
    if (p >= a.p && p <= a.p + a.n) return a;
  fail("%s: pointer %p outside every table array", what, (const void*)p);
}

// Reads of the walks (the host side of index.h's load policy).
struct HostLoad {
  static int scalar(const int* p, int i) {
    const IntArray& a = owner(p, "scalar table read");
    inside((p - a.p) + i, 1, a.n, "scalar table read");
    return p[i];
  }
  // buffer resource over n entries at p: the resource must lie in the array;
  // reads past n return zero (as the hardware's range check does)
  static int vector(const int* p, int i, int n) {
    const IntArray& a = owner(p, "vector table resource");
    inside(p - a.p, n, a.n, "vector table resource");
    return (i >= 0 && i < n) ? p[i] : 0;
  }
  static int uniform(int x) { return x; }
};

// ---- case file ---------------------------------------------------------------
struct Case {
  int B, Hq, Hkv, Sq, Skv, D;
  int win_left, win_right, docs, tables, mblk, tab_b, tab_h, kv_width, q_width;
  int paged, page_size, max_pages, num_pages, kv_lens, all_tiles;
  std::vector<int*> owned;
  fa_params p;
};

static int* read_array(FILE* f, long long n, Case& c) {
  int* a = static_cast<int*>(std::malloc(sizeof(int) * (n > 0 ? n : 1)));
  if (n > 0 && std::fread(a, sizeof(int), (size_t)n, f) != (size_t)n) {
    std::fprintf(stderr, "short case file\n");
    std::exit(2);
  }
  c.owned.push_back(a);
  g_arrays.push_back({a, n});
  return a;
}

static bool read_case(FILE* f, Case& c) {
  int hdr[22];
  if (std::fread(hdr, sizeof(int), 22, f) != 22) return false;
  int* h = hdr;
  c.B = *h++; c.Hq = *h++; c.Hkv = *h++; c.Sq = *h++; c.Skv = *h++; c.D = *h++;
  c.win_left = *h++; c.win_right = *h++; c.docs = *h++; c.tables = *h++; c.mblk = *h++;
  c.tab_b = *h++; c.tab_h = *h++; c.kv_width = *h++; c.q_width = *h++;
  c.paged = *h++; c.page_size = *h++; c.max_pages = *h++; c.num_pages = *h++; c.kv_lens = *h++;
  c.all_tiles = *h++;
  const int magic = *h++;
  if (magic != 0x46414958) {
    std::fprintf(stderr, "bad case file\n");
    std::exit(2);
  }
  std::memset(&c.p, 0, sizeof(c.p));
  fa_params& p = c.p;
  p.abi_version = FA_ABI_VERSION;
  p.dtype = FA_DTYPE_BF16;
  p.B = c.B; p.Hq = c.Hq; p.Hkv = c.Hkv; p.Sq = c.Sq; p.Skv = c.Skv; p.D = c.D;
  p.window_left = c.win_left;
  p.window_right = c.win_right;
  if (c.docs) {
    p.q_doc_ids = read_array(f, (long long)c.B * c.Sq, c);
    p.kv_doc_ids = read_array(f, (long long)c.B * c.Skv, c);
    p.doc_start = read_array(f, (long long)c.B * c.Sq, c);
    p.doc_end = read_array(f, (long long)c.B * c.Sq, c);
  }
  if (c.tables) {
    const long long rq = (long long)c.tab_b * c.tab_h * ((c.Sq + c.mblk - 1) / c.mblk);
    const long long rk = (long long)c.tab_b * c.tab_h * ((c.Skv + c.mblk - 1) / c.mblk);
    p.mask_block_q = p.mask_block_kv = c.mblk;
    p.table_b = c.tab_b;
    p.table_h = c.tab_h;
    p.kv_width = c.kv_width;
    p.q_width = c.q_width;
    p.kv_num_blocks = read_array(f, rq, c);
    p.kv_indices = read_array(f, rq * c.kv_width, c);
    p.full_kv_num_blocks = read_array(f, rq, c);
    p.full_kv_indices = read_array(f, rq * c.kv_width, c);
    p.q_num_blocks = read_array(f, rk, c);
    p.q_indices = read_array(f, rk * c.q_width, c);
    p.full_q_num_blocks = read_array(f, rk, c);
    p.full_q_indices = read_array(f, rk * c.q_width, c);
  }
  return true;
}

// ---- forward (fwd_bf16_kernel) -------------------------------------------
struct FwdOpts {
  int pack = 0, n_splits = 1;
  const int* page_table = nullptr;
  int page_size = 0, max_pages = 0, num_pages = 0;
  const int* kv_lens = nullptr;
};

template <int D, int BN, int NW, int NS>
static void model_fwd(const Problem& P, const FwdOpts& o) {
  constexpr int BM = 32 * NW, RB = D * 2, KSTEPS = D / 16, DT = D / 32, NSUB = BN / 32, TILE = BN * RB;
  constexpr int IPW = TILE / 1024 / NW;
  constexpr int LDS = 2 * NS * TILE;
  // lane-constant offsets: copies into each buffer, K A-operand reads, V^T reads
  for (int w = 0; w < NW; ++w)
    for (int lane = 0; lane < 64; ++lane) {
      for (int u = 0; u < IPW; ++u) {
        inside(tile_dma_offset<D, BN, NW>(lane, w, u), 16, TILE, "fwd K copy source (within the tile)");
        inside(tile_dma_offset<D, BN, NW, true>(lane, w, u), 16, TILE, "fwd V copy source (within the tile)");
        for (int buf = 0; buf < NS; ++buf) {
          inside(buf * TILE + (w * IPW + u) * 1024 + 16 * lane, 16, LDS, "fwd K copy into LDS");
          inside((NS + buf) * TILE + (w * IPW + u) * 1024 + 16 * lane, 16, LDS, "fwd V copy into LDS");
        }
      }
      RowTileOffsets<D> kt;
      kt.init(lane);
      for (int s = 0; s < KSTEPS; ++s)
        for (int j = 0; j < NSUB; ++j) inside(j * 32 * RB + kt.aoff[s], 16, TILE, "fwd K operand read");
      for (int i = 0; i < DT; ++i)
        for (int c = 0; c < BN / 16; ++c) {
          inside(fwd_voff_t<D>(lane, i) + 16 * c * RB, 8, TILE, "fwd V^T read (rows +0..3)");
          inside(fwd_voff_t<D>(lane, i) + (16 * c + 4) * RB, 8, TILE, "fwd V^T read (rows +4..7)");
        }
      // O staging: the wave's 32 rows of 2D bytes
      inside(w * 32 * RB, 32 * RB, LDS, "fwd O staging");
    }
  const int g = P.Hq / P.Hkv;
  const bool pack = o.pack > 1;
  const int rows = pack ? g * P.Sq : P.Sq;
  const int nheads = pack ? P.B * P.Hkv : P.B * P.Hq;
  const int nqt = (rows + BM - 1) / BM;
  const int n_items = nheads * nqt;
  const long long q_rows = (long long)P.B * P.Hq * P.Sq;
  const long long kv_rows = o.page_table ? (long long)o.num_pages * P.Hkv * o.page_size : (long long)P.B * P.Hkv * P.Skv;
  for (int bid = 0; bid < n_items * o.n_splits; ++bid) {
    const int split = o.n_splits > 1 ? bid / n_items : 0;
    int head, qt;
    work_item(bid - split * n_items, nheads, nqt, P.xcd_remap, pack ? 1 : P.head_group_q, false, &head, &qt);
    inside(head, 1, nheads, "fwd work item head");
    inside(qt, 1, nqt, "fwd work item tile");
    const int b = head / (pack ? P.Hkv : P.Hq);
    const int hk = pack ? head - b * P.Hkv : (head - b * P.Hq) / g;
    const long long row0 = pack ? (long long)(b * P.Hq + hk * g) * P.Sq : (long long)head * P.Sq;
    const int q0 = qt * BM;
    const int hu = pack ? hk * g : head - b * P.Hq;
    int skv = P.Skv;
    if (o.kv_lens) {
      skv = HostLoad::scalar(o.kv_lens, b);
      skv = skv < 0 ? 0 : (skv > P.Skv ? P.Skv : skv);
    }
    // Q rows: one resource over the work item's rows
    inside(row0, rows, q_rows, "fwd Q resource");
    for (int w = 0; w < NW; ++w)
      for (int lane = 0; lane < 64; ++lane) {
        const int rw = q0 + 32 * w + (lane & 31);
        const bool qvalid = rw < rows;
        const int qw = pack ? rw % P.Sq : rw;
        const int h = pack ? hu + rw / P.Sq : hu;
        if (P.alibi) inside(h, 1, P.Hq, "fwd ALiBi slope");
        int klo, khi;
        key_interval(P, b, qw, &klo, &khi);
        if (qvalid && (lane >> 5) == 0) {
          if (o.n_splits > 1) {
            inside(((long long)split * q_rows + row0 + rw) * D, D, (long long)o.n_splits * q_rows * D,
                   "fwd split partial O");
            inside(((long long)split * q_rows + row0 + rw) * 2, 2, (long long)o.n_splits * q_rows * 2,
                   "fwd split partial (m, l)");
          } else {
            inside(row0 + rw, 1, q_rows, "fwd LSE store");
          }
        }
      }
    if (o.n_splits <= 1)  // O rows: 32 per wave, rows past the item not stored
      for (int w = 0; w < NW; ++w) {
        const int left = rows - (q0 + 32 * w);
        for (int rr = 0; rr < 32 && rr < left; ++rr) inside((row0 + q0 + 32 * w + rr) * D, D, q_rows * D, "fwd O store");
      }
    // the kv walk
    KvWalkT<HostLoad> walk;
    walk.bn = BN;
    walk.mblk = P.mblk_kv;
    walk.sub = P.mblk_kv / BN;
    walk.nblk = P.n_kvblk;
    walk.dense = !P.has_tables;
    walk.ntiles_dense = (skv + BN - 1) / BN;
    walk.dense_masked = P.has_mask;
    walk.full = walk.part = nullptr;
    walk.nfull = walk.npart = 0;
    if (P.has_tables) {
      const int row = tab_row(P, b, hu, pack ? 0 : q0 / P.mblk_q, P.n_qblk);
      if (P.full_kv_num) {
        walk.nfull = clamp_count(HostLoad::scalar(P.full_kv_num, row), P.kv_width);
        walk.full = P.full_kv_idx + (long long)row * P.kv_width;
      }
      if (P.kv_num) {
        walk.npart = clamp_count(HostLoad::scalar(P.kv_num, row), P.kv_width);
        walk.part = P.kv_idx + (long long)row * P.kv_width;
      }
    }
    const int n_it = walk.count();
    const int it0 = o.n_splits > 1 ? (int)((long long)n_it * split / o.n_splits) : 0;
    const int it1 = o.n_splits > 1 ? (int)((long long)n_it * (split + 1) / o.n_splits) : n_it;
    const long long head_kv = (long long)(b * P.Hkv + hk) * P.Skv;
    for (int it = it0; it < it1; ++it) {
      const int kb = walk.kbase(walk.fetch(it));
      // the tile's copy (issued a tile or two earlier): rows [row0, skv) of the head
      const RowSpan sp = row_span(kb, skv, RB);
      if (o.page_table) {
        if (sp.row0 < skv) {
          const int pg = sp.row0 / o.page_size;
          const int phys = HostLoad::scalar(o.page_table + (long long)b * o.max_pages, pg);
          inside((long long)b * o.max_pages + pg, 1, (long long)P.B * o.max_pages, "page table read");
          const PageSpan ps = page_span(sp.row0, pg, skv, o.page_size, phys, o.num_pages, P.Hkv, hk);
          inside((long long)ps.row, ps.rows, kv_rows, "paged K / V resource");
          inside(sp.row0 - pg * o.page_size, ps.rows, o.page_size, "paged K / V resource (within its page)");
        }
      } else {
        inside(sp.row0, sp.bytes / RB, P.Skv, "fwd K / V tile resource (within its head)");
        inside(head_kv + sp.row0, sp.bytes / RB, kv_rows, "fwd K / V tile resource");
      }
    }
  }
}

// ---- dQ (dq_bf16_kernel) ---------------------------------------------------
template <int D, int BN, int NW>
static void model_dq(const Problem& P, bool fuse) {
  constexpr int BM = 32 * NW, RB = D * 2, KSTEPS = D / 16, DT = D / 32, NSUB = BN / 32, TILE = BN * RB;
  constexpr int IPW = TILE / 1024 / NW;
  constexpr int LDS = 4 * TILE;
  for (int w = 0; w < NW; ++w)
    for (int lane = 0; lane < 64; ++lane) {
      for (int u = 0; u < IPW; ++u) {
        inside(tile_dma_offset<D, BN, NW>(lane, w, u), 16, TILE, "dQ K / V copy source");
        for (int t = 0; t < 4; ++t) inside(t * TILE + (w * IPW + u) * 1024 + 16 * lane, 16, LDS, "dQ copy into LDS");
      }
      RowTileOffsets<D> rt;
      rt.init(lane);
      for (int s = 0; s < KSTEPS; ++s)
        for (int j = 0; j < NSUB; ++j) inside(j * 32 * RB + rt.aoff[s], 16, TILE, "dQ K / V operand read");
      for (int dt = 0; dt < DT; ++dt)
        for (int c = 0; c < 2 * NSUB; ++c)
          for (int rd = 0; rd < 2; ++rd) inside(rt.tr[rd][dt] + 16 * c * RB, 8, TILE, "dQ K^T read");
      inside(w * 32 * RB, 32 * RB, LDS, "dQ staging");
    }
  const int nqt = (P.Sq + BM - 1) / BM;
  const int grid = dq_grid(P, BM);
  const long long q_rows = (long long)P.B * P.Hq * P.Sq, kv_rows = (long long)P.B * P.Hkv * P.Skv;
  for (int bid = 0; bid < grid; ++bid) {
    int head, qt;
    work_item(bid, P.B * P.Hq, nqt, P.xcd_remap, P.head_group_q, false, &head, &qt);
    inside(head, 1, P.B * P.Hq, "dQ work item head");
    const int b = head / P.Hq, h = head - b * P.Hq, hk = h / (P.Hq / P.Hkv);
    const int q0 = qt * BM;
    inside((long long)head * P.Sq, P.Sq, q_rows, fuse ? "dQ Q / dO / O resource" : "dQ Q / dO resource");
    for (int w = 0; w < NW; ++w)
      for (int lane = 0; lane < 64; ++lane) {
        const int qw = q0 + 32 * w + (lane & 31);
        int klo, khi;
        key_interval(P, b, qw, &klo, &khi);
        if (qw < P.Sq) inside((long long)head * P.Sq + qw, 1, q_rows, fuse ? "dQ LSE read / Delta write" : "dQ LSE, Delta read");
      }
    for (int w = 0; w < NW; ++w)
      for (int rr = 0; rr < 32 && rr < P.Sq - (q0 + 32 * w); ++rr)
        inside(((long long)head * P.Sq + q0 + 32 * w + rr) * D, D, q_rows * D, "dQ store");
    KvWalkT<HostLoad> walk;
    walk.bn = BN;
    walk.mblk = P.mblk_kv;
    walk.sub = P.mblk_kv / BN;
    walk.nblk = P.n_kvblk;
    walk.dense = !P.has_tables;
    walk.ntiles_dense = (P.Skv + BN - 1) / BN;
    walk.dense_masked = P.has_mask;
    walk.full = walk.part = nullptr;
    walk.nfull = walk.npart = 0;
    if (P.has_tables) {
      const int row = tab_row(P, b, h, q0 / P.mblk_q, P.n_qblk);
      if (P.full_kv_num) {
        walk.nfull = clamp_count(HostLoad::scalar(P.full_kv_num, row), P.kv_width);
        walk.full = P.full_kv_idx + (long long)row * P.kv_width;
      }
      if (P.kv_num) {
        walk.npart = clamp_count(HostLoad::scalar(P.kv_num, row), P.kv_width);
        walk.part = P.kv_idx + (long long)row * P.kv_width;
      }
    }
    const long long head_kv = (long long)(b * P.Hkv + hk) * P.Skv;
    for (int it = 0; it < walk.count(); ++it) {
      const RowSpan sp = row_span(walk.kbase(walk.fetch(it)), P.Skv, RB);
      inside(sp.row0, sp.bytes / RB, P.Skv, "dQ K / V tile resource (within its head)");
      inside(head_kv + sp.row0, sp.bytes / RB, kv_rows, "dQ K / V tile resource");
    }
  }
}

// ---- dK / dV (dkdv_bf16_kernel) --------------------------------------------
template <int D, int BQ, int NW>
static void model_dkdv(const Problem& P) {
  constexpr int BKV = 32 * NW, RB = D * 2, KSTEPS = D / 16, DT = D / 32, NQS = BQ / 32, TILE = BQ * RB;
  constexpr int IPW = TILE / 1024 / NW, STAT = 1024, NST = BQ / 64;
  constexpr int LDS = 4 * TILE + 4 * STAT;
  for (int w = 0; w < NW; ++w)
    for (int lane = 0; lane < 64; ++lane) {
      for (int u = 0; u < IPW; ++u) {
        inside(tile_dma_offset<D, BQ, NW>(lane, w, u), 16, TILE, "dK/dV Q / dO copy source");
        for (int t = 0; t < 4; ++t) inside(t * TILE + (w * IPW + u) * 1024 + 16 * lane, 16, LDS, "dK/dV copy into LDS");
      }
      for (int x = 0; x < 4; ++x)  // LSE / Delta landing zones (both buffers)
        for (int r = 0; r < NST; ++r) inside(4 * TILE + x * STAT + (64 * r + lane) * 4, 4, LDS, "dK/dV statistics store");
      RowTileOffsets<D> rt;
      rt.init(lane);
      const int hh = lane >> 5;
      for (int J = 0; J < NQS; ++J) {
        for (int s = 0; s < KSTEPS; ++s) inside(J * 32 * RB + rt.aoff[s], 16, TILE, "dK/dV Q / dO operand read");
        for (int q = 0; q < 4; ++q) inside((32 * J + acc_row(4 * q, hh)) * 4, 16, STAT, "dK/dV LSE / Delta read");
      }
      for (int dt = 0; dt < DT; ++dt)
        for (int c = 0; c < 2 * NQS; ++c)
          for (int rd = 0; rd < 2; ++rd) inside(rt.tr[rd][dt] + 16 * c * RB, 8, TILE, "dK/dV Q^T / dO^T read");
      inside(w * 2 * 32 * RB, 2 * 32 * RB, LDS, "dK/dV staging");
    }
  const int g = P.Hq / P.Hkv;
  const int nkt = (P.Skv + BKV - 1) / BKV;
  const int grid = dkdv_grid(P, BKV);
  const long long q_rows = (long long)P.B * P.Hq * P.Sq, kv_rows = (long long)P.B * P.Hkv * P.Skv;
  for (int bid = 0; bid < grid; ++bid) {
    int head, kt;
    work_item(bid, P.B * P.Hkv, nkt, P.xcd_remap, P.head_group_kv, true, &head, &kt);
    inside(head, 1, P.B * P.Hkv, "dK/dV work item head");
    const int b = head / P.Hkv, hk = head - b * P.Hkv;
    const int k0 = kt * BKV;
    // the first tile's entries, requested before the counts
    if (P.has_tables && (P.tab_h == 1 || g == 1)) {
      const int row = tab_row(P, b, hk * g, k0 / P.mblk_kv, P.n_kvblk);
      if (P.full_q_num) HostLoad::vector(P.full_q_idx + (long long)row * P.q_width, 0, P.q_width);
      if (P.q_num) HostLoad::vector(P.q_idx + (long long)row * P.q_width, 0, P.q_width);
    }
    inside((long long)head * P.Skv, P.Skv, kv_rows, "dK/dV K / V resource");
    for (int w = 0; w < NW; ++w)
      for (int lane = 0; lane < 64; ++lane) {
        int qlo, qhi;
        query_interval(P, b, k0 + 32 * w + (lane & 31), &qlo, &qhi);
      }
    for (int w = 0; w < NW; ++w)
      for (int rr = 0; rr < 32 && rr < P.Skv - (k0 + 32 * w); ++rr)
        inside(((long long)head * P.Skv + k0 + 32 * w + rr) * D, D, kv_rows * D, "dK / dV store");
    QWalkT<HostLoad> walk;
    walk.P = &P;
    walk.b = b;
    walk.hq0 = hk * g;
    walk.g = g;
    walk.kvrow = k0 / P.mblk_kv;
    walk.sub = P.mblk_q / BQ;
    walk.bq = BQ;
    walk.dense = !P.has_tables;
    walk.ntiles_dense = (P.Sq + BQ - 1) / BQ;
    walk.init();
    const int n_it = walk.count();
    for (int it = 0; it < n_it; ++it) {
      const TileRef r = walk.fetch(it);
      inside(r.hq, 1, P.Hq, "dK/dV q head of a tile");
      const int qb = walk.qbase(r);
      const long long hoff = (long long)(b * P.Hq + r.hq) * P.Sq;
      const RowSpan sp = row_span(qb, P.Sq, RB);
      inside(sp.row0, sp.bytes / RB, P.Sq, "dK/dV Q / dO tile resource (within its head)");
      inside(hoff + sp.row0, sp.bytes / RB, q_rows, "dK/dV Q / dO tile resource");
      const int q = qb < P.Sq ? qb : P.Sq;
      inside(q, P.Sq - q, P.Sq, "dK/dV LSE / Delta resource (within its head)");
      inside(hoff + q, P.Sq - q, q_rows, "dK/dV LSE / Delta resource");
    }
    // the copy issued during the last tile targets qb = Sq (zeros)
    const RowSpan z = row_span(P.Sq, P.Sq, RB);
    if (z.bytes != 0) fail("past-the-end copy reads rows");
  }
}

// ---- dispatch on the tiles problem.h chose --------------------------------
template <int D>
static void run_fwd(const Problem& P, const Tiles& t, const FwdOpts& o) {
  if constexpr (D >= 64) {
    if (t.bn == 32) return t.ns == 3 ? model_fwd<D, 32, 4, 3>(P, o) : model_fwd<D, 32, 4, 2>(P, o);
    if (t.bn == 128) return t.ns == 1 ? model_fwd<D, 128, 4, 1>(P, o) : model_fwd<D, 128, 4, 2>(P, o);
    if (t.bm == 256) return model_fwd<D, 64, 8, 2>(P, o);
  }
  if (t.bm == 64) return model_fwd<D, 64, 2, 2>(P, o);
  model_fwd<D, 64, 4, 2>(P, o);
}

template <int D>
static void run_bwd(const Problem& P, const Tiles& t) {
  if constexpr (D >= 64) {
    if (t.bn == 32) model_dq<D, 32, 4>(P, true);
    else if (t.bn == 128) model_dq<D, 128, 4>(P, true);
    else if (t.bm == 256) model_dq<D, 64, 8>(P, true);
    else if (t.bm == 64) model_dq<D, 64, 2>(P, true);
    else model_dq<D, 64, 4>(P, true);
    if (t.bkv == 64) return model_dkdv<D, 64, 2>(P);
    if (t.bq == 128) return model_dkdv<D, 128, 4>(P);
  } else {
    if (t.bm == 64) model_dq<D, 64, 2>(P, true);
    else model_dq<D, 64, 4>(P, true);
  }
  model_dkdv<D, 64, 4>(P);
}

static const int kTileSets[][5] = {  // bm, bn, bkv, bq, stages (0: automatic)
    {0, 0, 0, 0, 0},      {64, 64, 128, 0, 0},  {128, 32, 128, 0, 0}, {128, 32, 128, 0, 3},
    {128, 128, 128, 0, 0}, {128, 128, 128, 0, 1}, {256, 64, 128, 0, 0}, {128, 64, 64, 0, 0},
    {128, 64, 128, 64, 0}, {128, 64, 128, 128, 0}};

static int check_case(Case& c) {
  int launches = 0;
  // large problems: the default tiles, 32-key three-stage tiles and 64-query
  // dK/dV tiles; small ones: every tile set
  const int pick[] = {0, 3, 8};
  const int n = c.all_tiles ? (int)(sizeof(kTileSets) / sizeof(kTileSets[0])) : 3;
  for (int i = 0; i < n; ++i) {
    const int* ts = kTileSets[c.all_tiles ? i : pick[i]];
    fa_params p = c.p;
    p.block_m = ts[0];
    p.block_n = ts[1];
    p.block_kv = ts[2];
    p.block_q = ts[3];
    p.lds_stages = ts[4];
    Tiles t;
    if (default_tiles(&p, &t) != FA_OK) continue;  // no instantiation for this head dim
    if (t.bq == 128 && c.D < 64) continue;
    Problem P;
    std::memset(&P, 0, sizeof(P));
    if (build_problem(&p, t, &P) != FA_OK) continue;
    if (P.has_tables && (P.mblk_q % t.bm || P.mblk_kv % t.bn)) continue;  // refused by the C ABI
    FwdOpts o;
    g_where = "forward";
    if (c.D == 32) run_fwd<32>(P, t, o); else if (c.D == 64) run_fwd<64>(P, t, o); else run_fwd<128>(P, t, o);
    ++launches;
    // split-KV and GQA packing as the C ABI would choose them (a 256-CU device)
    if (t.bm == 128 && t.bn == 64 && t.ns == 2) {
      o.pack = choose_pack(&p, t, P);
      o.n_splits = choose_splits(&p, t, P, 0, 256);
      g_where = "split-KV forward";
      if (c.D == 32) run_fwd<32>(P, t, o); else if (c.D == 64) run_fwd<64>(P, t, o); else run_fwd<128>(P, t, o);
      ++launches;
    }
    if (dkdv_query_tile(&p, P, &t) != FA_OK) continue;
    if (P.has_tables && (P.mblk_kv % t.bkv || P.mblk_q % t.bq)) continue;
    g_where = "backward";
    if (c.D == 32) run_bwd<32>(P, t); else if (c.D == 64) run_bwd<64>(P, t); else run_bwd<128>(P, t);
    ++launches;
  }
  return launches;
}

// Paged decode: one query row per (batch, q head) against a KV cache of
// shuffled pages and per-batch lengths, split and GQA-packed as fa_fwd_kvcache
// runs it.
static int check_paged(const Case& c) {
  const int B = c.B, Hq = c.Hq, Hkv = c.Hkv, Skv = c.Skv, ps = c.page_size, maxp = c.max_pages;
  fa_params p;
  std::memset(&p, 0, sizeof(p));
  p.abi_version = FA_ABI_VERSION;
  p.dtype = FA_DTYPE_BF16;
  p.B = B; p.Hq = Hq; p.Hkv = Hkv; p.Sq = c.Sq; p.Skv = Skv; p.D = c.D;
  p.window_left = p.window_right = -1;
  std::vector<int> pt_host((size_t)B * maxp), lens_host(B);
  unsigned s = 12345u;
  for (int i = 0; i < B * maxp; ++i) {
    s = s * 1664525u + 1013904223u;
    pt_host[i] = (int)((s >> 8) % (unsigned)(c.num_pages + 2)) - 1;  // includes -1 and num_pages: read as zeros
  }
  for (int b = 0; b < B; ++b) lens_host[b] = (b * 7919) % (Skv + 1);
  int* pt = static_cast<int*>(std::malloc(sizeof(int) * pt_host.size()));
  int* lens = static_cast<int*>(std::malloc(sizeof(int) * B));
  std::memcpy(pt, pt_host.data(), sizeof(int) * pt_host.size());
  std::memcpy(lens, lens_host.data(), sizeof(int) * B);
  g_arrays.push_back({pt, (long long)pt_host.size()});
  g_arrays.push_back({lens, (long long)B});
  Tiles t;
  if (default_tiles(&p, &t) != FA_OK) return 0;
  Problem P;
  std::memset(&P, 0, sizeof(P));
  if (build_problem(&p, t, &P) != FA_OK) return 0;
  FwdOpts o;
  o.pack = choose_pack(&p, t, P);
  o.n_splits = choose_splits(&p, t, P, 0, 256);
  o.page_table = pt;
  o.page_size = ps;
  o.max_pages = maxp;
  o.num_pages = c.num_pages;
  o.kv_lens = lens;
  g_where = "paged split-KV forward";
  if (c.D == 64) run_fwd<64>(P, t, o); else run_fwd<128>(P, t, o);
  g_arrays.pop_back();
  g_arrays.pop_back();
  std::free(pt);
  std::free(lens);
  return 1;
}

int main(int argc, char** argv) {
  if (argc < 2) {
    std::fprintf(stderr, "usage: %s cases.bin\n", argv[0]);
    return 2;
  }
  FILE* f = std::fopen(argv[1], "rb");
  if (!f) return 2;
  int cases = 0, launches = 0;
  for (;;) {
    Case c;
    if (!read_case(f, c)) break;
    launches += c.paged ? check_paged(c) : check_case(c);
    ++cases;
    for (int* a : c.owned) std::free(a);
    g_arrays.clear();
  }
  std::fclose(f);
  std::printf("ok %d %d %lld\n", cases, launches, g_checks);
  return 0;
}
