// bf16 forward FlexAttention kernel for gfx950 (the main forward path).
//
// Work item: (batch, q head, BM = 32*NW query rows) -- or, with GQA row
// packing, (batch, kv head, BM of the group's g * Sq rows); wave w owns rows
// q0 + 32w .. +31 for the whole kv walk.
//
// Per kv tile of BN keys (double-buffered in LDS, one barrier per tile):
//   * K and V tiles are copied HBM -> LDS with buffer_load ... lds (no
//     registers, no bounds branches: rows past the sequence read as zero),
//     issued one tile ahead and spread over the S phase; the block-table row
//     sits in a register (KvTab), so tiles make no table loads;
//   * S^T = K Q^T   (A = K rows from LDS in perm23 order, fetched two k-steps
//     ahead of the MFMAs; B = Q from VGPRs);
//   * online softmax with one query per lane, speculative: exponentials
//     against the current reference maximum, no per-tile maximum; only a lane
//     whose tile sum leaves [0, 2^16] sends the wave through the exact
//     maximum / rescale (see softmax below); the scale is folded into the
//     exponent's FMA; fully-live tiles skip the element mask, partial tiles
//     keep keys in [lo, hi] (window and contiguous documents are intervals
//     per query);
//   * O^T += V^T P^T (A = V^T fetched from the row-major V tile with
//     ds_read_b64_tr_b16, B = P^T straight from the S^T accumulators).
// LDS layouts (row = key, 16-byte chunks): K chunk c of row r sits in slot
// c ^ chunk_swz(r) — each 16 lanes of an A-operand load hit 16 distinct bank
// slots; V chunk c sits in slot c ^ tr_swz(r) — the 4 consecutive rows of one
// transposing read land in distinct quarter-rows.
#pragma once
#include "dma.h"
#include "fwd.h"

#ifndef FA_FWD_PRIO
#define FA_FWD_PRIO 1
#endif
#ifndef FA_FWD_OREG
#define FA_FWD_OREG 'v'
#endif

namespace fa {

// kCache: the KV-cache variant (GQA row packing, paged K / V, per-batch key
// counts).  Kept out of the plain variant: its per-tile address logic costs
// the training-shape forward 7 % even when unused (measured A/B).
// Waves per SIMD: three for 32-key tiles (32 KiB of LDS; 168 registers, 8 %
// faster than two at S = 8192, measured), two otherwise.
// NS: K / V tiles in LDS at once (the tuner's stage axis).  2: double
// buffering, the next tile copied during the current one; 3: copies two tiles
// ahead (32-key tiles: 48 KiB, still three workgroups per CU); 1: a single
// buffer, the next K tile copied once every wave has left the S phase and the
// next V tile after the PV phase (128-key tiles: 64 KiB, two workgroups per CU
// instead of one).
template <int D, int BN, int NW, bool kMods, class Mod = BuiltinMod, bool kCache = false, int NS = 2>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(
    occupancy_for(2 * NS * BN * D * 2, NW, BN == 32 ? 3 : 2))))
void fwd_bf16_kernel(FwdArgs a) {
  using E = Elt<uint16_t>;
  using frag = E::frag;
  constexpr int BM = 32 * NW;
  constexpr int RB = D * 2;             // bytes per row
  constexpr int KCH = D / 8;            // 16-byte chunks per row
  constexpr int KSTEPS = D / 16;
  constexpr int NSUB = BN / 32;
  constexpr int DT = D / 32;
  constexpr int TILE = BN * RB;         // bytes per K (or V) tile
  constexpr int IPW = TILE / 1024 / NW; // DMA instructions per wave per tile
  static_assert(KCH >= 4 && D % 32 == 0 && BN % 32 == 0, "tile shape");
  static_assert(TILE % (1024 * NW) == 0, "DMA split");
  static_assert(NS >= 1 && NS <= 3 && (!kCache || NS == 2), "LDS stages");
  static_assert(2 * NS * BN >= BM, "O rows staged through the K / V buffers");

  __shared__ __attribute__((aligned(1024))) char lds[2 * NS * TILE];  // K_0 .. K_{NS-1}, V_0 .. V_{NS-1}

  const Problem& P = a.p;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 31, hh = lane >> 5;
  // A work item's rows: Sq queries of one q head, or with GQA packing the
  // g * Sq rows of a kv head's q heads (contiguous in memory).
  const int g = P.Hq / P.Hkv;
  const bool pack = kCache && a.pack > 1;
  const int rows = pack ? g * P.Sq : P.Sq;
  const int nheads = pack ? P.B * P.Hkv : P.B * P.Hq;
  const int nqt = (rows + BM - 1) / BM;
  const int n_items = nheads * nqt;
  const int split = a.n_splits > 1 ? (int)blockIdx.x / n_items : 0;
  int head, qt;
  work_item((int)blockIdx.x - split * n_items, nheads, nqt, P.xcd_remap, pack ? 1 : P.head_group_q, false, &head,
            &qt);
  const int b = head / (pack ? P.Hkv : P.Hq);
  const int hk = pack ? head - b * P.Hkv : (head - b * P.Hq) / g;
  const size_t row0 = pack ? (size_t)(b * P.Hq + hk * g) * P.Sq : (size_t)head * P.Sq;  // first row in memory
  const int q0 = qt * BM;
  const int rw = q0 + 32 * w + lr;  // this lane's row of the work item
  const bool qvalid = rw < rows;
  const int qw = pack ? rw % P.Sq : rw;  // query position
  // q head: wave-uniform hu (the group's first head when packed) for the
  // block-table walk, which must stay scalar; h per lane for score / mask mods
  const int hu = pack ? hk * g : head - b * P.Hq;
  const int h = pack ? hu + rw / P.Sq : hu;
  // keys of this batch row
  // (through the scalar cache: the loop bounds and every tile address derive
  // from it and must stay wave-uniform scalars)
  const int skv = (kCache && a.kv_lens) ? max(0, min(scalar_load(a.kv_lens, b), P.Skv)) : P.Skv;

  const char* kbase_ptr = static_cast<const char*>(a.k) + (size_t)(b * P.Hkv + hk) * P.Skv * RB;
  const char* vbase_ptr = static_cast<const char*>(a.v) + (size_t)(b * P.Hkv + hk) * P.Skv * RB;

  // Q rows as B operands (rows past the sequence read as zero)
  frag qf[KSTEPS];
  {
    const i32x4 rq = make_rsrc(static_cast<const char*>(a.q) + row0 * RB, (uint32_t)rows * RB);
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) qf[s] = buf_load16(rq, rw * RB + (2 * s + hh) * 16);
  }
  const float slope = P.alibi ? P.alibi[h] : 0.f;
  const float cap_inv = P.softcap > 0.f ? 1.0f / P.softcap : 0.f;
  // every mask term is an interval of keys per query (the host routes
  // arbitrary document labels to the generic kernel)
  int klo, khi;
  key_interval(P, b, qw, &klo, &khi);
  khi = min(khi, skv - 1);

  // loop-invariant LDS / global offsets (index.h)
  int dma_off_k[IPW], dma_off_v[IPW];
#pragma unroll
  for (int u = 0; u < IPW; ++u) {
    dma_off_k[u] = tile_dma_offset<D, BN, NW>(lane, w, u);
    dma_off_v[u] = tile_dma_offset<D, BN, NW, true>(lane, w, u);
  }
  RowTileOffsets<D> kt;  // K read as A operand rows (aoff)
  kt.init(lane);
  const int* koffA = kt.aoff;
  // transposing reads of V: rows row + 16c (+4 for the upper half of the
  // fragment), chunk 4i + x of d tile i
  int voffT[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) voffT[i] = fwd_voff_t<D>(lane, i);

  KvWalk walk;
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
    // packed rows share table row 0 of their batch row (the host packs only
    // with tables broadcast over heads and Sq within one mask block)
    const int row = tab_row(P, b, hu, pack ? 0 : q0 / P.mblk_q, P.n_qblk);
    if (P.full_kv_num) {
      walk.nfull = clamp_count(scalar_load(P.full_kv_num, row), P.kv_width);
      walk.full = P.full_kv_idx + (size_t)row * P.kv_width;
    }
    if (P.kv_num) {
      walk.npart = clamp_count(scalar_load(P.kv_num, row), P.kv_width);
      walk.part = P.kv_idx + (size_t)row * P.kv_width;
    }
  }
  const int n_it = walk.count();

  // HBM -> LDS copies of the tile starting at key kb into buffer `buf`: the
  // resources (issue_plan), then the 2 * IPW copy instructions one at a time
  // (issue_one).  Inside the walk they are spread over the S phase's k steps:
  // issued back to back, the four waves' copies queue at the texture unit for
  // hundreds of cycles (1.5 % of the forward at S = 8192, measured).
  struct Copy { i32x4 rk, rv; char* kl; char* vl; };
  auto issue_plan = [&](int kb, int buf) {
    const RowSpan sp = row_span(kb, skv, RB);
    kb = sp.row0;
    const char* kp = kbase_ptr + (size_t)kb * RB;
    const char* vp = vbase_ptr + (size_t)kb * RB;
    uint32_t range = sp.bytes;
    if (kCache && a.page_table) {  // the tile lies inside one page (page_size is a multiple of BN)
      // a bad page id reads zeros (index.h: page_span)
      const int pg = kb / a.page_size;
      const int phys = kb < skv ? scalar_load(a.page_table + (size_t)b * a.max_pages, pg) : -1;
      const PageSpan ps = page_span(kb, pg, skv, a.page_size, phys, a.num_pages, P.Hkv, hk);
      kp = static_cast<const char*>(a.k) + ps.row * RB;
      vp = static_cast<const char*>(a.v) + ps.row * RB;
      range = (uint32_t)ps.rows * RB;
    }
    Copy c;
    c.rk = make_rsrc(kp, range);
    c.rv = make_rsrc(vp, range);
    c.kl = lds + buf * TILE;
    c.vl = lds + (NS + buf) * TILE;
    return c;
  };
  auto issue_one = [&](const Copy& c, int i) {
    if (i < IPW) dma16(c.rk, dma_off_k[i], c.kl + (w * IPW + i) * 1024, i == 0);
    else dma16(c.rv, dma_off_v[i - IPW], c.vl + (w * IPW + i - IPW) * 1024, i == IPW);
  };
  auto issue = [&](int kb, int buf) {
    const Copy c = issue_plan(kb, buf);
#pragma unroll
    for (int u = 0; u < 2 * IPW; ++u) issue_one(c, u);
  };

  f32x16 oacc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[i][e] = 0.f;
#pragma unroll
  for (int i = 0; i < DT; ++i) mfma_drain<FA_FWD_OREG>(oacc[i]);
  // Reference maximum m (log2 units, per row) and partial sum l.  The
  // exponentials of a tile are taken speculatively against the current m,
  // with no maximum over the tile: P = exp2(t - m) goes straight into the
  // bf16 fragments of the PV product and its float32 row sum into l (the
  // unrounded P, as the reference sums it before the bf16 cast of PV).
  // As long as a lane's sum over the tile stays within kSpill = 2^16
  // (no P above 2^16: bf16 keeps its relative precision and the fp32 O and l
  // stay far from overflow), the tile is done.  Otherwise (a row maximum grew
  // by more than 16 in log2 units, a row's first live tile, or inf / NaN) the
  // whole wave takes the exact path: row maximum, O and l rescaled to it, and
  // the exponentials recomputed.  The normalisation O / l does not depend on
  // which reference is used.
  constexpr float kSpill = 65536.0f;
  float m = -INFINITY, l = 0.f;

  // Exponentials of a whole tile against reference muse, into the bf16
  // fragments pf; returns the lane's float32 sum.  Without score mods sacc
  // keeps raw (masked) q.k: the max is taken on it (scale > 0) and the scale
  // is folded into the exponent's FMA.  With mods sacc holds y with the
  // log2-domain logit ea * y + eb: the logit itself (ea = 1, eb = 0), or with
  // the built-in soft-cap r = 1 / (2^(2 s log2(e) / cap) + 1), whose logit is
  // cap log2(e) tanh(s / cap) = cap log2(e) (1 - 2 r) (ea = -2 cap log2(e),
  // eb = cap log2(e)): the exponent is one FMA either way.  Masked elements
  // hold the y whose logit is -inf (-inf, or +inf for r).
  const bool rform = kMods && !Mod::kScore && P.softcap > 0.f;
  const float ea = rform ? -2.0f * P.softcap * kLog2e : 1.0f;
  const float eb = rform ? P.softcap * kLog2e : 0.0f;
  auto exps = [&](const f32x16* sacc, frag* pf, float muse) {
    float rs0 = 0.f, rs1 = 0.f;
#pragma unroll
    for (int c = 0; c < BN / 16; ++c) {
      float x[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const float s = sacc[c >> 1][8 * (c & 1) + t];
        if constexpr (kMods) x[t] = fast_exp2(fmaf(s, ea, eb - muse));
        else x[t] = fast_exp2(fmaf(s, P.scale_log2, -muse));
      }
      pf[c] = E::pack(x);
#pragma unroll
      for (int t = 0; t < 8; t += 2) {
        rs0 += x[t];
        rs1 += x[t + 1];
      }
    }
    return rs0 + rs1;
  };
  auto softmax = [&](const f32x16* sacc, frag* pf) {
    float rs = exps(sacc, pf, m == -INFINITY ? 0.f : m);
    if (__any(!(rs <= kSpill) || m == -INFINITY)) {  // exact path (wave-uniform)
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < NSUB; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, kMods ? sacc[j][e] * ea : sacc[j][e]);
      float mt = pair_max(mx);
      if constexpr (!kMods) mt *= P.scale_log2;
      else mt += eb;
      const float mnew = fmaxf(m, mt);
      if (__any(mnew > m)) {
        const float alpha = fast_exp2(m - (mnew == -INFINITY ? 0.f : mnew));
        l *= alpha;
#pragma unroll
        for (int i = 0; i < DT; ++i) mfma_drain<FA_FWD_OREG>(oacc[i]);
#pragma unroll
        for (int i = 0; i < DT; ++i)
#pragma unroll
          for (int e = 0; e < 16; ++e) oacc[i][e] *= alpha;
#pragma unroll
        for (int i = 0; i < DT; ++i) mfma_drain<FA_FWD_OREG>(oacc[i]);
        m = mnew;
      }
      rs = exps(sacc, pf, m == -INFINITY ? 0.f : m);
    }
    l += rs;
  };

  // The walk's block indices come from a register (KvTab: 0.9 % at S = 8192,
  // measured against a table load per tile).
  // With split-KV this workgroup takes tiles [it0, it1) of the walk.
  const int n_full = walk.count_full();
  const int it0 = a.n_splits > 1 ? (int)((long long)n_it * split / a.n_splits) : 0;
  const int it1 = a.n_splits > 1 ? (int)((long long)n_it * (split + 1) / a.n_splits) : n_it;
  const int sub_log2 = log2_if_pow2(walk.sub);
  KvTab tab;
  auto kbase_of = [&](int it) { return tab.kbase(walk, it, sub_log2, lane); };
  // the first NS - 1 tiles (with one buffer, the first) copied ahead
  constexpr int AHEAD = NS > 1 ? NS - 1 : 1;
#pragma unroll
  for (int i = 0; i < AHEAD; ++i)
    if (it0 + i < it1) issue(kbase_of(it0 + i), i);
  // unconditional, so the wait-count analysis sees the register loads above
  // complete on every path into the loop
  wait_vmem();
  __syncthreads();
  // One tile; buf_c (the LDS buffer the tile sits in, tile it0 + i in buffer
  // i % NS) is a compile-time constant, so every LDS operand address is a
  // per-lane register plus an immediate offset (the loop below runs NS tiles
  // per iteration).
  auto tile_step = [&](int it, auto buf_c) {
    constexpr int buf = decltype(buf_c)::value;
    const int kbase = kbase_of(it);
    bool masked = it >= n_full;
    // the tile copied during this one: AHEAD tiles ahead, into the buffer
    // read last in the previous tile (NS = 1: the same buffer, in two halves)
    const bool more = it + AHEAD < it1;
    Copy nc;
    if (more) nc = issue_plan(kbase_of(it + AHEAD), (buf + AHEAD) % NS);
    if (NS > 1 && kbase >= skv && more) {
#pragma unroll
      for (int i = 0; i < 2 * IPW; ++i) issue_one(nc, i);
    }
    if (kbase < skv) {  // workgroup-uniform
      masked = masked || (kbase + BN > skv);
      const char* kl = lds + buf * TILE;
      const char* vl = lds + (NS + buf) * TILE;

      f32x16 sacc[NSUB];
#pragma unroll
      for (int j = 0; j < NSUB; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) sacc[j][e] = 0.f;
      // K fragments KPF k-steps ahead of their MFMAs (ds_read_b128 latency
      // exceeds one step of two MFMAs)
      constexpr int KPF = 2, KR = KPF + 1;
      frag ka[KR][NSUB];
      if (FA_FWD_PRIO) __builtin_amdgcn_s_setprio(1);  // MFMA phase first in issue order
#pragma unroll
      for (int s = 0; s < KPF; ++s)
#pragma unroll
        for (int j = 0; j < NSUB; ++j) ka[s][j] = *reinterpret_cast<const u32x4*>(kl + j * 32 * RB + koffA[s]);
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        if (s + KPF < KSTEPS) {
#pragma unroll
          for (int j = 0; j < NSUB; ++j)
            ka[(s + KPF) % KR][j] = *reinterpret_cast<const u32x4*>(kl + j * 32 * RB + koffA[s + KPF]);
        }
#pragma unroll
        for (int j = 0; j < NSUB; ++j) sacc[j] = E::mma(ka[s % KR][j], qf[s], sacc[j]);
        // this k step's share of the next tile's copies
        if constexpr (NS > 1) {
#pragma unroll
          for (int i = 0; i < 2 * IPW; ++i)
            if (i * KSTEPS / (2 * IPW) == s && more) issue_one(nc, i);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (FA_FWD_PRIO) __builtin_amdgcn_s_setprio(0);
      if constexpr (NS == 1) {
        // every wave is past its K reads: the next K tile goes into the buffer
        __syncthreads();
        if (more) {
#pragma unroll
          for (int i = 0; i < IPW; ++i) issue_one(nc, i);
        }
      }

      if constexpr (kMods && !Mod::kScore) {
        // built-in ALiBi + soft-cap: slope (k - q) = slope (base_j + c_e) with
        // base_j the lane's key offset of sub-tile j and c_e a constant, so
        // two FMAs per element; with the soft-cap (a wave-uniform branch) the
        // tanh's factor 2 log2(e) / cap is folded into those FMAs and the
        // tile keeps r = 1 / (2^t + 1) (see exps): one exp2, one add, one rcp
        const float c2 = 2.0f * kLog2e * cap_inv;
#pragma unroll
        for (int j = 0; j < NSUB; ++j) {
          const float sb = slope * (float)(kbase + 32 * j + 8 * hh - qw);
          if (P.softcap > 0.f) {
            const float a2 = P.scale * c2, sl2 = slope * c2, sb2 = sb * c2;
#pragma unroll
            for (int e = 0; e < 16; ++e)
              sacc[j][e] = fast_rcp(fast_exp2(fmaf(sacc[j][e], a2, fmaf(sl2, (float)acc_row(e, 0), sb2))) + 1.0f);
          } else {  // log2(e) folded in the same way
            const float al = P.scale * kLog2e, sll = slope * kLog2e, sbl = sb * kLog2e;
#pragma unroll
            for (int e = 0; e < 16; ++e) sacc[j][e] = fmaf(sacc[j][e], al, fmaf(sll, (float)acc_row(e, 0), sbl));
          }
        }
      } else if constexpr (kMods) {
#pragma unroll
        for (int j = 0; j < NSUB; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            float dsdx;  // unused in the forward
            sacc[j][e] = mod_score_flat<Mod>(P, sacc[j][e], slope, b, h, qw, kbase + 32 * j + acc_row(e, hh), cap_inv,
                                             &dsdx);
          }
      }
      if (masked) {  // partial tile: keys outside [klo, khi] are dropped
        const float dead = rform ? INFINITY : -INFINITY;  // the y whose logit is -inf
        // key kbase + c_e with c_e = 32 j + acc_row(e, hh): the bounds are
        // taken relative to the tile, so each element compares a constant
        const int lo = klo - kbase - 8 * hh, hi = khi - kbase - 8 * hh;
#pragma unroll
        for (int j = 0; j < NSUB; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int c = 32 * j + acc_row(e, 0);
            bool keep = c >= lo && c <= hi;
            if constexpr (Mod::kMask) keep = keep && Mod::mask(P, b, h, qw, kbase + c + 8 * hh);
            sacc[j][e] = keep ? sacc[j][e] : dead;
          }
      }
      // V^T fragments of d tile i (two tiles in flight): tile 0's reads issue
      // before the softmax, tile i + 1's before tile i's MFMAs
      frag vt[2][BN / 16];
      auto load_vt = [&](int i) {
#pragma unroll
        for (int c = 0; c < BN / 16; ++c) {
          const uint2 lo = lds_read_tr16(vl + voffT[i] + (16 * c) * RB);
          const uint2 hi = lds_read_tr16(vl + voffT[i] + (16 * c + 4) * RB);
          vt[i & 1][c] = u32x4{lo.x, lo.y, hi.x, hi.y};
        }
      };
      load_vt(0);
      frag pf[BN / 16];
      softmax(sacc, pf);
      // the 2 wait states an MFMA needs after a VALU write of its operand,
      // once for all of P (the PV MFMAs then carry no s_nop)
      static_assert(BN / 16 == 8 || BN / 16 == 4 || BN / 16 == 2, "P fragments");
      if constexpr (BN / 16 == 8)
        asm volatile("s_nop 1" : "+v"(pf[0]), "+v"(pf[1]), "+v"(pf[2]), "+v"(pf[3]), "+v"(pf[4]), "+v"(pf[5]),
                     "+v"(pf[6]), "+v"(pf[7]));
      else if constexpr (BN / 16 == 4)
        asm volatile("s_nop 1" : "+v"(pf[0]), "+v"(pf[1]), "+v"(pf[2]), "+v"(pf[3]));
      else
        asm volatile("s_nop 1" : "+v"(pf[0]), "+v"(pf[1]));
      if (FA_FWD_PRIO) __builtin_amdgcn_s_setprio(1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < DT; ++i) {
        if (i + 1 < DT) load_vt(i + 1);
#pragma unroll
        for (int c = 0; c < BN / 16; ++c) mfma_acc<FA_FWD_OREG, false>(oacc[i], vt[i & 1][c], pf[c]);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (FA_FWD_PRIO) __builtin_amdgcn_s_setprio(0);
    }
    if constexpr (NS == 1) {
      // every wave is past its V reads: the next V tile (and, for a tile
      // past the keys, the K tile not copied above), then wait for both
      __syncthreads();
      if (more) {
#pragma unroll
        for (int i = 0; i < 2 * IPW; ++i)
          if (i >= IPW || kbase >= skv) issue_one(nc, i);
      }
      wait_vmem();
    } else if constexpr (NS == 2) {
      wait_vmem();
    } else {
      // the next tile's copies (issued a tile earlier) are done once at most
      // this tile's 2 * IPW copies remain
      if (more) wait_vmem_but<2 * IPW>();
      else wait_vmem();
    }
    __syncthreads();
  };
  int it = it0;
  if constexpr (NS == 1) {
    for (; it < it1; ++it) tile_step(it, Int<0>{});
  } else if constexpr (NS == 2) {
    for (; it + 1 < it1; it += 2) {
      tile_step(it, Int<0>{});
      tile_step(it + 1, Int<1>{});
    }
    if (it < it1) tile_step(it, Int<0>{});
  } else {
    for (; it + 2 < it1; it += 3) {
      tile_step(it, Int<0>{});
      tile_step(it + 1, Int<1>{});
      tile_step(it + 2, Int<2>{});
    }
    if (it < it1) tile_step(it, Int<0>{});
    if (it + 1 < it1) tile_step(it + 1, Int<1>{});
  }

#pragma unroll
  for (int i = 0; i < DT; ++i) mfma_drain<FA_FWD_OREG>(oacc[i]);
  const float lt = pair_sum(l);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  if (a.n_splits > 1) {  // partial O (relative to 2^m) and (m, l) for the merge
    const size_t all_rows = (size_t)P.B * P.Hq * P.Sq;
    const size_t row = row0 + rw;
    if (qvalid) {
      float* po = a.part + ((size_t)split * all_rows + row) * D;
#pragma unroll
      for (int i = 0; i < DT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          *reinterpret_cast<f32x4*>(po + 32 * i + 8 * j + 4 * hh) =
              f32x4{oacc[i][4 * j], oacc[i][4 * j + 1], oacc[i][4 * j + 2], oacc[i][4 * j + 3]};
      if (hh == 0) {
        float* pml = a.part + (size_t)a.n_splits * all_rows * D + ((size_t)split * all_rows + row) * 2;
        *reinterpret_cast<float2*>(pml) = make_float2(m, lt);
      }
    }
    return;
  }
  // O rows of this wave, staged through the (now idle) K / V buffers
  store_rows_bf16<D>(oacc, inv, lds + w * (32 * RB),
                     static_cast<uint16_t*>(a.o) + (row0 + q0 + 32 * w) * D, rows - (q0 + 32 * w),
                     lane);
  if (qvalid && hh == 0) a.lse[row0 + rw] = lt > 0.f ? (m + log2f(lt)) * kLn2 : -INFINITY;
}

// Split-KV merge: one thread per (row, column) of O.  With the splits'
// partials O_s (relative to 2^m_s) and sums l_s: M = max m_s, L = sum l_s
// 2^(m_s - M), O = sum O_s 2^(m_s - M) / L, LSE = (M + log2 L) ln 2.
template <int D>
__global__ __launch_bounds__(256) void fwd_split_merge(FwdArgs a) {
  const Problem& P = a.p;
  const size_t rows = (size_t)P.B * P.Hq * P.Sq;
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t row = idx / D;
  const int d = (int)(idx - row * D);
  if (row >= rows) return;
  const float* pml = a.part + (size_t)a.n_splits * rows * D;
  float mm = -INFINITY;
  for (int s = 0; s < a.n_splits; ++s) mm = fmaxf(mm, pml[((size_t)s * rows + row) * 2]);
  float L = 0.f, O = 0.f;
  if (mm != -INFINITY) {
    for (int s = 0; s < a.n_splits; ++s) {
      const float ms = pml[((size_t)s * rows + row) * 2];
      const float c = ms == -INFINITY ? 0.f : fast_exp2(ms - mm);
      L += pml[((size_t)s * rows + row) * 2 + 1] * c;
      O += a.part[((size_t)s * rows + row) * D + d] * c;
    }
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  const uint32_t ob = pack_bf16x2(O * inv, 0.f);
  static_cast<uint16_t*>(a.o)[row * D + d] = (uint16_t)(ob & 0xffffu);
  if (d == 0) a.lse[row] = L > 0.f ? (mm + log2f(L)) * kLn2 : -INFINITY;
}

}  // namespace fa
