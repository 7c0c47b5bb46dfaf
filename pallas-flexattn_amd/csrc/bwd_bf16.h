// bf16 backward FlexAttention kernels for gfx950 (the main backward path).
//
// Both kernels stage row-major tiles (rows = keys or queries, D bf16 per row)
// in LDS with buffer_load ... lds, double-buffered one tile ahead, and read
// them two ways:
//   * as MFMA A operands "row r, eight consecutive d" (ds_read_b128, rows in
//     perm23 order so the fp32 results feed the next MFMA from registers);
//   * transposed, "column d, eight consecutive rows" (two ds_read_b64_tr_b16),
//     for the products that contract over the tile's rows (K^T in dQ, Q^T and
//     dO^T in dK/dV) — no transposed copy is ever written.
// Chunk c (16 bytes) of row r sits in slot c ^ chunk_swz(r), which keeps
// both access patterns free of bank conflicts.  Every MFMA phase fetches the
// operands of step k+1 before issuing the MFMAs of step k.
//
//   dq_bf16_kernel   (batch, q head, 32*NW queries): Q, dO rows in VGPRs;
//                    S^T = K Q^T, dP^T = V dO^T, dS^T = P^T (dP^T - Delta),
//                    dQ^T += K^T dS^T over the kv-side block tables.
//   dkdv_bf16_kernel (batch, kv head, 32*NW keys): K, V rows in VGPRs;
//                    S = Q K^T, dP = dO V^T, dV^T += dO^T P, dK^T += Q^T dS
//                    over the q-side tables of every q head of the GQA group,
//                    each q tile one hand-ordered step sequence.
// Partial tiles apply the element mask, an interval per lane (windows and
// contiguous documents; other document layouts use the generic kernels);
// full tiles skip it.
#pragma once
#include "bwd.h"
#include "dma.h"

#ifndef FA_DKDV_APF
#define FA_DKDV_APF 3  // measured: 2 -> 3 about 0.5 % faster at S = 8192, 4 no better
#endif

namespace fa {

// Lane-constant LDS offsets for reading a swizzled row-major bf16 tile
// (chunk c of row r in slot c ^ chunk_swz(r); offsets from index.h).
template <int D>
struct RowTile : RowTileOffsets<D> {
  using RowTileOffsets<D>::RB;
  using RowTileOffsets<D>::aoff;
  using RowTileOffsets<D>::tr;
  // A operand: rows 32*j + perm23(lane%32), d = 16*s + 8*(lane/32) + [0..7]
  __device__ __forceinline__ u32x4 a_frag(const char* tile, int j, int s) const {
    return *reinterpret_cast<const u32x4*>(tile + j * 32 * RB + aoff[s]);
  }
  // transposed A operand: row d = 32*dt + lane%32, k = tile rows 16*c + 8*(lane/32) + [0..7]
  // (the swizzle depends on r & 15 only, so rows +16c are a constant offset)
  __device__ __forceinline__ u32x4 t_frag(const char* tile, int dt, int c) const {
    const uint2 lo = lds_read_tr16(tile + tr[0][dt] + 16 * c * RB);
    const uint2 hi = lds_read_tr16(tile + tr[1][dt] + 16 * c * RB);
    return u32x4{lo.x, lo.y, hi.x, hi.y};
  }
};

// per-lane DMA source offsets for copying an R-row tile with NW waves
template <int D, int R, int NW>
struct TileDma {
  static constexpr int RB = D * 2;
  static constexpr int IPW = R * RB / 1024 / NW;
  static_assert((R * RB) % (1024 * NW) == 0, "DMA split");
  int off[IPW];
  __device__ __forceinline__ void init(int lane, int w) {
#pragma unroll
    for (int u = 0; u < IPW; ++u) off[u] = tile_dma_offset<D, R, NW>(lane, w, u);
  }
  // resource for rows [row0, row0 + R) of a tensor with `rows` rows at `base`
  // (rows past the end read as zero; row0 >= rows copies zeros)
  __device__ __forceinline__ static i32x4 rsrc(const char* base, int row0, int rows) {
    const RowSpan sp = row_span(row0, rows, RB);
    return make_rsrc(base + (size_t)sp.row0 * RB, sp.bytes);
  }
  // the u-th of this wave's IPW copy instructions (u a compile-time constant
  // after unrolling; u = 0 is the descriptor's first use)
  __device__ __forceinline__ void one(const i32x4& rs, int u, char* lds_tile, int w) const {
    dma16(rs, off[u], lds_tile + (w * IPW + u) * 1024, u == 0);
  }
  __device__ __forceinline__ void issue(const char* base, int row0, int rows, char* lds_tile, int w) const {
    const i32x4 rs = rsrc(base, row0, rows);
#pragma unroll
    for (int u = 0; u < IPW; ++u) one(rs, u, lds_tile, w);
  }
};

// acc += A(tileA rows 32j..) * bA[s]  and  acc2 += A(tileB rows 32j..) * bB[s]
// over all k steps, operands fetched PF steps ahead (one step is two MFMAs,
// 64 cycles; an LDS read under load takes longer than that).
struct NoHook {
  __device__ __forceinline__ void operator()(int) const {}
};
template <int D, int PF = 1, class Hook = NoHook>
__device__ __forceinline__ void mma_rows2(const RowTile<D>& rt, const char* ta, const char* tb, int j,
                                          const u32x4* ba, const u32x4* bb, f32x16& acc, f32x16& acc2,
                                          const Hook& hook = Hook()) {
  using E = Elt<uint16_t>;
  constexpr int KS = D / 16;
  constexpr int R = PF + 1;
  u32x4 fa[R], fb[R];
#pragma unroll
  for (int s = 0; s < PF && s < KS; ++s) {
    fa[s] = rt.a_frag(ta, j, s);
    fb[s] = rt.a_frag(tb, j, s);
  }
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    if (s + PF < KS) {
      fa[(s + PF) % R] = rt.a_frag(ta, j, s + PF);
      fb[(s + PF) % R] = rt.a_frag(tb, j, s + PF);
    }
    acc = E::mma(fa[s % R], ba[s], acc);
    acc2 = E::mma(fb[s % R], bb[s], acc2);
    hook(s);
  }
}

// Steps it = from .. to - 1 of a double-buffered tile walk, the buffer of
// step it being it & 1, passed as a compile-time constant so that LDS
// operand addresses fold into immediate offsets: steps run in pairs.
template <class Step, class Masked>
__device__ __forceinline__ void run_tiles(int from, int to, Step& step, Masked masked_c) {
  int it = from;
  if ((it & 1) && it < to) step(it++, masked_c, Bool<1>{});
  for (; it + 1 < to; it += 2) {
    step(it, masked_c, Bool<0>{});
    step(it + 1, masked_c, Bool<1>{});
  }
  if (it < to) step(it, masked_c, Bool<0>{});
}

__device__ __forceinline__ void zero(f32x16& x) {
#pragma unroll
  for (int e = 0; e < 16; ++e) x[e] = 0.f;
}

// ------------------------------------------------------------------- dQ ----
template <int D, int BN, int NW, bool kMods, class Mod = BuiltinMod>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(occupancy_for(4 * BN * D * 2, NW, 2))))
void dq_bf16_kernel(BwdArgs a) {
  using E = Elt<uint16_t>;
  using frag = E::frag;
  constexpr int BM = 32 * NW;
  constexpr int RB = D * 2;
  constexpr int KSTEPS = D / 16;
  constexpr int NSUB = BN / 32;
  constexpr int DT = D / 32;
  constexpr int NC = BN / 16;
  constexpr int TILE = BN * RB;
  static_assert(4 * BN >= BM, "dQ rows staged through the K / V buffers");
  __shared__ __attribute__((aligned(1024))) char lds[4 * TILE];  // K0 K1 V0 V1

  const Problem& P = a.p;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 31, hh = lane >> 5;
  const int nqt = (P.Sq + BM - 1) / BM;
  int head, qt;
  work_item(blockIdx.x, P.B * P.Hq, nqt, P.xcd_remap, P.head_group_q, false, &head, &qt);
  const int b = head / P.Hq, h = head - b * P.Hq;
  const int hk = h / (P.Hq / P.Hkv);
  const int q0 = qt * BM;
  const int qw = q0 + 32 * w + lr;
  const bool qvalid = qw < P.Sq;

  frag qf[KSTEPS], df[KSTEPS];
  frag of[KSTEPS];  // O rows, only with a.fuse_delta
  const bool fuse = a.fuse_delta != 0;
  {
    const i32x4 rq = make_rsrc(static_cast<const char*>(a.q) + (size_t)head * P.Sq * RB, (uint32_t)P.Sq * RB);
    const i32x4 rd = make_rsrc(static_cast<const char*>(a.dout) + (size_t)head * P.Sq * RB, (uint32_t)P.Sq * RB);
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      qf[s] = buf_load16(rq, qw * RB + (2 * s + hh) * 16);
      df[s] = buf_load16(rd, qw * RB + (2 * s + hh) * 16);
    }
    if (fuse) {
      const i32x4 ro = make_rsrc(static_cast<const char*>(a.o) + (size_t)head * P.Sq * RB, (uint32_t)P.Sq * RB);
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) of[s] = buf_load16(ro, qw * RB + (2 * s + hh) * 16);
    }
  }
  const size_t rowi = (size_t)head * P.Sq + qw;
  // a row with no live key (LSE = -inf) gets P = 0 everywhere, like rows past Sq
  const float lse_row = qvalid ? a.lse[rowi] : -INFINITY;
  const float lse2 = lse_row > -INFINITY ? lse_row * kLog2e : INFINITY;
  float dl = (!fuse && qvalid) ? a.delta[rowi] : 0.f;
  const float slope = P.alibi ? P.alibi[h] : 0.f;
  const float cap_inv = P.softcap > 0.f ? 1.0f / P.softcap : 0.f;
  // with mods a tile holds y with the log2-domain logit ea * y: the logit
  // itself, or with the built-in soft-cap tanh(s / cap) (ea = cap log2(e))
  const float ea = (kMods && !Mod::kScore && P.softcap > 0.f) ? P.softcap * kLog2e : 1.0f;
  int klo, khi;  // keys visible to this lane's query (masks are intervals here)
  key_interval(P, b, qw, &klo, &khi);

  const char* kbase_ptr = static_cast<const char*>(a.k) + (size_t)(b * P.Hkv + hk) * P.Skv * RB;
  const char* vbase_ptr = static_cast<const char*>(a.v) + (size_t)(b * P.Hkv + hk) * P.Skv * RB;
  RowTile<D> rt;
  rt.init(lane);
  TileDma<D, BN, NW> dma;
  dma.init(lane, w);

  KvWalk walk;
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
      walk.nfull = clamp_count(scalar_load(P.full_kv_num, row), P.kv_width);
      walk.full = P.full_kv_idx + (size_t)row * P.kv_width;
    }
    if (P.kv_num) {
      walk.npart = clamp_count(scalar_load(P.kv_num, row), P.kv_width);
      walk.part = P.kv_idx + (size_t)row * P.kv_width;
    }
  }
  const int n_it = walk.count();
  auto issue = [&](int kb, int buf) {
    dma.issue(kbase_ptr, kb, P.Skv, lds + buf * TILE, w);
    dma.issue(vbase_ptr, kb, P.Skv, lds + (2 + buf) * TILE, w);
  };

  f32x16 dqa[DT];  // accumulated in place
#pragma unroll
  for (int i = 0; i < DT; ++i) {
    zero(dqa[i]);
    mfma_drain<'v'>(dqa[i]);
  }

  // One kv tile: per 32-key sub-tile S^T, dP^T -> dS^T (packed), then that
  // sub-tile's share of dQ^T += K^T dS^T (K^T fragments one step ahead), so
  // the next sub-tile's MFMAs can overlap this one's exponentials.
  // A single code path for full and partial tiles: only the in-place masking
  // of S^T is conditional, so the loop-carried accumulators keep their
  // registers.
  auto tile = [&](int kbase, const char* kl, const char* vl, auto masked_c, auto&& copies) {
    constexpr bool kMasked = decltype(masked_c)::value;
    frag sf[2];
#pragma unroll
    for (int j = 0; j < NSUB; ++j) {
      f32x16 sacc, pacc;
      zero(sacc);
#pragma unroll
      for (int e = 0; e < 16; ++e) pacc[e] = dl;  // Delta - dP after the MFMAs (dO negated)
      // MFMA phases at raised wave priority, so the SIMD's other wave runs its
      // exponentials beside them (2.5 % at C2, measured)
      __builtin_amdgcn_s_setprio(1);
      if (j == 0) mma_rows2<D>(rt, kl, vl, j, qf, df, sacc, pacc, copies);
      else mma_rows2<D>(rt, kl, vl, j, qf, df, sacc, pacc);
      __builtin_amdgcn_s_setprio(0);
      float dsdx[16];
      if constexpr (kMods && !Mod::kScore) {
        // built-in ALiBi + soft-cap: slope (k - q) = sb + slope c_e, the
        // soft-cap's tanh as one exp2, one rcp and FMAs (wave-uniform branch)
        // with its factor 2 log2(e) / cap folded into the score FMAs; the
        // tile keeps tanh itself (the logit is ea tanh, see below)
        const float sb = slope * (float)(kbase + 32 * j + 8 * hh - qw);
        if (P.softcap > 0.f) {
          const float c2 = 2.0f * kLog2e * cap_inv;
          const float a2 = P.scale * c2, sl2 = slope * c2, sb2 = sb * c2;
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const float th =
                fmaf(-2.0f, fast_rcp(fast_exp2(fmaf(sacc[e], a2, fmaf(sl2, (float)acc_row(e, 0), sb2))) + 1.0f), 1.0f);
            sacc[e] = th;
            dsdx[e] = fmaf(-th, th, 1.0f);
          }
        } else {  // log2(e) folded in the same way
          const float al = P.scale * kLog2e, sll = slope * kLog2e, sbl = sb * kLog2e;
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            sacc[e] = fmaf(sacc[e], al, fmaf(sll, (float)acc_row(e, 0), sbl));
            dsdx[e] = 1.f;
          }
        }
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          dsdx[e] = 1.f;
          if constexpr (kMods)
            sacc[e] = mod_score_flat<Mod>(P, sacc[e], slope, b, h, qw, kbase + 32 * j + acc_row(e, hh), cap_inv,
                                      &dsdx[e]);
        }
      }
      if constexpr (kMasked) {
        // key kbase + 32 j + acc_row(e, hh), compared against tile-relative
        // bounds (a constant per element)
        const int lo = klo - kbase - 32 * j - 8 * hh, hi = khi - kbase - 32 * j - 8 * hh;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int c = acc_row(e, 0);
          bool keep = c >= lo && c <= hi;
          if constexpr (Mod::kMask) keep = keep && Mod::mask(P, b, h, qw, kbase + 32 * j + c + 8 * hh);
          sacc[e] = keep ? sacc[e] : -INFINITY;
        }
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float pv;
        if constexpr (kMods) pv = fast_exp2(fmaf(sacc[e], ea, -lse2));
        else pv = fast_exp2(fmaf(sacc[e], P.scale_log2, -lse2));
        if constexpr (kMods) pacc[e] = -pv * pacc[e] * dsdx[e];
        else pacc[e] = -pv * pacc[e];
      }
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        float y[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) y[t] = pacc[8 * half + t];
        sf[half] = E::pack(y);
      }
      // the 2 wait states an MFMA needs after a VALU write of its operand
      asm volatile("s_nop 1" : "+v"(sf[0]), "+v"(sf[1]));
      // x = (d tile, chunk half) of this sub-tile: chunk c = 2j + half
      frag kt[2];
      kt[0] = rt.t_frag(kl, 0, 2 * j);
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int x = 0; x < 2 * DT; ++x) {
        if (x + 1 < 2 * DT) kt[(x + 1) & 1] = rt.t_frag(kl, (x + 1) >> 1, 2 * j + ((x + 1) & 1));
        mfma_acc<'v', false>(dqa[x >> 1], kt[x & 1], sf[x & 1]);
      }
      __builtin_amdgcn_s_setprio(0);
    }
  };

  // Full tiles run first, in a loop of their own without the element mask;
  // the partial tiles follow.  Keys past Skv need no mask: their K and V rows
  // read as zero, so dS K^T gets nothing from them.
  // Table entries are fetched two tiles ahead, resolved one tile ahead.
  int kb_next = 0;
  TileRef ref_next{0, 0, 0};
  if (n_it > 0) {
    kb_next = walk.kbase(walk.fetch(0));
    issue(kb_next, 0);
    if (n_it > 1) ref_next = walk.fetch(1);
  }
  // unconditional, so the wait-count analysis sees the register loads above
  // complete on every path into the loop
  wait_vmem();
  __syncthreads();
  if (fuse) {
    // Delta = sum_d O dO of this lane's row (rows past Sq read as zero): the
    // lane holds 16-byte chunks 2 s + hh; they are summed pairwise at chunk
    // distances D/16, ..., 2 inside the lane and 1 across the lane pair, the
    // order of the Delta kernel's shuffle tree, so the rows are bit-identical
    float x[KSTEPS];
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) x[s] = chunk_dot_bf16(of[s], df[s]);
#pragma unroll
    for (int st = KSTEPS / 2; st >= 1; st >>= 1)
#pragma unroll
      for (int s = 0; s < st; ++s) x[s] = x[s] + x[s + st];
    dl = pair_sum(x[0]);
    if (qvalid && hh == 0) a.delta[rowi] = dl;
  }
  // dO is kept negated (bf16 sign flips), so the dP^T MFMA accumulates -dP
  // onto its starting value: started from Delta it gives Delta - dP, and
  // dS = -P (Delta - dP) takes one multiply per element
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s) df[s] ^= 0x80008000u;
  // (the buffer index is a compile-time constant, tiles run in pairs, so
  // LDS operand addresses fold into immediate offsets)
  // the next tile's copies are spread over the first sub-tile's k steps (as
  // in the forward: issued back to back they queue at the texture unit;
  // 0.7 % of this kernel at S = 8192, measured)
  constexpr int IPW = TileDma<D, BN, NW>::IPW;
  auto step = [&](int it, auto masked_c, auto buf_c) {
    constexpr int buf = decltype(buf_c)::value;  // == it & 1
    const int kbase = kb_next;
    const bool more = it + 1 < n_it;
    i32x4 rk = {0, 0, 0, 0}, rv = {0, 0, 0, 0};
    // the next tile's start and copy resources, and the table entry of the
    // tile after it: scalar work, run behind the tile's first MFMAs (before
    // them, the workgroup's waves would run it on the shared scalar unit at
    // once while their matrix cores wait)
    auto prep = [&]() {
      if (more) {
        kb_next = walk.kbase(ref_next);
        rk = TileDma<D, BN, NW>::rsrc(kbase_ptr, kb_next, P.Skv);
        rv = TileDma<D, BN, NW>::rsrc(vbase_ptr, kb_next, P.Skv);
      }
      if (it + 2 < n_it) ref_next = walk.fetch(it + 2);
    };
    char* nk = lds + (buf ^ 1) * TILE;
    char* nv = lds + (2 + (buf ^ 1)) * TILE;
    auto issue_copies = [&](int s) {
#pragma unroll
      for (int i = 0; i < 2 * IPW; ++i)
        if (i * KSTEPS / (2 * IPW) == s && more) {
          if (i < IPW) dma.one(rk, i, nk, w);
          else dma.one(rv, i - IPW, nv, w);
        }
    };
    auto copies = [&](int s) {
      if (s == 0) prep();
      issue_copies(s);
    };
    if (kbase < P.Skv) {
      tile(kbase, lds + buf * TILE, lds + (2 + buf) * TILE, masked_c, copies);
    } else {
      prep();
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) issue_copies(s);
    }
    wait_vmem();
    __syncthreads();
  };
  const int n_full = walk.count_full();
  run_tiles(0, n_full, step, False{});
  run_tiles(n_full, n_it, step, True{});

#pragma unroll
  for (int i = 0; i < DT; ++i) mfma_drain<'v'>(dqa[i]);
  // dQ rows of this wave, staged through the (now idle) tile buffers
  store_rows_bf16<D>(dqa, P.scale, lds + w * (32 * RB),
                     static_cast<uint16_t*>(a.dq) + ((size_t)head * P.Sq + q0 + 32 * w) * D, P.Sq - (q0 + 32 * w),
                     lane);
}

// ---------------------------------------------------------------- dK dV ----
template <int D, int BQ, int NW, bool kMods, class Mod = BuiltinMod>
__global__ __launch_bounds__(NW * 64) void dkdv_bf16_kernel(BwdArgs a) {
  using E = Elt<uint16_t>;
  using frag = E::frag;
  constexpr int BKV = 32 * NW;
  constexpr int RB = D * 2;
  constexpr int KSTEPS = D / 16;
  constexpr int NQS = BQ / 32;
  constexpr int DT = D / 32;
  constexpr int NC = BQ / 16;
  constexpr int TILE = BQ * RB;
  constexpr int STAT = 1024;  // LSE / Delta landing zone per buffer (BQ floats used)
  constexpr int APF = FA_DKDV_APF;  // operand prefetch depth (steps)
  static_assert(BQ * 4 <= STAT, "stat tile");
  __shared__ __attribute__((aligned(1024))) char lds[4 * TILE + 4 * STAT];  // Q0 Q1 dO0 dO1 L0 L1 D0 D1

  const Problem& P = a.p;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 31, hh = lane >> 5;
  const int nkt = (P.Skv + BKV - 1) / BKV;
  const int g = P.Hq / P.Hkv;
  int head, kt;
  work_item(blockIdx.x, P.B * P.Hkv, nkt, P.xcd_remap, P.head_group_kv, true, &head, &kt);
  const int b = head / P.Hkv, hk = head - b * P.Hkv;
  const int k0 = kt * BKV;
  const int kw = k0 + 32 * w + lr;
  const bool kvalid = kw < P.Skv;

  // The first tile's table entry is requested first of all (both lists'
  // first entries; rows hold q_width >= 1 entries), ahead of the K / V rows
  // and of the counts, so the first tile's copy waits for neither (valid when
  // the first tile comes from the first head's lists).
  const bool spec0 = P.has_tables && (P.tab_h == 1 || g == 1);
  int first_full = 0, first_part = 0;
  if (spec0) {
    const int row = tab_row(P, b, hk * g, k0 / P.mblk_kv, P.n_kvblk);
    if (P.full_q_num) first_full = vload_i32(P.full_q_idx + (size_t)row * P.q_width, 0, P.q_width);
    if (P.q_num) first_part = vload_i32(P.q_idx + (size_t)row * P.q_width, 0, P.q_width);
  }
  frag kf[KSTEPS], vf[KSTEPS];
  {
    const i32x4 rk = make_rsrc(static_cast<const char*>(a.k) + (size_t)head * P.Skv * RB, (uint32_t)P.Skv * RB);
    const i32x4 rv = make_rsrc(static_cast<const char*>(a.v) + (size_t)head * P.Skv * RB, (uint32_t)P.Skv * RB);
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      kf[s] = buf_load16(rk, kw * RB + (2 * s + hh) * 16);
      vf[s] = buf_load16(rv, kw * RB + (2 * s + hh) * 16);
    }
  }
  int qlo, qhi;  // queries that see this lane's key (masks are intervals here)
  query_interval(P, b, kw, &qlo, &qhi);

  // LDS operand offsets.  ds_read's immediate offset has 16 bits, and the dO
  // tiles and the statistics lie above 64 KiB: their reads go through lane
  // offsets that already include the region's start (kept opaque, so the
  // compiler holds them in registers instead of adding the start before
  // every read), leaving only tile-relative immediates.
  RowTile<D> rt, rtd;
  rt.init(lane);
  rtd.init(lane);
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s) {
    rtd.aoff[s] += 2 * TILE;
    asm volatile("" : "+v"(rtd.aoff[s]));
  }
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      rtd.tr[r][t] += 2 * TILE;
      asm volatile("" : "+v"(rtd.tr[r][t]));
    }
  int stat_off = 4 * TILE + 32 * hh;  // + acc_row(e, hh) - acc_row(e, 0), in bytes
  asm volatile("" : "+v"(stat_off));
  const char* const statp = lds + stat_off;
  TileDma<D, BQ, NW> dma;
  dma.init(lane, w);

  QWalk walk;
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

  // Copies of the next q tile (Q, dO rows, LSE and Delta) into buffer `buf`,
  // as NDMA single instructions per wave so the fast path can spread them
  // over its MFMA steps (the texture unit takes one copy instruction at a
  // time; four waves issuing all of theirs at once after a barrier queue for
  // hundreds of cycles).  A tile at qb >= Sq copies zeros.
  // The LSE and Delta tiles go through a register (one value per lane):
  // waves 0, 1 (wave 0 of a 2-wave group) load LSE and store -LSE * log2(e)
  // later in the step (stat_store), so the exponent needs one FMA per
  // element; waves 2, 3 (wave 1) load and store Delta.  The choice is a
  // wave-uniform select, not a branch, and waves with the same role write
  // identical data.
  struct TileCopy {
    i32x4 rq, rdo, rst;
    int buf;
  };
  constexpr int NST = BQ / 64;  // LSE / Delta values per lane and tile
  static_assert(BQ == 64 || BQ == 128, "q tile of 64 or 128 rows");
  constexpr int NDMA = 2 * TileDma<D, BQ, NW>::IPW + NST;
  const bool stat_delta = (w & (NW >= 4 ? 2 : 1)) != 0;
  const float stat_scale = stat_delta ? 1.0f : -kLog2e;
  auto plan = [&](int hq, int qb, int buf) {
    const size_t hoff = (size_t)(b * P.Hq + hq) * P.Sq;
    TileCopy c;
    c.rq = TileDma<D, BQ, NW>::rsrc(static_cast<const char*>(a.q) + hoff * RB, qb, P.Sq);
    c.rdo = TileDma<D, BQ, NW>::rsrc(static_cast<const char*>(a.dout) + hoff * RB, qb, P.Sq);
    const int q = qb < P.Sq ? qb : P.Sq;
    c.rst = make_rsrc((stat_delta ? a.delta : a.lse) + hoff + q, (uint32_t)(P.Sq - q) * 4);
    c.buf = buf;
    return c;
  };
  float stat_in[NST];
#pragma unroll
  for (int r = 0; r < NST; ++r) stat_in[r] = 0.f;
  auto copy_part = [&](const TileCopy& c, int k) {
    constexpr int IPW = TileDma<D, BQ, NW>::IPW;
    if (k < IPW) dma.one(c.rq, k, lds + c.buf * TILE, w);
    else if (k < 2 * IPW) dma.one(c.rdo, k - IPW, lds + (2 + c.buf) * TILE, w);
    else stat_in[k - 2 * IPW] = __builtin_bit_cast(float, raw_buffer_load_b32(c.rst, (64 * (k - 2 * IPW) + lane) * 4, 0, 0));
  };
  auto stat_store = [&](const TileCopy& c) {
    // lanes past BQ store into the unused rest of the landing zone
#pragma unroll
    for (int r = 0; r < NST; ++r)
      *reinterpret_cast<float*>(lds + 4 * TILE + ((stat_delta ? 2 : 0) + c.buf) * STAT + (64 * r + lane) * 4) =
          stat_in[r] * stat_scale;
  };
  auto issue = [&](int hq, int qb, int buf) {
    const TileCopy c = plan(hq, qb, buf);
#pragma unroll
    for (int k = 0; k < NDMA; ++k) copy_part(c, k);
    stat_store(c);
  };

  f32x16 dka[DT], dva[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) {  // AGPRs, accumulated in place
    zero(dka[i]);
    zero(dva[i]);
    mfma_drain<'a'>(dka[i]);
    mfma_drain<'a'>(dva[i]);
  }

  // One q tile (full or partial, with or without score mods): a fixed
  // sequence of 2*NQS*KS steps of two MFMAs each.  Its 32-row sub-tiles run
  // in pairs (2u, 2u + 1), four phases per pair
  //   A0: S_0, dP_0  |  A1: S_1, dP_1  |  C0: dV^T, dK^T += (sub-tile 0)  |  C1
  // with the exponentials / dS of sub-tile 0 (E0) spread over A1's steps and
  // those of sub-tile 1 (E1) over C0's, so VALU work issues while the matrix
  // core is busy; the next pair's accumulators are set up during C1.  Every
  // step also fetches the LDS operands of the step PF ahead (across phase and
  // pair boundaries; row fragments in A, transposed ones in C) and the LSE
  // quad due next (Delta is the dP MFMAs' initial value).  Score mods, when
  // present, are evaluated branch-free in the exponential's stage.
  // sched_barrier fences keep the compiler to this order.
  auto tile_fast = [&](int qbase, int hq, float slope, const char* ql, const float* lsel,
                       const float* dltl, auto&& prep, auto&& copy_k, auto&& stat_k, auto&& fetch_k,
                       auto masked_c) {
    constexpr bool kMasked = decltype(masked_c)::value;
    constexpr int KS = KSTEPS, NSTEP = 2 * NQS * KS, PF = APF, R = PF + 1;
    // first step of the last pair's A0 phase (steps with no E work; for a
    // single pair, the first step of C1)
    constexpr int kFetchStep = NQS > 2 ? 4 * KS * (NQS / 2 - 1) + 1 : 3 * KS + 1;
    static_assert(NDMA + 1 < NSTEP, "the next tile's copies fit the steps before its LSE store");
    static_assert(2 * DT == KS && NQS % 2 == 0, "fast path shape");
    // Partial tiles: element e of sub-tile J is query qbase + 32 J + 8 hh +
    // r(e), r(e) = acc_row(e, 0) < 24.  rmask[J] has bit r set iff that query
    // sees this lane's key; the packed P and dS words are ANDed with the
    // matching 0 / 0xffff halves, so masked elements contribute exact zeros
    // whatever their exponential came out as.
    uint32_t rmask[NQS];
#pragma unroll
    for (int j = 0; j < NQS; ++j) rmask[j] = 0u;
    if constexpr (kMasked) {
#pragma unroll
      for (int j = 0; j < NQS; ++j) {
        const int base = qbase + 32 * j + 8 * hh;
        const int lo = max(qlo - base, 0), hi = min(qhi - base, 31);
        const uint32_t up = 0xffffffffu >> (31 - max(hi, 0));
        const uint32_t dn = 0xffffffffu << min(lo, 31);
        rmask[j] = (hi >= lo) ? (up & dn) : 0u;
        if constexpr (Mod::kMask) {  // user mask on the rows this lane holds
          uint32_t bits = 0u;
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int r = acc_row(e, 0);
            bits |= Mod::mask(P, b, hq, base + r, kw) ? (1u << r) : 0u;
          }
          rmask[j] &= bits;
        }
      }
    }
    // 0xffff / 0 halves for the two elements of pair p (rows r, r + 1)
    auto pair_mask = [&](int J, int p) {
      const int r = acc_row(2 * p, 0);
      const uint32_t lo = (uint32_t)__builtin_amdgcn_sbfe((int)rmask[J], r, 1);
      const uint32_t hi = (uint32_t)__builtin_amdgcn_sbfe((int)rmask[J], r + 1, 1);
      return (lo & 0xffffu) | (hi & 0xffff0000u);
    };
    // E work in pairs of elements, spread evenly over the KS steps of its
    // phase (A1 for sub-tile 2u, C0 for 2u + 1): pair p at step p * KS / 8,
    // the LSE quad it needs read one step earlier.
    auto pair_step = [](int p) { return p * KS / 8; };
    // local accumulators of the current pair: sacc from zero, pacc from Delta
    // (dP accumulates onto it: pacc = Delta - dP, V negated)
    f32x16 sacc[2], pacc[2];
    auto init_pair = [&](int u) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        zero(sacc[j]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 d4 = *reinterpret_cast<const f32x4*>(dltl + 32 * (2 * u + j) + acc_row(4 * q, 0));
#pragma unroll
          for (int i = 0; i < 4; ++i) pacc[j][4 * q + i] = d4[i];
        }
      }
    };
    frag pf[2][2], sf[2][2];
    frag ring[R][2];
    f32x4 ls[2][4];
    auto load = [&](int t) {
      const int ph = t / KS, s = t % KS, u = ph / 4, lph = ph % 4;
      if (lph < 2) {
        ring[t % R][0] = rt.a_frag(ql, 2 * u + lph, s);
        ring[t % R][1] = rtd.a_frag(ql, 2 * u + lph, s);
      } else {
        const int J = 2 * u + lph - 2;
        ring[t % R][0] = rtd.t_frag(ql, s >> 1, 2 * J + (s & 1));
        ring[t % R][1] = rt.t_frag(ql, s >> 1, 2 * J + (s & 1));
      }
    };
    auto load_stats = [&](int J, int q) {
      const int r0 = 32 * J + acc_row(4 * q, 0);
      ls[J & 1][q] = *reinterpret_cast<const f32x4*>(lsel + r0);
    };
    // A pair's E work in two stages a step apart, so the exponentials'
    // latency passes under the next step's MFMAs: e_exp (P), then e_use (dS,
    // and the bf16 packing once a half of the sub-tile is complete).
    float pvq[8][2], dsq[8][2];
    const float cap_inv = P.softcap > 0.f ? 1.0f / P.softcap : 0.f;
    // built-in mods: the lane's ALiBi offset per sub-tile and the soft-cap constants
    // with the score's factor f (2 log2(e) / cap with the soft-cap, log2(e)
    // without) folded into the lane's ALiBi base, the slope and the scale
    float asb[NQS], msl = 0.f, msc = 0.f, mea = 1.0f;
#pragma unroll
    for (int j = 0; j < NQS; ++j) asb[j] = 0.f;
    bool capped = false;
    if constexpr (kMods && !Mod::kScore) {
      capped = P.softcap > 0.f;
      const float f = capped ? 2.0f * kLog2e * cap_inv : kLog2e;
#pragma unroll
      for (int j = 0; j < NQS; ++j) asb[j] = f * slope * (float)(kw - (qbase + 32 * j + 8 * hh));
      msl = -f * slope;
      msc = f * P.scale;
      mea = capped ? P.softcap * kLog2e : 1.0f;
    }
    auto e_exp = [&](int J, int p) {
      const int j = J & 1;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int e = 2 * p + i, q = e >> 2;
        if constexpr (kMods && !Mod::kScore) {
          // built-in ALiBi + soft-cap (branch-free: both results, selected):
          // u = f (scale q.k + slope (k - q)); tanh(s / cap) = 1 - 2 / (2^u + 1)
          // as one exp2 and one rcp; the logit is cap log2(e) tanh, or u
          const float u = fmaf(sacc[j][e], msc, fmaf(msl, (float)acc_row(e, 0), asb[J]));
          const float th = fmaf(-2.0f, fast_rcp(fast_exp2(u) + 1.0f), 1.0f);
          dsq[p][i] = capped ? fmaf(-th, th, 1.0f) : 1.0f;
          pvq[p][i] = fast_exp2(fmaf(mea, capped ? th : u, ls[j][q][e & 3]));
        } else if constexpr (kMods) {
          // score mods (log2-domain logit) and d s / d(scale q.k) for dS
          const float t = mod_score_flat<Mod>(P, sacc[j][e], slope, b, hq, qbase + 32 * J + acc_row(e, hh), kw,
                                              cap_inv, &dsq[p][i]);
          pvq[p][i] = fast_exp2(t + ls[j][q][e & 3]);
        } else {
          pvq[p][i] = fast_exp2(fmaf(sacc[j][e], P.scale_log2, ls[j][q][e & 3]));
        }
      }
    };
    auto e_use = [&](int J, int p) {
      const int j = J & 1;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int e = 2 * p + i;
        sacc[j][e] = pvq[p][i];
        if constexpr (kMods) pacc[j][e] = -pvq[p][i] * pacc[j][e] * dsq[p][i];
        else pacc[j][e] = -pvq[p][i] * pacc[j][e];
      }
      if ((p & 3) == 3) {
        const int half = p >> 2;
        float x[8], y[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          x[t] = sacc[j][8 * half + t];
          y[t] = pacc[j][8 * half + t];
        }
        pf[j][half] = E::pack(x);
        sf[j][half] = E::pack(y);
        if constexpr (kMasked) {
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const uint32_t m = pair_mask(J, 4 * half + w);
            pf[j][half][w] &= m;
            sf[j][half][w] &= m;
          }
        }
        // the 2 wait states an MFMA needs after a VALU write of its operand
        // (a half can be read in the very next step)
        asm volatile("s_nop 1" : "+v"(pf[j][half]), "+v"(sf[j][half]));
      }
    };
    init_pair(0);
#pragma unroll
    for (int t = 0; t < PF; ++t) load(t);
    // the next tile's walk and copy plan (scalar work) while the first
    // operand reads are in flight
    __builtin_amdgcn_sched_barrier(0);
    prep();
#pragma unroll
    for (int t = 0; t < NSTEP; ++t) {
      const int ph = t / KS, s = t % KS, u = ph / 4, lph = ph % 4;
      if (t + PF < NSTEP) load(t + PF);
      // LSE of the quads whose first pair comes in the next step (sub-tile J's
      // E work runs in phase 4 (J / 2) + (J % 2) + 1)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int J = 0; J < NQS; ++J)
          if ((4 * (J >> 1) + (J & 1) + 1) * KS + pair_step(2 * q) == t + 1) load_stats(J, q);
      if (lph < 2) {
        sacc[lph] = E::mma(ring[t % R][0], kf[s], sacc[lph]);
        pacc[lph] = E::mma(ring[t % R][1], vf[s], pacc[lph]);
      } else {
        const int j = lph - 2;
        // the packing fences P and dS (see e_use), so no s_nop here
        mfma_acc<'a', false>(dva[s >> 1], ring[t % R][0], pf[j][s & 1]);
        mfma_acc<'a', false>(dka[s >> 1], ring[t % R][1], sf[j][s & 1]);
      }
      if (t > 0) {  // second stage of last step's pairs
        const int pph = (t - 1) / KS, plph = pph % 4;
        if (plph == 1 || plph == 2) {
#pragma unroll
          for (int p = 0; p < 8; ++p)
            if (pair_step(p) == (t - 1) % KS) e_use(2 * (pph / 4) + plph - 1, p);
        }
      }
      if (lph == 1 || lph == 2) {
#pragma unroll
        for (int p = 0; p < 8; ++p)
          if (pair_step(p) == s) e_exp(2 * u + lph - 1, p);
      }
      // the next pair's accumulators, once sub-tile 2u + 1's E work is done
      // (its last pair's second stage runs in C1's first step)
      if (lph == 3 && s == 1 && 2 * u + 2 < NQS) init_pair(u + 1);
      // the next tile's copies, one per step; its LSE stored near the end
      if (t < NDMA) copy_k(t);
      if (t == NSTEP - 2) stat_k();
      // the table entry of the tile after next: its scalar work runs beside
      // the MFMAs of a step with no exponentials or copies, its load passes
      // under the rest of the tile (at the tile's end all four waves would
      // run it on the shared scalar unit at once)
      if (t == kFetchStep) fetch_k();
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Full tiles run first, in a loop of their own without the element mask;
  // the partial tiles follow.  Rows past Sq need no mask: their Q, dO, LSE and
  // Delta read as zero, so P = 1 and dS = 0 there and dO^T P, Q^T dS get
  // nothing from them.  Keys past Skv only touch lanes that are not stored.
  // Table entries are fetched two tiles ahead, resolved one tile ahead.
  int hq_next = 0, qb_next = 0;
  TileRef ref_next{0, 0, 0};
  if (n_it > 0) {
    const TileRef r0 = spec0 ? TileRef{walk.count_full() > 0 ? first_full : first_part, 0, walk.hq0} : walk.fetch(0);
    hq_next = r0.hq;
    qb_next = walk.qbase(r0);
    issue(hq_next, qb_next, 0);
    if (n_it > 1) ref_next = walk.fetch(1);
  }
  // unconditional, so the wait-count analysis sees the register loads above
  // complete on every path into the loop
  wait_vmem();
  __syncthreads();
  // V is kept negated (bf16 sign flips), so the dP MFMA accumulates -dP onto
  // whatever its accumulator starts from: the fast path starts it from Delta
  // and gets Delta - dP, dS = -P (Delta - dP) with one multiply per element.
  // (Done here, after the prologue's wait, so the K / V loads overlap the
  // table lookups and the first tile's copy.)
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s) {
    vf[s] ^= 0x80008000u;
    // K and V live in AGPRs (the S and dP MFMAs read their B operand from
    // there): beside the dK / dV accumulators the AGPR file has 128 registers
    // left, and the 64 VGPRs this frees hold the LDS offsets of the dO and
    // statistics reads (about 70 VALU instructions fewer per q tile).
    asm volatile("" : "+a"(vf[s]));
    asm volatile("" : "+a"(kf[s]));
  }
  auto step = [&](int it, auto masked_c, auto buf_c) {
    constexpr int buf = decltype(buf_c)::value;  // == it & 1, a constant (immediate LDS offsets)
    const int hq = hq_next, qbase = qb_next;
    // the next tile and its copies (past the last tile they target qb = Sq:
    // zeros into the idle buffer); run by tile_fast once its first LDS reads
    // are issued
    TileCopy next;
    auto prep = [&]() {
      if (it + 1 < n_it) {
        hq_next = ref_next.hq;
        qb_next = walk.qbase(ref_next);
      } else {
        qb_next = P.Sq;
      }
      next = plan(hq_next, qb_next, buf ^ 1);
    };
    auto copy_k = [&](int k) { copy_part(next, k); };
    auto stat_k = [&]() { stat_store(next); };
    auto fetch_next = [&]() { ref_next = walk.fetch(min(it + 2, n_it - 1)); };
    if (qbase < P.Sq) {
      const float slope = (kMods && P.alibi) ? P.alibi[hq] : 0.f;
      tile_fast(qbase, hq, slope, lds + buf * TILE,
                reinterpret_cast<const float*>(statp + buf * STAT),
                reinterpret_cast<const float*>(statp + (2 + buf) * STAT), prep, copy_k, stat_k,
                fetch_next, masked_c);
    } else {
      prep();
#pragma unroll
      for (int k = 0; k < NDMA; ++k) copy_k(k);
      fetch_next();
      stat_k();
    }
    wait_vmem();
    __syncthreads();
  };
  const int n_full = walk.count_full();
  run_tiles(0, n_full, step, False{});
  run_tiles(n_full, n_it, step, True{});

#pragma unroll
  for (int i = 0; i < DT; ++i) {
    mfma_drain<'a'>(dka[i]);
    mfma_drain<'a'>(dva[i]);
  }
  // dK, dV rows of this wave, staged through the (now idle) tile buffers
  {
    const int rows_left = P.Skv - (k0 + 32 * w);
    uint16_t* dkp = static_cast<uint16_t*>(a.dk) + ((size_t)head * P.Skv + k0 + 32 * w) * D;
    uint16_t* dvp = static_cast<uint16_t*>(a.dv) + ((size_t)head * P.Skv + k0 + 32 * w) * D;
    char* stage = lds + w * 2 * (32 * RB);
    store_rows_bf16<D>(dka, P.scale, stage, dkp, rows_left, lane);
    store_rows_bf16<D>(dva, 1.0f, stage + 32 * RB, dvp, rows_left, lane);
  }
}

}  // namespace fa
