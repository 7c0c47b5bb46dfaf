// Forward FlexAttention on fp8 inputs (OCP e4m3: Q, K, and V stored
// transposed), with power-of-two scales per 128-row block, on gfx950's
// v_mfma_scale_f32_32x32x64_f8f6f4.  Not in the reference (its kernels are
// bf16 / fp32 only); the masks, block tables, work order and the built-in
// score mods are the bf16 forward's.
//
// Layout (one workgroup = 4 waves = 128 query rows of one (batch, q head)):
//   * S^T = K Q^T per 32-key sub-tile: A = K rows (keys), B = Q^T (the lane's
//     query, 32 consecutive head-dim bytes per lane half, held in registers
//     for the whole walk), 64-deep k steps over D.  The E8M0 scale operands
//     carry the K block's scale (uniform) and the lane's Q block scale, so
//     the accumulator is q.k of the dequantised rows exactly (fp32 sums).
//   * K rows are read in the order perm_f8: accumulator element e of lane
//     half h is then key 16 h + e of the sub-tile, so a lane holds the P of
//     keys 16 h + [0, 16) of both sub-tiles -- 32 consecutive k of the PV
//     product's B operand, packed by v_cvt_pk_fp8_f32 without any exchange.
//   * O^T += V^T P^T: A = V^T rows (head-dim index, keys along the row, read
//     in two 16-byte pieces), B = P^T, the E8M0 A scale the V block's.
//   * P is stored as p * 2^3 (kPBias): e4m3 keeps p >= 2^-9 normal and
//     p >= 2^-12 at all; the fp32 row sum l takes the unrounded values and
//     the final O / l cancels the bias.  The speculative softmax of the bf16
//     forward carries over with kSpill = 448 (the e4m3 maximum): a lane's tile
//     sum within 448 bounds every stored value by it, no conversion
//     overflows, and any larger sum takes the exact path (row maximum,
//     rescale), after which every value is at most 2^3.
#pragma once
#include "dma.h"
#include "fwd.h"
#include "kargs.h"

namespace fa {

typedef int i32x8 __attribute__((ext_vector_type(8)));

constexpr int kFp8ScaleRows = 128;  // rows per scale block (queries or keys)

struct Fp8FwdArgs {
  Problem p;
  const uint8_t* q;      // (B, Hq, Sq, D) e4m3
  const uint8_t* k;      // (B, Hkv, Skv, D) e4m3
  const uint8_t* vt;     // (B, Hkv, D, ldv) e4m3: V transposed, keys padded to ldv
  int ldv;               // multiple of 128, >= Skv; padding keys are zero
  const float* q_scale;  // (B * Hq, ceil(Sq / 128)), powers of two
  const float* k_scale;  // (B * Hkv, ceil(Skv / 128))
  const float* v_scale;  // (B * Hkv, ceil(Skv / 128))
  void* o;               // bf16 (B, Hq, Sq, D)
  float* lse;            // (B, Hq, Sq), natural-log units
};

// E8M0 code of a power-of-two float (its biased exponent): the scale operand
// of the scaled MFMA means 2^(code - 127), as the float's exponent field does.
__device__ __forceinline__ int e8m0_code(float s) { return (int)((__float_as_uint(s) >> 23) & 0xffu); }

// physical key (within a 32-key sub-tile) read as A row r of S^T = K Q^T:
// accumulator element e of lane half h (row 8 (e / 4) + 4 h + e % 4) is key
// 16 h + e
__device__ __forceinline__ int perm_f8(int r) { return (((r >> 2) & 1) << 4) | (((r >> 3) & 3) << 2) | (r & 3); }

// K tiles: rows of D bytes (KCH = D / 16 chunks of 16 B); a 16-lane group of
// an A-operand read takes rows perm_f8(0..15) (or 16..31), i.e. [0, 8) and
// [16, 24) (or [8, 16) and [24, 32)), one logical chunk: the swizzle maps
// them to 16 distinct 16-byte bank slots (64 banks x 4 B).
template <int KCH>
__device__ __forceinline__ int swz_k8(int r) {
  static_assert(KCH == 4 || KCH == 8, "chunks per K row");
  if constexpr (KCH == 8) return ((r >> 1) & 3) | (((r >> 4) & 1) << 2);
  else return ((r >> 2) & 1) | (((r >> 4) & 1) << 1);
}
// V^T tiles: rows of 64 bytes (4 chunks); a 16-lane group reads 16
// consecutive rows, one logical chunk
__device__ __forceinline__ int swz_v8(int r) { return (r >> 2) & 3; }

__device__ __forceinline__ i32x8 cat8(u32x4 lo, u32x4 hi) {
  return i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

// acc += A B with e4m3 A, B and E8M0 scales sa (A rows), sb (B columns)
__device__ __forceinline__ f32x16 mma_f8(i32x8 a, i32x8 b, f32x16 acc, int sa, int sb) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc, 0, 0, 0, sa, 0, sb);
}

template <int D, int NW, bool kMods>
// (three waves per SIMD: the 32 KiB of LDS allows five workgroups per CU, and
// the third wave hides more of the softmax than the registers it takes cost:
// 8 % faster than two at causal S = 8192; with score mods two, whose 256
// registers hold the longer per-score chain without spilling)
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(occupancy_for(4 * 64 * D, NW, kMods ? 2 : 3))))
void fwd_fp8_kernel(Fp8FwdArgs a) {
  constexpr int BN = 64;              // keys per tile
  constexpr int BM = 32 * NW;
  constexpr int KCH = D / 16;         // 16-byte chunks per K row
  constexpr int KS = D / 64;          // 64-deep k steps over D
  constexpr int DT = D / 32;          // d tiles of O
  constexpr int TILE = BN * D;        // bytes per K (or V^T) tile
  constexpr int IPW = TILE / 1024 / NW;
  constexpr float kSpill = 448.0f;    // e4m3 maximum
  constexpr float kPBias = 3.0f;      // P stored as p * 2^kPBias
  static_assert(D == 64 || D == 128, "head dim");
  static_assert(TILE % (1024 * NW) == 0, "DMA split");
  static_assert(4 * TILE >= BM * 2 * D, "O rows staged through the K / V buffers");

  __shared__ __attribute__((aligned(1024))) char lds[4 * TILE];  // K0 K1 V0 V1

  const Problem& P = a.p;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 31, hh = lane >> 5;
  const int g = P.Hq / P.Hkv;
  const int nqt = (P.Sq + BM - 1) / BM;
  int head, qt;
  work_item((int)blockIdx.x, P.B * P.Hq, nqt, P.xcd_remap, P.head_group_q, false, &head, &qt);
  const int b = head / P.Hq, h = head - b * P.Hq, hk = h / g;
  const int q0 = qt * BM;
  const int qw = q0 + 32 * w + lr;
  const bool qvalid = qw < P.Sq;
  const int skv = P.Skv;
  const int nqb = (P.Sq + kFp8ScaleRows - 1) / kFp8ScaleRows;
  const int nkb = (skv + kFp8ScaleRows - 1) / kFp8ScaleRows;
  const int kvh = b * P.Hkv + hk;

  const char* kbase_ptr = reinterpret_cast<const char*>(a.k) + (size_t)kvh * skv * D;
  const char* vbase_ptr = reinterpret_cast<const char*>(a.vt) + (size_t)kvh * D * a.ldv;

  // Q rows as B operands (rows past the sequence read as zero) and their scale
  i32x8 qf[KS];
  {
    const i32x4 rq = make_rsrc(reinterpret_cast<const char*>(a.q) + (size_t)head * P.Sq * D, (uint32_t)P.Sq * D);
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qf[s] = cat8(buf_load16(rq, qw * D + 64 * s + 32 * hh), buf_load16(rq, qw * D + 64 * s + 32 * hh + 16));
  }
  const int scq = e8m0_code(a.q_scale[(size_t)head * nqb + (qvalid ? qw : P.Sq - 1) / kFp8ScaleRows]);
  const float slope = P.alibi ? P.alibi[h] : 0.f;
  const float cap_inv = P.softcap > 0.f ? 1.0f / P.softcap : 0.f;
  int klo, khi;
  key_interval(P, b, qw, &klo, &khi);
  khi = min(khi, skv - 1);

  // loop-invariant LDS / global offsets (chunk slot p of LDS row r holds
  // global chunk p ^ swizzle(r))
  int dma_off_k[IPW], dma_off_v[IPW];
#pragma unroll
  for (int u = 0; u < IPW; ++u) {
    const int gi = (w * IPW + u) * 64 + lane;
    const int rk = gi / KCH, pk = gi % KCH;
    dma_off_k[u] = rk * D + ((pk ^ swz_k8<KCH>(rk)) * 16);
    const int rv = gi / 4, pv = gi % 4;
    dma_off_v[u] = rv * a.ldv + ((pv ^ swz_v8(rv)) * 16);
  }
  // K fragment reads: row perm_f8(lr) (+ 32 j), logical chunks 4 s + 2 hh + x
  int koff[KS][2];
  {
    const int r = perm_f8(lr);
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int x = 0; x < 2; ++x) koff[s][x] = r * D + (((4 * s + 2 * hh + x) ^ swz_k8<KCH>(r)) * 16);
  }
  // V^T fragment reads: row lr (+ 32 i), logical chunks hh (keys 16 hh ..) and
  // 2 + hh (keys 32 + 16 hh ..)
  int voff[2];
#pragma unroll
  for (int x = 0; x < 2; ++x) voff[x] = lr * BN + (((2 * x + hh) ^ swz_v8(lr)) * 16);

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

  // HBM -> LDS copies of the tile starting at key kb into buffer `buf`
  // (a tile past the end copies zeros: empty ranges at the head's base)
  // (plan, then one copy instruction at a time: inside the walk they are
  // spread over the S phase's MFMAs, as in the bf16 forward)
  struct Copy { i32x4 rk, rv; char* kl; char* vl; };
  auto issue_plan = [&](int kb, int buf) {
    const bool live = kb < skv;
    kb = live ? kb : 0;
    Copy c;
    c.rk = make_rsrc(kbase_ptr + (size_t)kb * D, live ? (uint32_t)(skv - kb) * D : 0u);
    c.rv = make_rsrc(vbase_ptr + kb, live ? (uint32_t)D * a.ldv - (uint32_t)kb : 0u);
    c.kl = lds + buf * TILE;
    c.vl = lds + (2 + buf) * TILE;
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
  // E8M0 codes of the K and V blocks holding key kb (wave-uniform)
  const int* ksc = reinterpret_cast<const int*>(a.k_scale) + (size_t)kvh * nkb;
  const int* vsc = reinterpret_cast<const int*>(a.v_scale) + (size_t)kvh * nkb;

  f32x16 oacc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[i][e] = 0.f;
  float m = -INFINITY, l = 0.f;

  // With mods a tile holds y with the log2-domain logit ea * y + eb, as in
  // the bf16 forward: the logit (ea = 1, eb = 0), or with the soft-cap
  // r = 1 / (2^t + 1) (ea = -2 cap log2(e), eb = cap log2(e)); masked
  // elements hold the y whose logit is -inf.
  const bool rform = kMods && P.softcap > 0.f;
  const float ea = rform ? -2.0f * P.softcap * kLog2e : 1.0f;
  const float eb = rform ? P.softcap * kLog2e : 0.0f;
  // p * 2^kPBias of a whole tile against reference muse into the e4m3 operand
  // pf (element e of sub-tile j is byte 16 j + e); returns the lane's sum
  auto exps = [&](const f32x16* sacc, i32x8& pf, float muse) {
    float rs0 = 0.f, rs1 = 0.f;
    const float mb = muse - kPBias;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; e += 4) {
        float x[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float s = sacc[j][e + t];
          if constexpr (kMods) x[t] = fast_exp2(fmaf(s, ea, eb - mb));
          else x[t] = fast_exp2(fmaf(s, P.scale_log2, -mb));
        }
        int word = __builtin_amdgcn_cvt_pk_fp8_f32(x[0], x[1], 0, false);
        word = __builtin_amdgcn_cvt_pk_fp8_f32(x[2], x[3], word, true);
        pf[4 * j + e / 4] = word;
        rs0 += x[0] + x[2];
        rs1 += x[1] + x[3];
      }
    return rs0 + rs1;
  };
  auto softmax = [&](const f32x16* sacc, i32x8& pf) {
    float rs = exps(sacc, pf, m == -INFINITY ? 0.f : m);
    if (__any(!(rs <= kSpill) || m == -INFINITY)) {  // exact path (wave-uniform)
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < 2; ++j)
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
        for (int i = 0; i < DT; ++i)
#pragma unroll
          for (int e = 0; e < 16; ++e) oacc[i][e] *= alpha;
        m = mnew;
      }
      rs = exps(sacc, pf, m == -INFINITY ? 0.f : m);
    }
    l += rs;
  };

  const int n_full = walk.count_full();
  const int sub_log2 = log2_if_pow2(walk.sub);
  KvTab tab;
  auto kbase_of = [&](int it) { return tab.kbase(walk, it, sub_log2, lane); };
  if (n_it > 0) issue(kbase_of(0), 0);
  wait_vmem();
  __syncthreads();
  auto tile_step = [&](int it, auto buf_c) {
    constexpr int buf = decltype(buf_c)::value;
    const int kbase = kbase_of(it);
    bool masked = it >= n_full;
    const bool more = it + 1 < n_it;
    Copy nc;
    if (more) nc = issue_plan(kbase_of(it + 1), buf ^ 1);
    if (kbase >= skv && more) {
#pragma unroll
      for (int i = 0; i < 2 * IPW; ++i) issue_one(nc, i);
    }
    if (kbase < skv) {  // workgroup-uniform
      masked = masked || (kbase + BN > skv);
      const char* kl = lds + buf * TILE;
      const char* vl = lds + (2 + buf) * TILE;
      const int kblk = kbase / kFp8ScaleRows;
      const int sck = (scalar_load(ksc, kblk) >> 23) & 0xff;
      const int scv = (scalar_load(vsc, kblk) >> 23) & 0xff;

      f32x16 sacc[2];
      __builtin_amdgcn_s_setprio(1);  // MFMA phases first in issue order (4 % at C2, measured)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
#pragma unroll
        for (int e = 0; e < 16; ++e) sacc[j][e] = 0.f;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const char* kr = kl + j * 32 * D;
          const i32x8 kf = cat8(*reinterpret_cast<const u32x4*>(kr + koff[s][0]),
                                *reinterpret_cast<const u32x4*>(kr + koff[s][1]));
          sacc[j] = mma_f8(kf, qf[s], sacc[j], sck, scq);
          // this step's share of the next tile's copies
#pragma unroll
          for (int i = 0; i < 2 * IPW; ++i)
            if (i * 2 * KS / (2 * IPW) == j * KS + s && more) issue_one(nc, i);
        }
      }
      __builtin_amdgcn_s_setprio(0);
      if constexpr (kMods) {
        // ALiBi + soft-cap as in the bf16 forward: slope (k - q) = sb + slope e,
        // the score's factor (2 log2(e) / cap with the soft-cap, log2(e)
        // without) folded into the FMAs; with the soft-cap the tile keeps
        // r = 1 / (2^t + 1) (one exp2, one rcp), a wave-uniform branch
        const float f = P.softcap > 0.f ? 2.0f * kLog2e * cap_inv : kLog2e;
        const float af = P.scale * f, slf = slope * f;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float sbf = slope * (float)(kbase + 32 * j + 16 * hh - qw) * f;
          if (P.softcap > 0.f) {
#pragma unroll
            for (int e = 0; e < 16; ++e)
              sacc[j][e] = fast_rcp(fast_exp2(fmaf(sacc[j][e], af, fmaf(slf, (float)e, sbf))) + 1.0f);
          } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) sacc[j][e] = fmaf(sacc[j][e], af, fmaf(slf, (float)e, sbf));
          }
        }
      }
      if (masked) {  // partial tile: keys outside [klo, khi] are dropped
        const float dead = rform ? INFINITY : -INFINITY;  // the y whose logit is -inf
        const int lo = klo - kbase - 16 * hh, hi = khi - kbase - 16 * hh;  // tile-relative bounds
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int c = 32 * j + e;
            sacc[j][e] = (c >= lo && c <= hi) ? sacc[j][e] : dead;
          }
      }
      i32x8 pf;
      softmax(sacc, pf);
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int i = 0; i < DT; ++i) {
        const char* vr = vl + i * 32 * BN;
        const i32x8 vf = cat8(*reinterpret_cast<const u32x4*>(vr + voff[0]),
                              *reinterpret_cast<const u32x4*>(vr + voff[1]));
        oacc[i] = mma_f8(vf, pf, oacc[i], scv, 127);
      }
      __builtin_amdgcn_s_setprio(0);
    }
    wait_vmem();
    __syncthreads();
  };
  int it = 0;
  for (; it + 1 < n_it; it += 2) {
    tile_step(it, Bool<0>{});
    tile_step(it + 1, Bool<1>{});
  }
  if (it < n_it) tile_step(it, Bool<0>{});

  const float lt = pair_sum(l);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  // O rows of this wave, staged through the (now idle) K / V buffers
  store_rows_bf16<D>(oacc, inv, lds + w * (32 * 2 * D),
                     static_cast<uint16_t*>(a.o) + ((size_t)head * P.Sq + q0 + 32 * w) * D, P.Sq - (q0 + 32 * w),
                     lane);
  if (qvalid && hh == 0) a.lse[(size_t)head * P.Sq + qw] = lt > 0.f ? (m - kPBias + log2f(lt)) * kLn2 : -INFINITY;
}

// ---- quantisation ------------------------------------------------------------
// Rows (B * H heads of S rows of D bf16) to e4m3 with one power-of-two scale
// per 128-row block: scale = 2^ceil(log2(amax / 448)) (1 for an all-zero
// block; the largest power of two whose product with 448 still covers
// amax; exponent clamped to [-126, 127]), element = RNE(x / scale): the
// division by a power of two is exact, so the element stays within +-448.
// One workgroup (256 threads) per block.
// With `transpose` the block is written as D rows of the padded key axis
// (ld bytes per row, V^T layout of the fp8 forward), else row-major.
struct QuantArgs {
  const uint16_t* x;  // (heads, S, D) bf16
  uint8_t* out;       // (heads, S, D) or (heads, D, ld)
  float* scale;       // (heads, ceil(S / 128))
  int heads, S, D, ld, transpose;
};

__device__ __forceinline__ float bf16_to_f32(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }

// 4 x 4 byte transpose: o[c] byte r = byte c of word r (v_perm_b32 picks
// bytes of {S0, S1}, selector values 0-3 from S1, 4-7 from S0)
__device__ __forceinline__ void transpose_bytes4(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3, uint32_t* o) {
  const uint32_t t0 = __builtin_amdgcn_perm(w1, w0, 0x05010400u);  // w0.b0 w1.b0 w0.b1 w1.b1
  const uint32_t t1 = __builtin_amdgcn_perm(w1, w0, 0x07030602u);  // w0.b2 w1.b2 w0.b3 w1.b3
  const uint32_t t2 = __builtin_amdgcn_perm(w3, w2, 0x05010400u);
  const uint32_t t3 = __builtin_amdgcn_perm(w3, w2, 0x07030602u);
  o[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
  o[1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
  o[2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
  o[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}

// One pass over the block: each working thread holds eight 16-byte chunks
// (64 values) in registers from the load through the block maximum to the
// conversion.  Row-major output: chunk tid + NT j of the block, stored as 8
// bytes.  Transposed output: rows 8 g .. 8 g + 7 of chunk c (g = tid % 16,
// c = tid / 16), the 8 x 8 bytes transposed in registers and stored as 8
// bytes of each of the chunk's 8 V^T rows (16 lanes fill a 128-byte row).
template <int D>
__global__ __launch_bounds__(256) void quant_fp8_kernel(QuantArgs a) {
  constexpr int R = kFp8ScaleRows;
  constexpr int NCH = D / 8;         // 16-byte chunks per row
  constexpr int NT = R * NCH / 8;    // threads with work (8 chunks each): 256, 128, 64
  static_assert(R == 128 && NT <= 256 && NT == 16 * NCH, "block shape");
  __shared__ float red[4];
  const int nb = (a.S + R - 1) / R;
  const int head = blockIdx.x / nb, blk = blockIdx.x - head * nb;
  const int r0 = blk * R;
  const int rows = min(R, a.S - r0);
  const uint16_t* src = a.x + ((size_t)head * a.S + r0) * D;
  const int tid = threadIdx.x;
  const bool tr = a.transpose != 0;
  const bool act = tid < NT;
  const int g = tid & 15, c = tid >> 4;
  auto row_of = [&](int j) { return tr ? 8 * g + j : (tid + NT * j) / NCH; };
  auto chunk_of = [&](int j) { return tr ? c : (tid + NT * j) % NCH; };
  u32x4 v[8];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = row_of(j);
    v[j] = u32x4{0u, 0u, 0u, 0u};
    if (act && r < rows) v[j] = *reinterpret_cast<const u32x4*>(src + r * D + chunk_of(j) * 8);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      amax = fmaxf(amax, fabsf(__uint_as_float(v[j][t] << 16)));
      amax = fmaxf(amax, fabsf(__uint_as_float(v[j][t] & 0xffff0000u)));
    }
  // block maximum: across the wave, then the four waves
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  // smallest e with 448 * 2^e >= amax (frexp-style on the ratio, exact)
  // (clamped to [-126, 127]: the scale stays a normal float, whose exponent
  // field is its E8M0 code; a non-finite amax leaves scale 1)
  int e = 0;
  if (amax > 0.f && amax < INFINITY) {
    int ex;
    const float f = frexpf(amax / 448.0f, &ex);  // amax / 448 = f 2^ex, f in [0.5, 1)
    e = (f == 0.5f) ? ex - 1 : ex;
    e = e < -126 ? -126 : (e > 127 ? 127 : e);
  }
  const float inv = ldexpf(1.0f, -e);
  if (tid == 0) a.scale[(size_t)head * nb + blk] = ldexpf(1.0f, e);
  if (!act) return;
  // convert (rows past S are zero): lo = values 0-3 of the chunk, hi = 4-7
  uint32_t lo[8], hi[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float x[8];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      x[2 * t] = __uint_as_float(v[j][t] << 16) * inv;
      x[2 * t + 1] = __uint_as_float(v[j][t] & 0xffff0000u) * inv;
    }
    int w0 = __builtin_amdgcn_cvt_pk_fp8_f32(x[0], x[1], 0, false);
    w0 = __builtin_amdgcn_cvt_pk_fp8_f32(x[2], x[3], w0, true);
    int w1 = __builtin_amdgcn_cvt_pk_fp8_f32(x[4], x[5], 0, false);
    w1 = __builtin_amdgcn_cvt_pk_fp8_f32(x[6], x[7], w1, true);
    lo[j] = (uint32_t)w0;
    hi[j] = (uint32_t)w1;
  }
  if (!tr) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int r = row_of(j);
      if (r < rows) *reinterpret_cast<u32x2*>(a.out + ((size_t)head * a.S + r0 + r) * D + chunk_of(j) * 8) = u32x2{lo[j], hi[j]};
    }
    return;
  }
  // V^T: row d = 8 c + k of the block holds bytes k of rows 8 g .. 8 g + 7
  uint32_t tl[8], th[8];  // tl[k]: rows 8g..8g+3 of head-dim index 8c + k, th[k]: rows 8g+4..8g+7
  transpose_bytes4(lo[0], lo[1], lo[2], lo[3], tl);
  transpose_bytes4(lo[4], lo[5], lo[6], lo[7], th);
  transpose_bytes4(hi[0], hi[1], hi[2], hi[3], tl + 4);
  transpose_bytes4(hi[4], hi[5], hi[6], hi[7], th + 4);
  uint8_t* dst = a.out + ((size_t)head * D + 8 * c) * a.ld + r0 + 8 * g;
#pragma unroll
  for (int k = 0; k < 8; ++k) *reinterpret_cast<u32x2*>(dst + (size_t)k * a.ld) = u32x2{tl[k], th[k]};
}

}  // namespace fa
