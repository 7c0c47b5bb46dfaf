// Backward FlexAttention kernels for gfx950.
//
//   delta_kernel : Delta[q] = sum_d O[q,d] * dO[q,d]            (fp32)
//   dkdv_kernel  : one workgroup per (batch, kv head, BKV = 32*NW keys); each
//                  wave owns 32 keys and keeps K, V (as MFMA B operands) and the
//                  dK^T, dV^T accumulators in registers while it walks the
//                  q-side block tables of every q head of its GQA group:
//                    S  = Q K^T,  dP = dO V^T          (lane = key, rows = queries)
//                    P  = exp(S - LSE),  dS = P (dP - Delta) * softcap'
//                    dV^T += dO^T P,  dK^T += Q^T dS   (P / dS reused from registers)
//                  Q, dO (row-major) and Q^T, dO^T (for the last two products)
//                  are staged in swizzled LDS per q tile.
//   dq_kernel    : one workgroup per (batch, q head, BQ = 32*NW queries), the
//                  forward's structure: Q and dO rows in registers,
//                    S^T = K Q^T, dP^T = V dO^T   (lane = query)
//                    dQ^T += K^T dS^T
//                  K, V (row-major) and K^T staged in LDS per kv tile.
// All products accumulate in fp32; P and dS are rounded to the input dtype
// before their MFMAs, as in the reference (flash_attn.py:244-245, :349).
#pragma once
#include "fwd.h"

namespace fa {

struct BwdArgs {
  Problem p;
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const float* lse;
  const void* dout;
  void* dq;
  void* dk;
  void* dv;
  float* delta;  // workspace (B, Hq, Sq)
  // bf16 dQ tile kernel only: compute Delta itself from O and dO and write it
  // to `delta` (the whole backward then runs dQ before dK/dV, no Delta pass)
  int fuse_delta;
};

// sum_j O[j] dO[j] over one 16-byte chunk of bf16 (8 elements), in the order
// both Delta paths use (the Delta kernel and the dQ kernel's fused form give
// bit-identical rows)
__device__ __forceinline__ float chunk_dot_bf16(u32x4 o, u32x4 d) {
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) acc += bf16_lo(o[j]) * bf16_lo(d[j]) + bf16_hi(o[j]) * bf16_hi(d[j]);
  return acc;
}

// ---------------------------------------------------------------- Delta ----
template <typename T, int D>
__global__ __launch_bounds__(256) void delta_kernel(BwdArgs a, int nrows) {
  constexpr int ES = sizeof(T);
  constexpr int KCH = D * ES / 16;  // threads per row
  constexpr int RPB = 256 / KCH;
  const int tid = threadIdx.x;
  const int row = blockIdx.x * RPB + tid / KCH, c = tid % KCH;
  const bool ok = row < nrows;
  const u32x4 ov = ld16(static_cast<const T*>(a.o) + (size_t)row * D + c * (16 / ES), ok);
  const u32x4 dv = ld16(static_cast<const T*>(a.dout) + (size_t)row * D + c * (16 / ES), ok);
  float acc = 0.f;
  if constexpr (ES == 2) {
    acc = chunk_dot_bf16(ov, dv);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc += __uint_as_float(ov[j]) * __uint_as_float(dv[j]);
  }
#pragma unroll
  for (int s = KCH / 2; s >= 1; s >>= 1) acc += __shfl_xor(acc, s, 64);
  if (ok && c == 0) a.delta[row] = acc;
}

using QWalk = QWalkT<DeviceLoad>;

// ----------------------------------------------------------------- dK dV ---
template <typename T, int D, int BQ, int NW, bool kMods, class Mod = BuiltinMod>
__global__ __launch_bounds__(NW * 64) void dkdv_kernel(BwdArgs a) {
  using E = Elt<T>;
  using frag = typename E::frag;
  constexpr int BKV = 32 * NW;
  constexpr int NT = NW * 64;
  constexpr int ES = sizeof(T);
  constexpr int EPC = 16 / ES;
  constexpr int KCH = D * ES / 16;
  constexpr int KSTEPS = D / 16;
  constexpr int NQS = BQ / 32;  // 32-query sub-tiles per q tile
  constexpr int DT = D / 32;
  constexpr int GROUPS = (BQ / 4) * KCH;  // 4-row x 1-chunk load groups per tensor
  constexpr int GLOADS = (GROUPS + NT - 1) / NT;
  using RTile = LdsTile<T, BQ, D, 0>;  // Q / dO row-major, rows read via perm23
  using TTile = LdsTile<T, D, BQ, 1>;  // Q^T / dO^T
  static_assert(D % 32 == 0 && BQ % 32 == 0, "tile shape");

  __shared__ __attribute__((aligned(16))) char lds_q[RTile::kBytes];
  __shared__ __attribute__((aligned(16))) char lds_do[RTile::kBytes];
  __shared__ __attribute__((aligned(16))) char lds_qt[TTile::kBytes];
  __shared__ __attribute__((aligned(16))) char lds_dot[TTile::kBytes];
  __shared__ __attribute__((aligned(16))) float lds_lse[BQ];
  __shared__ __attribute__((aligned(16))) float lds_dl[BQ];

  const Problem& P = a.p;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int lr = lane & 31, hh = lane >> 5;
  const int nkt = (P.Skv + BKV - 1) / BKV;
  const int g = P.Hq / P.Hkv;
  int head, kt;
  work_item(blockIdx.x, P.B * P.Hkv, nkt, P.xcd_remap, P.head_group_kv, true, &head, &kt);
  const int b = head / P.Hkv, hk = head - b * P.Hkv;
  const int k0 = kt * BKV;
  const int kw = k0 + 32 * w + lr;  // this lane's key (as B-operand column)
  const bool kvalid = kw < P.Skv;

  const T* kp = static_cast<const T*>(a.k) + ((size_t)head * P.Skv) * D;
  const T* vp = static_cast<const T*>(a.v) + ((size_t)head * P.Skv) * D;
  frag kf[KSTEPS], vf[KSTEPS];
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s) {
    kf[s] = ld_frag<T>(kp + (size_t)kw * D + 16 * s + 8 * hh, kvalid);
    vf[s] = ld_frag<T>(vp + (size_t)kw * D + 16 * s + 8 * hh, kvalid);
  }
  const int kdoc = (P.q_doc && kvalid) ? P.kv_doc[(size_t)b * P.Skv + kw] : 0;

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

  u32x4 qst[GLOADS][4], dst[GLOADS][4];
  float lse_st = 0.f, dl_st = 0.f;
  auto gload = [&](int it) {
    int hq, qbase;
    bool msk;
    walk.get(it, &hq, &qbase, &msk);
    const size_t hoff = ((size_t)(b * P.Hq + hq) * P.Sq) * D;
    const T* qp = static_cast<const T*>(a.q) + hoff;
    const T* dp = static_cast<const T*>(a.dout) + hoff;
#pragma unroll
    for (int u = 0; u < GLOADS; ++u) {
      const int gi = tid + NT * u;
      const int rg = gi / KCH, c = gi - rg * KCH;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int qi = qbase + 4 * rg + r;
        const bool ok = gi < GROUPS && qi < P.Sq;
        qst[u][r] = ld16(qp + (size_t)qi * D + c * EPC, ok);
        dst[u][r] = ld16(dp + (size_t)qi * D + c * EPC, ok);
      }
    }
    if (tid < BQ) {
      const int qi = qbase + tid;
      const size_t ri = (size_t)(b * P.Hq + hq) * P.Sq + qi;
      // rows past Sq and rows with no live key (LSE = -inf): P = 0
      const float l = qi < P.Sq ? a.lse[ri] : -INFINITY;
      lse_st = l > -INFINITY ? l * kLog2e : INFINITY;
      dl_st = qi < P.Sq ? a.delta[ri] : 0.f;
    }
  };
  auto lds_store = [&]() {
#pragma unroll
    for (int u = 0; u < GLOADS; ++u) {
      const int gi = tid + NT * u;
      const int rg = gi / KCH, c = gi - rg * KCH;
      if (gi < GROUPS) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          *reinterpret_cast<u32x4*>(lds_q + RTile::off(4 * rg + r, c)) = qst[u][r];
          *reinterpret_cast<u32x4*>(lds_do + RTile::off(4 * rg + r, c)) = dst[u][r];
        }
        write_transposed4<TTile, T>(lds_qt, qst[u], 4 * rg, c * EPC);
        write_transposed4<TTile, T>(lds_dot, dst[u], 4 * rg, c * EPC);
      }
    }
    if (tid < BQ) {
      lds_lse[tid] = lse_st;
      lds_dl[tid] = dl_st;
    }
  };

  f32x16 dka[DT], dva[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) dka[i][e] = dva[i][e] = 0.f;

  if (n_it > 0) gload(0);
  for (int it = 0; it < n_it; ++it) {
    int hq, qbase;
    bool masked;
    walk.get(it, &hq, &qbase, &masked);
    __syncthreads();
    lds_store();
    __syncthreads();
    if (it + 1 < n_it) gload(it + 1);
    if (qbase >= P.Sq) continue;  // workgroup-uniform
    masked = masked || (k0 + BKV > P.Skv);
    const float slope = P.alibi ? P.alibi[hq] : 0.f;

    f32x16 sacc[NQS], pacc[NQS];
#pragma unroll
    for (int j = 0; j < NQS; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[j][e] = pacc[j][e] = 0.f;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
      for (int j = 0; j < NQS; ++j) {
        const frag qa = RTile::read(lds_q, 32 * j + perm23(lr), 16 * s + 8 * hh);
        sacc[j] = E::mma(qa, kf[s], sacc[j]);
        const frag da = RTile::read(lds_do, 32 * j + perm23(lr), 16 * s + 8 * hh);
        pacc[j] = E::mma(da, vf[s], pacc[j]);
      }

    // P and dS, rows = queries acc_row(e), column = this lane's key
#pragma unroll
    for (int j = 0; j < NQS; ++j)
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int r0 = 32 * j + acc_row(4 * e4, hh);
        const f32x4 ls = *reinterpret_cast<const f32x4*>(&lds_lse[r0]);
        const f32x4 dl = *reinterpret_cast<const f32x4*>(&lds_dl[r0]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e = 4 * e4 + i;
          const int qi = qbase + r0 + i;
          float dsdx;
          float t = mod_score_t<Mod, kMods>(P, sacc[j][e], slope, b, hq, qi, kw, &dsdx);
          if (masked) {
            const bool ok = kvalid && qi < P.Sq && mod_mask_ok<Mod>(P, b, hq, qi, kw, q_doc_of(P, b, qi), kdoc);
            if (!ok) t = -INFINITY;
          }
          const float pv = fast_exp2(t - ls[i]);
          sacc[j][e] = pv;
          pacc[j][e] = pv * (pacc[j][e] - dl[i]) * dsdx;
        }
      }

    frag pf[BQ / 16], sf[BQ / 16];
#pragma unroll
    for (int c = 0; c < BQ / 16; ++c) {
      float x[8], y[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        x[t] = sacc[c >> 1][8 * (c & 1) + t];
        y[t] = pacc[c >> 1][8 * (c & 1) + t];
      }
      pf[c] = E::pack(x);
      sf[c] = E::pack(y);
    }
#pragma unroll
    for (int i = 0; i < DT; ++i)
#pragma unroll
      for (int c = 0; c < BQ / 16; ++c) {
        const frag dta = TTile::read(lds_dot, 32 * i + lr, 16 * c + 8 * hh);
        dva[i] = E::mma(dta, pf[c], dva[i]);
        const frag qta = TTile::read(lds_qt, 32 * i + lr, 16 * c + 8 * hh);
        dka[i] = E::mma(qta, sf[c], dka[i]);
      }
  }

  if (kvalid) {
    T* dkp = static_cast<T*>(a.dk) + ((size_t)head * P.Skv + kw) * D;
    T* dvp = static_cast<T*>(a.dv) + ((size_t)head * P.Skv + kw) * D;
#pragma unroll
    for (int i = 0; i < DT; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d0 = 32 * i + 8 * j + 4 * hh;
        const float k0v = dka[i][4 * j] * P.scale, k1v = dka[i][4 * j + 1] * P.scale;
        const float k2v = dka[i][4 * j + 2] * P.scale, k3v = dka[i][4 * j + 3] * P.scale;
        if constexpr (sizeof(T) == 2) {
          *reinterpret_cast<u32x2*>(dkp + d0) = u32x2{pack_bf16x2(k0v, k1v), pack_bf16x2(k2v, k3v)};
          *reinterpret_cast<u32x2*>(dvp + d0) =
              u32x2{pack_bf16x2(dva[i][4 * j], dva[i][4 * j + 1]), pack_bf16x2(dva[i][4 * j + 2], dva[i][4 * j + 3])};
        } else {
          *reinterpret_cast<f32x4*>(dkp + d0) = f32x4{k0v, k1v, k2v, k3v};
          *reinterpret_cast<f32x4*>(dvp + d0) = f32x4{dva[i][4 * j], dva[i][4 * j + 1], dva[i][4 * j + 2], dva[i][4 * j + 3]};
        }
      }
  }
}

// -------------------------------------------------------------------- dQ ---
template <typename T, int D, int BN, int NW, bool kMods, class Mod = BuiltinMod>
__global__ __launch_bounds__(NW * 64) void dq_kernel(BwdArgs a) {
  using E = Elt<T>;
  using frag = typename E::frag;
  constexpr int BM = 32 * NW;
  constexpr int NT = NW * 64;
  constexpr int ES = sizeof(T);
  constexpr int EPC = 16 / ES;
  constexpr int KCH = D * ES / 16;
  constexpr int KSTEPS = D / 16;
  constexpr int NSUB = BN / 32;
  constexpr int DT = D / 32;
  constexpr int GROUPS = (BN / 4) * KCH;
  constexpr int GLOADS = (GROUPS + NT - 1) / NT;
  using RTile = LdsTile<T, BN, D, 0>;  // K, V row-major (rows read via perm23)
  using TTile = LdsTile<T, D, BN, 1>;  // K^T
  static_assert(D % 32 == 0 && BN % 32 == 0, "tile shape");

  __shared__ __attribute__((aligned(16))) char lds_k[RTile::kBytes];
  __shared__ __attribute__((aligned(16))) char lds_v[RTile::kBytes];
  __shared__ __attribute__((aligned(16))) char lds_kt[TTile::kBytes];

  const Problem& P = a.p;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int lr = lane & 31, hh = lane >> 5;
  const int nqt = (P.Sq + BM - 1) / BM;
  int head, qt;
  work_item(blockIdx.x, P.B * P.Hq, nqt, P.xcd_remap, P.head_group_q, false, &head, &qt);
  const int b = head / P.Hq, h = head - b * P.Hq;
  const int hk = h / (P.Hq / P.Hkv);
  const int q0 = qt * BM;
  const int qw = q0 + 32 * w + lr;
  const bool qvalid = qw < P.Sq;

  const size_t qoff = ((size_t)head * P.Sq) * D;
  const T* qp = static_cast<const T*>(a.q) + qoff;
  const T* dop = static_cast<const T*>(a.dout) + qoff;
  const T* kp = static_cast<const T*>(a.k) + ((size_t)(b * P.Hkv + hk) * P.Skv) * D;
  const T* vp = static_cast<const T*>(a.v) + ((size_t)(b * P.Hkv + hk) * P.Skv) * D;

  frag qf[KSTEPS], df[KSTEPS];
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s) {
    qf[s] = ld_frag<T>(qp + (size_t)qw * D + 16 * s + 8 * hh, qvalid);
    df[s] = ld_frag<T>(dop + (size_t)qw * D + 16 * s + 8 * hh, qvalid);
  }
  const size_t rowi = (size_t)head * P.Sq + qw;
  // a row with no live key (LSE = -inf) gets P = 0 everywhere, like rows past Sq
  const float lse_row = qvalid ? a.lse[rowi] : -INFINITY;
  const float lse2 = lse_row > -INFINITY ? lse_row * kLog2e : INFINITY;
  const float dl = qvalid ? a.delta[rowi] : 0.f;
  const float slope = P.alibi ? P.alibi[h] : 0.f;
  const int qdoc = (P.q_doc && qvalid) ? P.q_doc[(size_t)b * P.Sq + qw] : 0;

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

  u32x4 kst[GLOADS][4], vst[GLOADS][4];
  auto gload = [&](int it) {
    int kbase;
    bool msk;
    walk.get(it, &kbase, &msk);
#pragma unroll
    for (int u = 0; u < GLOADS; ++u) {
      const int gi = tid + NT * u;
      const int rg = gi / KCH, c = gi - rg * KCH;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kbase + 4 * rg + r;
        const bool ok = gi < GROUPS && key < P.Skv;
        kst[u][r] = ld16(kp + (size_t)key * D + c * EPC, ok);
        vst[u][r] = ld16(vp + (size_t)key * D + c * EPC, ok);
      }
    }
  };
  auto lds_store = [&]() {
#pragma unroll
    for (int u = 0; u < GLOADS; ++u) {
      const int gi = tid + NT * u;
      const int rg = gi / KCH, c = gi - rg * KCH;
      if (gi < GROUPS) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          *reinterpret_cast<u32x4*>(lds_k + RTile::off(4 * rg + r, c)) = kst[u][r];
          *reinterpret_cast<u32x4*>(lds_v + RTile::off(4 * rg + r, c)) = vst[u][r];
        }
        write_transposed4<TTile, T>(lds_kt, kst[u], 4 * rg, c * EPC);
      }
    }
  };

  f32x16 dqa[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) dqa[i][e] = 0.f;

  if (n_it > 0) gload(0);
  for (int it = 0; it < n_it; ++it) {
    int kbase;
    bool masked;
    walk.get(it, &kbase, &masked);
    __syncthreads();
    lds_store();
    __syncthreads();
    if (it + 1 < n_it) gload(it + 1);
    if (kbase >= P.Skv) continue;  // workgroup-uniform
    masked = masked || (kbase + BN > P.Skv);

    f32x16 sacc[NSUB], pacc[NSUB];
#pragma unroll
    for (int j = 0; j < NSUB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[j][e] = pacc[j][e] = 0.f;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
      for (int j = 0; j < NSUB; ++j) {
        const frag ka = RTile::read(lds_k, 32 * j + perm23(lr), 16 * s + 8 * hh);
        sacc[j] = E::mma(ka, qf[s], sacc[j]);
        const frag va = RTile::read(lds_v, 32 * j + perm23(lr), 16 * s + 8 * hh);
        pacc[j] = E::mma(va, df[s], pacc[j]);
      }
#pragma unroll
    for (int j = 0; j < NSUB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = kbase + 32 * j + acc_row(e, hh);
        float dsdx;
        float t = mod_score_t<Mod, kMods>(P, sacc[j][e], slope, b, h, qw, key, &dsdx);
        if (masked && !(key < P.Skv && mod_mask_ok<Mod>(P, b, h, qw, key, qdoc, kv_doc_of(P, b, key)))) t = -INFINITY;
        const float pv = fast_exp2(t - lse2);
        pacc[j][e] = pv * (pacc[j][e] - dl) * dsdx;
      }
    frag sf[BN / 16];
#pragma unroll
    for (int c = 0; c < BN / 16; ++c) {
      float y[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) y[t] = pacc[c >> 1][8 * (c & 1) + t];
      sf[c] = E::pack(y);
    }
#pragma unroll
    for (int i = 0; i < DT; ++i)
#pragma unroll
      for (int c = 0; c < BN / 16; ++c) {
        const frag kta = TTile::read(lds_kt, 32 * i + lr, 16 * c + 8 * hh);
        dqa[i] = E::mma(kta, sf[c], dqa[i]);
      }
  }

  if (qvalid) {
    T* dqp = static_cast<T*>(a.dq) + rowi * D;
#pragma unroll
    for (int i = 0; i < DT; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d0 = 32 * i + 8 * j + 4 * hh;
        const float x0 = dqa[i][4 * j] * P.scale, x1 = dqa[i][4 * j + 1] * P.scale;
        const float x2 = dqa[i][4 * j + 2] * P.scale, x3 = dqa[i][4 * j + 3] * P.scale;
        if constexpr (sizeof(T) == 2) {
          *reinterpret_cast<u32x2*>(dqp + d0) = u32x2{pack_bf16x2(x0, x1), pack_bf16x2(x2, x3)};
        } else {
          *reinterpret_cast<f32x4*>(dqp + d0) = f32x4{x0, x1, x2, x3};
        }
      }
  }
}

}  // namespace fa
