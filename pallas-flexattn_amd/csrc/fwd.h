// Forward FlexAttention kernel for gfx950.
//
// One workgroup = NW waves = one tile of BM = 32*NW query rows of one
// (batch, q-head).  Each wave owns 32 query rows for the whole kv loop:
//   * its Q rows sit in registers as the B operand of S^T = K Q^T,
//   * S^T (keys x queries) comes out with one query per lane, so the online
//     softmax row statistics are per-lane scalars plus one exchange between
//     the two lane halves,
//   * P^T is re-packed in registers as the B operand of O^T += V^T P^T.
// K (rows = keys) and V^T (rows = head dim) tiles of BN keys are staged in
// swizzled LDS; the next tile's global loads are issued before the current
// tile's MFMAs (register double buffering).
// The kv loop walks the block tables: fully-live blocks first (no element
// mask), then partial blocks (mask evaluated per element).
#pragma once
#include "dma.h"
#include "kargs.h"

namespace fa {

struct FwdArgs {
  Problem p;
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;  // (B, Hq, Sq), natural-log units
  // Split-KV (n_splits > 1, bf16 DMA kernel only): workgroup blockIdx.x takes
  // split blockIdx.x / items of its item's walk and writes, instead of o and
  // lse, its unnormalised partial O (relative to 2^m) and (m, l) to `part`:
  // (n_splits, B*Hq*Sq, D) floats, then (n_splits, B*Hq*Sq, 2).
  int n_splits = 1;
  float* part = nullptr;
  // bf16 DMA kernel only:
  // GQA row packing (pack > 1): a work item is (batch, kv head, BM rows) of
  // the g = Hq / Hkv query heads' rows taken as one sequence of g * Sq rows
  // (row r: q head hk * g + r / Sq, query r % Sq; in memory these rows are
  // contiguous), so a K / V tile serves the whole group.  For short Sq (decode).
  int pack = 0;
  // Paged K / V: k, v are (num_pages, Hkv, page_size, D) caches and key t of
  // batch row b sits in page page_table[b * max_pages + t / page_size].
  const int* page_table = nullptr;
  int page_size = 0, max_pages = 0, num_pages = 0;
  // Keys of batch row b are [0, kv_lens[b]) (each <= Skv); null: all Skv.
  const int* kv_lens = nullptr;
};

using KvWalk = KvWalkT<DeviceLoad>;

// A kv walk's block indices held in one register: lane i holds entry e0 + i
// of the row (full list first), reloaded every 64 entries, so the tiles make
// no table loads (a load consumed by the walk would also wait for every copy
// issued before it).
struct KvTab {
  int e0 = -64, reg = 0;
  __device__ __forceinline__ void load(const KvWalk& w, int first, int lane) {
    const int e = first + lane;  // past a list's end the loads return 0 (never read)
    const int vf = vload_i32(w.full, e, w.nfull);
    const int vp = vload_i32(w.part, e - w.nfull, w.npart);
    reg = e < w.nfull ? vf : vp;
    e0 = first;
  }
  // first key of tile it (wave-uniform)
  __device__ __forceinline__ int kbase(const KvWalk& w, int it, int sub_log2, int lane) {
    if (w.dense) return it * w.bn;
    const int bi = div_pow2_or(it, w.sub, sub_log2);
    if (bi - e0 >= 64 || bi < e0) load(w, bi & ~63, lane);
    return tile_start(__builtin_amdgcn_readlane(reg, bi - e0), w.nblk, w.mblk, it - bi * w.sub, w.bn);
  }
};

template <typename T, int D, int BN, int NW, bool kMods, class Mod = BuiltinMod>
__global__ __launch_bounds__(NW * 64) void fwd_kernel(FwdArgs a) {
  using E = Elt<T>;
  using frag = typename E::frag;
  constexpr int BM = 32 * NW;
  constexpr int NT = NW * 64;
  constexpr int ES = sizeof(T);
  constexpr int EPC = 16 / ES;           // elements per 16-byte chunk
  constexpr int KCH = D * ES / 16;       // chunks per K row
  constexpr int KSTEPS = D / 16;
  constexpr int NSUB = BN / 32;
  constexpr int DT = D / 32;
  constexpr int KLOADS = (BN * KCH + NT - 1) / NT;
  constexpr int VGROUPS = (BN / 4) * KCH;
  constexpr int VLOADS = (VGROUPS + NT - 1) / NT;
  using KTile = LdsTile<T, BN, D, 0>;
  using VTile = LdsTile<T, D, BN, 1>;
  static_assert(D % 32 == 0 && BN % 32 == 0, "tile shape");

  __shared__ __attribute__((aligned(16))) char lds_k[KTile::kBytes];
  __shared__ __attribute__((aligned(16))) char lds_v[VTile::kBytes];

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

  const T* qp = static_cast<const T*>(a.q) + ((size_t)head * P.Sq) * D;
  const T* kp = static_cast<const T*>(a.k) + ((size_t)(b * P.Hkv + hk) * P.Skv) * D;
  const T* vp = static_cast<const T*>(a.v) + ((size_t)(b * P.Hkv + hk) * P.Skv) * D;

  frag qf[KSTEPS];
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s) qf[s] = ld_frag<T>(qp + (size_t)qw * D + 16 * s + 8 * hh, qvalid);

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

  u32x4 kst[KLOADS];
  u32x4 vst[VLOADS][4];
  auto gload = [&](int it) {
    int kbase;
    bool msk;
    walk.get(it, &kbase, &msk);
#pragma unroll
    for (int u = 0; u < KLOADS; ++u) {
      const int g = tid + NT * u;
      const int row = g / KCH, c = g - row * KCH;
      const int key = kbase + row;
      kst[u] = ld16(kp + (size_t)key * D + c * EPC, row < BN && key < P.Skv);
    }
#pragma unroll
    for (int u = 0; u < VLOADS; ++u) {
      const int g = tid + NT * u;
      const int kg = g / KCH, c = g - kg * KCH;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kbase + 4 * kg + r;
        vst[u][r] = ld16(vp + (size_t)key * D + c * EPC, g < VGROUPS && key < P.Skv);
      }
    }
  };
  auto lds_store = [&]() {
#pragma unroll
    for (int u = 0; u < KLOADS; ++u) {
      const int g = tid + NT * u;
      const int row = g / KCH, c = g - row * KCH;
      if (row < BN) *reinterpret_cast<u32x4*>(lds_k + KTile::off(row, c)) = kst[u];
    }
#pragma unroll
    for (int u = 0; u < VLOADS; ++u) {
      const int g = tid + NT * u;
      const int kg = g / KCH, c = g - kg * KCH;
      if (g < VGROUPS) write_transposed4<VTile, T>(lds_v, vst[u], 4 * kg, c * EPC);
    }
  };

  f32x16 oacc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[i][e] = 0.f;
  float m = -INFINITY, l = 0.f;

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

    f32x16 sacc[NSUB];
#pragma unroll
    for (int j = 0; j < NSUB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[j][e] = 0.f;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
      for (int j = 0; j < NSUB; ++j) {
        const frag kf = KTile::read(lds_k, 32 * j + perm23(lr), 16 * s + 8 * hh);
        sacc[j] = E::mma(kf, qf[s], sacc[j]);
      }

    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < NSUB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = kbase + 32 * j + acc_row(e, hh);
        float t = mod_score_t<Mod, kMods>(P, sacc[j][e], slope, b, h, qw, key, nullptr);
        if (masked && !(key < P.Skv && mod_mask_ok<Mod>(P, b, h, qw, key, qdoc, kv_doc_of(P, b, key)))) t = -INFINITY;
        sacc[j][e] = t;
        mx = fmaxf(mx, t);
      }
    mx = fmaxf(mx, xor32(mx));
    const float mnew = fmaxf(m, mx);
    const float muse = (mnew == -INFINITY) ? 0.f : mnew;
    const float alpha = fast_exp2(m - muse);
    float rs = 0.f;
#pragma unroll
    for (int j = 0; j < NSUB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float pv = fast_exp2(sacc[j][e] - muse);
        sacc[j][e] = pv;
        rs += pv;
      }
    l = l * alpha + rs;
    m = mnew;
#pragma unroll
    for (int i = 0; i < DT; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) oacc[i][e] *= alpha;

    frag pf[BN / 16];
#pragma unroll
    for (int c = 0; c < BN / 16; ++c) {
      float x[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) x[t] = sacc[c >> 1][8 * (c & 1) + t];
      pf[c] = E::pack(x);
    }
#pragma unroll
    for (int i = 0; i < DT; ++i)
#pragma unroll
      for (int c = 0; c < BN / 16; ++c) {
        const frag vf = VTile::read(lds_v, 32 * i + lr, 16 * c + 8 * hh);
        oacc[i] = E::mma(vf, pf[c], oacc[i]);
      }
  }

  const float lt = l + xor32(l);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  if (qvalid) {
    T* op = static_cast<T*>(a.o) + ((size_t)head * P.Sq + qw) * D;
#pragma unroll
    for (int i = 0; i < DT; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d0 = 32 * i + 8 * j + 4 * hh;
        const float x0 = oacc[i][4 * j] * inv, x1 = oacc[i][4 * j + 1] * inv;
        const float x2 = oacc[i][4 * j + 2] * inv, x3 = oacc[i][4 * j + 3] * inv;
        if constexpr (sizeof(T) == 2) {
          *reinterpret_cast<u32x2*>(op + d0) = u32x2{pack_bf16x2(x0, x1), pack_bf16x2(x2, x3)};
        } else {
          *reinterpret_cast<f32x4*>(op + d0) = f32x4{x0, x1, x2, x3};
        }
      }
    if (hh == 0) a.lse[(size_t)head * P.Sq + qw] = lt > 0.f ? (m + log2f(lt)) * kLn2 : -INFINITY;
  }
}

}  // namespace fa
