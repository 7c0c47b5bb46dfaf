// Block-mask construction on the device for the mask descriptors of
// fa_params (a window on q - kv and/or equal document ids): the work of
// create_block_mask (block_mask.py:54-129) without a host pass over the tiles.
//
//   mb_block_docs  per block of each side: its document id when every token
//                  of the block shares one, else kMixedDoc;
//   mb_classify    per tile (one wave): the reference's 3x3 sampling rule
//                  (block_mask.py:85-109) and the exact live / full state.
//                  Windows are intervals on q - kv, so most tiles resolve from
//                  the tile's corners; with documents, tiles whose two blocks
//                  each lie in one document compare the two ids, a tile with
//                  one such block tests each element of the other block
//                  against the window's interval, and only tiles whose two
//                  blocks both cross a document boundary test every element;
//   mb_compact     per table row (one workgroup): ascending index lists of
//                  the selected tiles by a ballot scan, padded with -1, and
//                  the row's count folded into a running maximum.
//
// Tile flags (one byte per tile, row-major [row][i][j]): bit 0 live, bit 1
// full, bit 2 kept by the sampling rule.
#pragma once
#include <stdint.h>

#include <hip/hip_runtime.h>

namespace fa {

constexpr int kMixedDoc = INT32_MIN;

struct MaskBuild {
  int rows, q_len, kv_len, block, nq, nk;
  int left, right;  // < 0: unlimited
  const int32_t* doc;  // (rows, doc_len) or null
  int doc_len;
  int32_t* qdoc;       // (rows, nq) block documents (workspace)
  int32_t* kdoc;       // (rows, nk)
  uint8_t* flags;      // (rows, nq, nk)
};

__device__ __forceinline__ bool mb_window(const MaskBuild& m, int q, int k) {
  const int d = q - k;
  return (m.left < 0 || d <= m.left) && (m.right < 0 || -d <= m.right);
}

__device__ __forceinline__ bool mb_keep(const MaskBuild& m, const int32_t* doc_row, int q, int k) {
  return mb_window(m, q, k) && (doc_row == nullptr || doc_row[q] == doc_row[k]);
}

// grid: (rows, max(nq, nk)); one wave per block and side
__global__ __launch_bounds__(64) void mb_block_docs(MaskBuild m) {
  const int row = blockIdx.x, blk = blockIdx.y, lane = threadIdx.x;
  const int32_t* d = m.doc + (size_t)row * m.doc_len;
#pragma unroll
  for (int side = 0; side < 2; ++side) {
    const int n = side ? m.nk : m.nq;
    const int len = side ? m.kv_len : m.q_len;
    if (blk >= n) continue;
    const int a = blk * m.block, e = min(a + m.block, len);
    int lo = INT32_MAX, hi = INT32_MIN;
    for (int t = a + lane; t < e; t += 64) {
      lo = min(lo, d[t]);
      hi = max(hi, d[t]);
    }
    for (int o = 32; o >= 1; o >>= 1) {
      lo = min(lo, __shfl_xor(lo, o));
      hi = max(hi, __shfl_xor(hi, o));
    }
    if (lane == 0) (side ? m.kdoc : m.qdoc)[(size_t)row * n + blk] = lo == hi ? lo : kMixedDoc;
  }
}

constexpr int kMaxMaskBlock = 1024;

// grid: (rows, nq); 256 threads, wave w takes the tiles j = w, w + 4, ...
__global__ __launch_bounds__(256) void mb_classify(MaskBuild m) {
  __shared__ int kd_lds[4][kMaxMaskBlock];
  const int row = blockIdx.x, i = blockIdx.y;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int32_t* doc_row = m.doc ? m.doc + (size_t)row * m.doc_len : nullptr;
  const int qa = i * m.block, qe = min(qa + m.block, m.q_len);  // [qa, qe)
  const int qs[3] = {qa, (qa + qe) / 2, qe - 1};
  const int qd = doc_row ? m.qdoc[(size_t)row * m.nq + i] : 0;
  // window bounds on d = q - kv as a closed interval [lo, hi] (64-bit: no overflow)
  const long long lo = m.right >= 0 ? -(long long)m.right : LLONG_MIN / 2;
  const long long hi = m.left >= 0 ? (long long)m.left : LLONG_MAX / 2;
  for (int j = w; j < m.nk; j += 4) {
    const int ka = j * m.block, ke = min(ka + m.block, m.kv_len);
    const bool complete = qa + m.block <= m.q_len && ka + m.block <= m.kv_len;
    // sampling rule: 3 x 3 points, lanes 0..8
    bool samp = false;
    if (lane < 9) {
      const int ks[3] = {ka, (ka + ke) / 2, ke - 1};
      samp = mb_keep(m, doc_row, qs[lane / 3], ks[lane % 3]);
    }
    samp = __any(samp);
    // exact state
    const long long dmin = (long long)qa - (ke - 1), dmax = (long long)(qe - 1) - ka;
    const bool wlive = (dmin > lo ? dmin : lo) <= (dmax < hi ? dmax : hi);
    const bool wfull = dmin >= lo && dmax <= hi;
    bool live, full;
    if (!wlive) {
      live = full = false;
    } else if (!doc_row) {
      live = true;
      full = wfull && complete;
    } else {
      const int kd = m.kdoc[(size_t)row * m.nk + j];
      if (qd != kMixedDoc && kd != kMixedDoc) {
        live = qd == kd;
        full = live && wfull && complete;
      } else if (kd != kMixedDoc || qd != kMixedDoc) {
        // one block lies in one document: per element of the other block
        // (lanes take them), same id or not, and if so the window's interval
        // over the uniform block
        const bool q_side = kd != kMixedDoc;  // lanes walk the query rows
        const int uni = q_side ? kd : qd;
        const int a0 = q_side ? qa : ka, a1 = q_side ? qe : ke;  // walked block [a0, a1)
        const int b0 = q_side ? ka : qa, b1 = (q_side ? ke : qe) - 1;  // uniform block [b0, b1]
        bool any = false, all = complete;
        for (int r = lane; r < m.block; r += 64) {
          const int x = a0 + r;
          if (x >= a1) {
            all = false;
            continue;
          }
          if (doc_row[x] != uni) {
            all = false;
            continue;
          }
          // q rows see keys [q - left, q + right]; k columns are seen by rows [k - right, k + left]
          int lo_b = b0, hi_b = b1;
          const int below = q_side ? m.left : m.right, above = q_side ? m.right : m.left;
          if (below >= 0) lo_b = max(lo_b, x - below);
          if (above >= 0) hi_b = min(hi_b, x + above);
          any |= lo_b <= hi_b;
          all &= lo_b == b0 && hi_b == b1;
        }
        live = __any(any);
        full = live && __all(all);
      } else {
        // both blocks cross a document boundary: every element (a padded tile
        // element outside either sequence counts as masked).  The key block's
        // ids go to this wave's LDS row; each lane takes query rows and
        // compares the keys inside the row's window.
        int* kid = kd_lds[w];
        for (int t = lane; t < ke - ka; t += 64) kid[t] = doc_row[ka + t];
        __builtin_amdgcn_wave_barrier();
        bool any = false, all = complete;
        for (int r = lane; r < m.block; r += 64) {
          const int q = qa + r;
          if (q >= qe) {
            all = false;
            continue;
          }
          const int dq = doc_row[q];
          int k0 = ka, k1 = ke - 1;  // keys of the block inside q's window
          if (m.left >= 0) k0 = max(k0, q - m.left);
          if (m.right >= 0) k1 = min(k1, q + m.right);
          if (k0 > ka || k1 < ke - 1) all = false;
          for (int k = k0; k <= k1; ++k) {
            const bool same = kid[k - ka] == dq;
            any |= same;
            all &= same;
          }
        }
        __builtin_amdgcn_wave_barrier();
        live = __any(any);
        full = live && __all(all);
      }
    }
    if (lane == 0) m.flags[((size_t)row * m.nq + i) * m.nk + j] = (uint8_t)(live | (full << 1) | (samp << 2));
  }
}

// One table row per workgroup (256 threads): the entries e = 0 .. n - 1 of the
// row (tile flags at flags + e * stride) that satisfy `want` are listed in
// ascending order in out[0 .. count), the rest of out[0 .. n) is -1, num[0] =
// count, and *max_count = max(*max_count, count).
struct CompactList {
  int32_t* num;
  int32_t* idx;
  int32_t* max_count;
  uint8_t sel_mask, sel_value;  // entry selected iff (flag & sel_mask) == sel_value
};

__device__ __forceinline__ void mb_compact_row(const uint8_t* flags, long long stride, int n, const CompactList& L,
                                               size_t row_off_num, size_t row_off_idx) {
  __shared__ int wave_tot[4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int base = 0;
  for (int c = 0; c < n; c += 256) {
    const int e = c + tid;
    const bool sel = e < n && (flags[(long long)e * stride] & L.sel_mask) == L.sel_value;
    const unsigned long long bal = __ballot(sel);
    const int before = __popcll(bal & ((1ull << lane) - 1ull));
    if (lane == 0) wave_tot[w] = __popcll(bal);
    __syncthreads();
    int off = base;
    for (int x = 0; x < w; ++x) off += wave_tot[x];
    const int tot = wave_tot[0] + wave_tot[1] + wave_tot[2] + wave_tot[3];
    if (sel) L.idx[row_off_idx + off + before] = e;
    base += tot;
    __syncthreads();
  }
  for (int e = base + tid; e < n; e += 256) L.idx[row_off_idx + e] = -1;
  if (tid == 0) {
    L.num[row_off_num] = base;
    atomicMax(L.max_count, base);
  }
}

// grid: (rows, nq + nk, 5 lists); list 0..2 walk kv rows (sampled, partial,
// full), lists 3..4 walk q columns (partial, full)
struct CompactArgs {
  MaskBuild m;
  CompactList lists[5];
};

__global__ __launch_bounds__(256) void mb_compact(CompactArgs a) {
  const MaskBuild& m = a.m;
  const int row = blockIdx.x, r = blockIdx.y, which = blockIdx.z;
  const CompactList& L = a.lists[which];
  if (which < 3) {
    if (r >= m.nq) return;
    const uint8_t* f = m.flags + ((size_t)row * m.nq + r) * m.nk;
    mb_compact_row(f, 1, m.nk, L, (size_t)row * m.nq + r, ((size_t)row * m.nq + r) * m.nk);
  } else {
    if (r >= m.nk) return;
    const uint8_t* f = m.flags + (size_t)row * m.nq * m.nk + r;
    mb_compact_row(f, m.nk, m.nq, L, (size_t)row * m.nk + r, ((size_t)row * m.nk + r) * m.nq);
  }
}

__global__ void mb_zero(int32_t* p, int n) {
  if ((int)threadIdx.x < n) p[threadIdx.x] = 0;
}

}  // namespace fa
