// Drives the host twins (fa_*_host) over small problems with every mask kind,
// GQA, ragged lengths, document labels and block tables, so that a build
// with AddressSanitizer / UndefinedBehaviorSanitizer checks their index
// arithmetic.  Prints "ok <n>" after n problems; any sanitizer report aborts.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "flexattn.h"

static float frand(unsigned* s) {
  *s = *s * 1664525u + 1013904223u;
  return ((*s >> 8) & 0xffff) / 32768.0f - 1.0f;
}

static uint16_t to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

struct Case {
  int B, Hq, Hkv, Sq, Skv, D, dtype, wl, wr, docs, tables, alibi;
  float softcap;
};

static int run(const Case& c, unsigned seed) {
  const size_t es = c.dtype == FA_DTYPE_BF16 ? 2 : 4;
  const size_t nq = (size_t)c.B * c.Hq * c.Sq * c.D, nk = (size_t)c.B * c.Hkv * c.Skv * c.D;
  std::vector<unsigned char> q(nq * es), k(nk * es), v(nk * es), o(nq * es), dout(nq * es), dq(nq * es),
      dk(nk * es), dv(nk * es);
  auto fill = [&](std::vector<unsigned char>& x, size_t n) {
    for (size_t i = 0; i < n; ++i) {
      const float f = frand(&seed);
      if (es == 2) {
        const uint16_t h = to_bf16(f);
        std::memcpy(&x[2 * i], &h, 2);
      } else {
        std::memcpy(&x[4 * i], &f, 4);
      }
    }
  };
  fill(q, nq);
  fill(k, nk);
  fill(v, nk);
  fill(dout, nq);
  std::vector<float> lse((size_t)c.B * c.Hq * c.Sq), slopes(c.Hq);
  for (int h = 0; h < c.Hq; ++h) slopes[h] = std::pow(2.0f, -8.0f * (h + 1) / c.Hq);
  fa_params p;
  std::memset(&p, 0, sizeof p);
  p.abi_version = FA_ABI_VERSION;
  p.dtype = c.dtype;
  p.B = c.B, p.Hq = c.Hq, p.Hkv = c.Hkv, p.Sq = c.Sq, p.Skv = c.Skv, p.D = c.D;
  p.window_left = c.wl, p.window_right = c.wr;
  p.softcap = c.softcap;
  if (c.alibi) p.alibi_slopes = slopes.data();
  std::vector<int32_t> qd((size_t)c.B * c.Sq), kd((size_t)c.B * c.Skv);
  if (c.docs) {
    for (auto& x : qd) x = (int)(frand(&seed) * 2 + 2);
    for (auto& x : kd) x = (int)(frand(&seed) * 2 + 2);
    p.q_doc_ids = qd.data();
    p.kv_doc_ids = kd.data();
  }
  // block tables at 64: every kv block partial for even q blocks, the first
  // half full and the rest partial for odd ones, plus out-of-range entries
  const int blk = 64, nqb = (c.Sq + blk - 1) / blk, nkb = (c.Skv + blk - 1) / blk;
  std::vector<int32_t> knum(nqb), kidx((size_t)nqb * (nkb + 1)), fnum(nqb), fidx((size_t)nqb * (nkb + 1));
  if (c.tables) {
    for (int i = 0; i < nqb; ++i) {
      int np = 0, nf = 0;
      for (int j = 0; j < nkb; ++j) {
        if ((i & 1) && j < nkb / 2) fidx[(size_t)i * (nkb + 1) + nf++] = j;
        else kidx[(size_t)i * (nkb + 1) + np++] = j;
      }
      kidx[(size_t)i * (nkb + 1) + np++] = nkb + 7;  // skipped
      knum[i] = np + 3;                               // clamped to the width
      fnum[i] = nf;
    }
    p.mask_block_q = p.mask_block_kv = blk;
    p.table_b = p.table_h = 1;
    p.kv_width = nkb + 1;
    p.kv_num_blocks = knum.data(), p.kv_indices = kidx.data();
    p.full_kv_num_blocks = fnum.data(), p.full_kv_indices = fidx.data();
  }
  int rc = fa_fwd_host(&p, q.data(), k.data(), v.data(), o.data(), lse.data(), 2);
  if (!rc) rc = fa_bwd_host(&p, q.data(), k.data(), v.data(), o.data(), lse.data(), dout.data(), dq.data(), dk.data(),
                            dv.data(), 3);
  return rc;
}

int main() {
  const Case cases[] = {
      {1, 2, 2, 64, 64, 32, FA_DTYPE_F32, -1, 0, 0, 0, 0, 0.f},
      {2, 4, 2, 77, 130, 64, FA_DTYPE_BF16, -1, -1, 0, 0, 1, 20.f},
      {1, 3, 1, 200, 150, 16, FA_DTYPE_F32, 20, 5, 1, 0, 0, 0.f},
      {2, 2, 2, 190, 190, 48, FA_DTYPE_BF16, -1, 0, 0, 1, 0, 0.f},
      {1, 4, 4, 1, 300, 128, FA_DTYPE_BF16, -1, -1, 0, 1, 1, 0.f},
      {1, 1, 1, 33, 1, 8, FA_DTYPE_F32, 0, 0, 1, 1, 0, 5.f},
  };
  int n = 0;
  for (const Case& c : cases) {
    const int rc = run(c, 1234u + n);
    if (rc) {
      std::printf("case %d failed: %d\n", n, rc);
      return 1;
    }
    ++n;
  }
  std::printf("ok %d\n", n);
  return 0;
}
