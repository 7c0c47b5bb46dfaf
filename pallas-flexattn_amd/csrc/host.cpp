// Host execution of the attention path on host memory: the counterpart of the
// reference's interpret=True (its Pallas kernels run by the interpreter on
// the CPU, flash_attn.py:121,156,182,197,270,304,373,401).  Same fa_params,
// same results up to summation order: scores, softmax and products in fp32,
// with the GPU kernels' bf16 roundings for bf16 tensors (P before P V, dS
// before dS K / dS^T Q, the stored outputs).  Plain C++ threads over heads;
// no GPU is touched.  Not a fallback: the GPU entry points never call it.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/flexattn.h"

namespace {

struct Prob {
  const fa_params* p;
  bool bf16;
  float scale;
  int g;          // q heads per kv head
  int nqb, nkb;   // mask blocks along q / kv (tables only)
  bool tables;
};

float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

uint16_t f32_to_bf16(float f) {  // round to nearest even; NaN stays NaN
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// row `r` of a (heads, rows, D) tensor as fp32
void load_row(const void* base, bool bf16, size_t row, int D, float* out) {
  if (bf16) {
    const uint16_t* s = static_cast<const uint16_t*>(base) + row * D;
    for (int d = 0; d < D; ++d) out[d] = bf16_to_f32(s[d]);
  } else {
    std::memcpy(out, static_cast<const float*>(base) + row * D, sizeof(float) * D);
  }
}

void store_row(void* base, bool bf16, size_t row, int D, const float* in) {
  if (bf16) {
    uint16_t* d16 = static_cast<uint16_t*>(base) + row * D;
    for (int d = 0; d < D; ++d) d16[d] = f32_to_bf16(in[d]);
  } else {
    std::memcpy(static_cast<float*>(base) + row * D, in, sizeof(float) * D);
  }
}

int validate(const fa_params* p, Prob* pr) {
  if (!p) return FA_ERR_NULL;
  if (p->abi_version != FA_ABI_VERSION) return FA_ERR_VERSION;
  if (p->dtype != FA_DTYPE_BF16 && p->dtype != FA_DTYPE_F32) return FA_ERR_DTYPE;
  if (p->B < 1 || p->Hq < 1 || p->Hkv < 1 || p->Sq < 1 || p->Skv < 1 || p->D < 1 || p->D > 1024) return FA_ERR_SHAPE;
  if (p->Hq % p->Hkv) return FA_ERR_SHAPE;
  if (!(p->softcap >= 0.f) || !(p->scale >= 0.f)) return FA_ERR_SHAPE;
  if ((p->q_doc_ids == nullptr) != (p->kv_doc_ids == nullptr)) return FA_ERR_NULL;
  pr->p = p;
  pr->bf16 = p->dtype == FA_DTYPE_BF16;
  pr->scale = p->scale > 0.f ? p->scale : 1.0f / std::sqrt((float)p->D);
  pr->g = p->Hq / p->Hkv;
  pr->tables = p->kv_num_blocks || p->full_kv_num_blocks;
  pr->nqb = pr->nkb = 0;
  if (pr->tables) {
    if ((p->kv_num_blocks == nullptr) != (p->kv_indices == nullptr)) return FA_ERR_TABLES;
    if ((p->full_kv_num_blocks == nullptr) != (p->full_kv_indices == nullptr)) return FA_ERR_TABLES;
    if (p->mask_block_q < 1 || p->mask_block_kv < 1 || p->kv_width < 0) return FA_ERR_TABLES;
    if (p->table_b != 1 && p->table_b != p->B) return FA_ERR_TABLES;
    if (p->table_h != 1 && p->table_h != p->Hq) return FA_ERR_TABLES;
    pr->nqb = (p->Sq + p->mask_block_q - 1) / p->mask_block_q;
    pr->nkb = (p->Skv + p->mask_block_kv - 1) / p->mask_block_kv;
  }
  return FA_OK;
}

// Per-kv-block state for query block qb of head (b, h): 0 skipped, 1 partial
// (element mask), 2 full (no element mask).  Without tables every block is
// partial (the element mask decides).
void block_states(const Prob& pr, int b, int h, int qb, std::vector<uint8_t>* st) {
  const fa_params* p = pr.p;
  if (!pr.tables) {
    st->assign(1, 1);
    return;
  }
  st->assign(pr.nkb, 0);
  const int tb = p->table_b == 1 ? 0 : b, th = p->table_h == 1 ? 0 : h;
  const size_t row = ((size_t)tb * (p->table_h < 1 ? 1 : p->table_h) + th) * pr.nqb + qb;
  auto walk = [&](const int32_t* num, const int32_t* idx, uint8_t state) {
    if (!num) return;
    const int n = std::max(0, std::min(num[row], p->kv_width));
    for (int t = 0; t < n; ++t) {
      const int kb = idx[row * p->kv_width + t];
      if (kb >= 0 && kb < pr.nkb && (*st)[kb] == 0) (*st)[kb] = state;
    }
  };
  walk(p->full_kv_num_blocks, p->full_kv_indices, 2);
  walk(p->kv_num_blocks, p->kv_indices, 1);
}

bool elem_ok(const fa_params* p, int b, int i, int j) {
  if (p->window_left >= 0 && i - j > p->window_left) return false;
  if (p->window_right >= 0 && j - i > p->window_right) return false;
  if (p->q_doc_ids && p->q_doc_ids[(size_t)b * p->Sq + i] != p->kv_doc_ids[(size_t)b * p->Skv + j]) return false;
  return true;
}

// Scores of query row i against every key of head (b, h) into s (-inf where
// dead) and d score' / d score into dsds; returns whether any key is live.
bool row_scores(const Prob& pr, int b, int h, int i, const float* qi, const float* kh, const std::vector<uint8_t>& st,
                float* s, float* dsds) {
  const fa_params* p = pr.p;
  const int D = p->D;
  const float slope = p->alibi_slopes ? p->alibi_slopes[h] : 0.f;
  bool any = false;
  for (int j = 0; j < p->Skv; ++j) {
    const uint8_t state = pr.tables ? st[j / p->mask_block_kv] : 1;
    if (state == 0 || (state == 1 && !elem_ok(p, b, i, j))) {
      s[j] = -INFINITY;
      dsds[j] = 0.f;
      continue;
    }
    const float* kj = kh + (size_t)j * D;
    float acc = 0.f;
    for (int d = 0; d < D; ++d) acc += qi[d] * kj[d];
    float x = acc * pr.scale + slope * (float)(j - i);
    float dd = 1.f;
    if (p->softcap > 0.f) {
      const float t = std::tanh(x / p->softcap);
      x = p->softcap * t;
      dd = 1.f - t * t;
    }
    s[j] = x;
    dsds[j] = dd;
    any = true;
  }
  return any;
}

template <class F>
void parallel_for(int n, int nthreads, F&& fn) {
  int nt = nthreads > 0 ? nthreads : (int)std::max(1u, std::thread::hardware_concurrency());
  nt = std::min(nt, n);
  if (nt <= 1) {
    for (int i = 0; i < n; ++i) fn(i);
    return;
  }
  std::vector<std::thread> ts;
  for (int t = 0; t < nt; ++t)
    ts.emplace_back([&, t]() {
      for (int i = t; i < n; i += nt) fn(i);
    });
  for (auto& th : ts) th.join();
}

// Whole (B * H, rows, D) tensor of head (b, h) as fp32
std::vector<float> load_head(const void* base, bool bf16, size_t head, int rows, int D) {
  std::vector<float> out((size_t)rows * D);
  for (int r = 0; r < rows; ++r) load_row(base, bf16, head * rows + r, D, out.data() + (size_t)r * D);
  return out;
}

}  // namespace

extern "C" {

int fa_fwd_host(const fa_params* p, const void* q, const void* k, const void* v, void* o, float* lse, int nthreads) {
  Prob pr;
  int rc = validate(p, &pr);
  if (rc) return rc;
  if (!q || !k || !v || !o || !lse) return FA_ERR_NULL;
  const int D = p->D, Sq = p->Sq, Skv = p->Skv;
  parallel_for(p->B * p->Hq, nthreads, [&](int head) {
    const int b = head / p->Hq, h = head - b * p->Hq, hk = b * p->Hkv + h / pr.g;
    const std::vector<float> kh = load_head(k, pr.bf16, hk, Skv, D), vh = load_head(v, pr.bf16, hk, Skv, D);
    std::vector<float> qi(D), s(Skv), dsds(Skv), oi(D);
    std::vector<uint8_t> st;
    int cur_qb = -1;
    for (int i = 0; i < Sq; ++i) {
      const int qb = pr.tables ? i / p->mask_block_q : 0;
      if (qb != cur_qb) {
        block_states(pr, b, h, qb, &st);
        cur_qb = qb;
      }
      load_row(q, pr.bf16, (size_t)head * Sq + i, D, qi.data());
      std::fill(oi.begin(), oi.end(), 0.f);
      float m = -INFINITY, l = 0.f;
      if (row_scores(pr, b, h, i, qi.data(), kh.data(), st, s.data(), dsds.data())) {
        for (int j = 0; j < Skv; ++j) m = std::max(m, s[j]);
        for (int j = 0; j < Skv; ++j) {
          if (s[j] == -INFINITY) continue;
          const float pj = std::exp(s[j] - m);
          l += pj;
          const float pc = pr.bf16 ? round_bf16(pj) : pj;
          const float* vj = vh.data() + (size_t)j * D;
          for (int d = 0; d < D; ++d) oi[d] += pc * vj[d];
        }
      }
      const float inv = l > 0.f ? 1.f / l : 0.f;
      for (int d = 0; d < D; ++d) oi[d] *= inv;
      store_row(o, pr.bf16, (size_t)head * Sq + i, D, oi.data());
      lse[(size_t)head * Sq + i] = l > 0.f ? m + std::log(l) : -INFINITY;
    }
  });
  return FA_OK;
}

int fa_bwd_preprocess_host(const fa_params* p, const void* o, const void* dout, float* delta, int nthreads) {
  Prob pr;
  int rc = validate(p, &pr);
  if (rc) return rc;
  if (!o || !dout || !delta) return FA_ERR_NULL;
  const int D = p->D, Sq = p->Sq;
  parallel_for(p->B * p->Hq, nthreads, [&](int head) {
    std::vector<float> oi(D), di(D);
    for (int i = 0; i < Sq; ++i) {
      const size_t r = (size_t)head * Sq + i;
      load_row(o, pr.bf16, r, D, oi.data());
      load_row(dout, pr.bf16, r, D, di.data());
      float acc = 0.f;
      for (int d = 0; d < D; ++d) acc += oi[d] * di[d];
      delta[r] = acc;
    }
  });
  return FA_OK;
}

int fa_bwd_dkdv_host(const fa_params* p, const void* q, const void* k, const void* v, const void* dout,
                     const float* lse, const float* delta, void* dk, void* dv, int nthreads) {
  Prob pr;
  int rc = validate(p, &pr);
  if (rc) return rc;
  if (!q || !k || !v || !dout || !lse || !delta || !dk || !dv) return FA_ERR_NULL;
  const int D = p->D, Sq = p->Sq, Skv = p->Skv;
  parallel_for(p->B * p->Hkv, nthreads, [&](int kvh) {
    const int b = kvh / p->Hkv, hk = kvh - b * p->Hkv;
    const std::vector<float> kh = load_head(k, pr.bf16, kvh, Skv, D), vh = load_head(v, pr.bf16, kvh, Skv, D);
    std::vector<float> dK((size_t)Skv * D, 0.f), dV((size_t)Skv * D, 0.f);
    std::vector<float> qi(D), di(D), s(Skv), dsds(Skv);
    std::vector<uint8_t> st;
    for (int h = hk * pr.g; h < (hk + 1) * pr.g; ++h) {
      const size_t head = (size_t)b * p->Hq + h;
      int cur_qb = -1;
      for (int i = 0; i < Sq; ++i) {
        const int qb = pr.tables ? i / p->mask_block_q : 0;
        if (qb != cur_qb) {
          block_states(pr, b, h, qb, &st);
          cur_qb = qb;
        }
        const size_t r = head * Sq + i;
        const float L = lse[r];
        if (L == -INFINITY) continue;  // no live key: P = 0 everywhere
        load_row(q, pr.bf16, r, D, qi.data());
        load_row(dout, pr.bf16, r, D, di.data());
        if (!row_scores(pr, b, h, i, qi.data(), kh.data(), st, s.data(), dsds.data())) continue;
        const float Di = delta[r];
        for (int j = 0; j < Skv; ++j) {
          if (s[j] == -INFINITY) continue;
          const float pj = std::exp(s[j] - L);
          const float* vj = vh.data() + (size_t)j * D;
          float dp = 0.f;
          for (int d = 0; d < D; ++d) dp += di[d] * vj[d];
          float ds = pj * (dp - Di) * dsds[j];
          const float pc = pr.bf16 ? round_bf16(pj) : pj;
          if (pr.bf16) ds = round_bf16(ds);
          float* dvj = dV.data() + (size_t)j * D;
          float* dkj = dK.data() + (size_t)j * D;
          for (int d = 0; d < D; ++d) {
            dvj[d] += pc * di[d];
            dkj[d] += ds * qi[d];
          }
        }
      }
    }
    for (int j = 0; j < Skv; ++j) {
      float* dkj = dK.data() + (size_t)j * D;
      for (int d = 0; d < D; ++d) dkj[d] *= pr.scale;
      store_row(dk, pr.bf16, (size_t)kvh * Skv + j, D, dkj);
      store_row(dv, pr.bf16, (size_t)kvh * Skv + j, D, dV.data() + (size_t)j * D);
    }
  });
  return FA_OK;
}

int fa_bwd_dq_host(const fa_params* p, const void* q, const void* k, const void* v, const void* dout,
                   const float* lse, const float* delta, void* dq, int nthreads) {
  Prob pr;
  int rc = validate(p, &pr);
  if (rc) return rc;
  if (!q || !k || !v || !dout || !lse || !delta || !dq) return FA_ERR_NULL;
  const int D = p->D, Sq = p->Sq, Skv = p->Skv;
  parallel_for(p->B * p->Hq, nthreads, [&](int head) {
    const int b = head / p->Hq, h = head - b * p->Hq, hk = b * p->Hkv + h / pr.g;
    const std::vector<float> kh = load_head(k, pr.bf16, hk, Skv, D), vh = load_head(v, pr.bf16, hk, Skv, D);
    std::vector<float> qi(D), di(D), s(Skv), dsds(Skv), dqi(D);
    std::vector<uint8_t> st;
    int cur_qb = -1;
    for (int i = 0; i < Sq; ++i) {
      const int qb = pr.tables ? i / p->mask_block_q : 0;
      if (qb != cur_qb) {
        block_states(pr, b, h, qb, &st);
        cur_qb = qb;
      }
      const size_t r = (size_t)head * Sq + i;
      std::fill(dqi.begin(), dqi.end(), 0.f);
      const float L = lse[r];
      load_row(q, pr.bf16, r, D, qi.data());
      load_row(dout, pr.bf16, r, D, di.data());
      if (L != -INFINITY && row_scores(pr, b, h, i, qi.data(), kh.data(), st, s.data(), dsds.data())) {
        const float Di = delta[r];
        for (int j = 0; j < Skv; ++j) {
          if (s[j] == -INFINITY) continue;
          const float pj = std::exp(s[j] - L);
          const float* vj = vh.data() + (size_t)j * D;
          float dp = 0.f;
          for (int d = 0; d < D; ++d) dp += di[d] * vj[d];
          float ds = pj * (dp - Di) * dsds[j];
          if (pr.bf16) ds = round_bf16(ds);
          const float* kj = kh.data() + (size_t)j * D;
          for (int d = 0; d < D; ++d) dqi[d] += ds * kj[d];
        }
      }
      for (int d = 0; d < D; ++d) dqi[d] *= pr.scale;
      store_row(dq, pr.bf16, r, D, dqi.data());
    }
  });
  return FA_OK;
}

int fa_bwd_host(const fa_params* p, const void* q, const void* k, const void* v, const void* o, const float* lse,
                const void* dout, void* dq, void* dk, void* dv, int nthreads) {
  Prob pr;
  int rc = validate(p, &pr);
  if (rc) return rc;
  if (!q || !k || !v || !o || !lse || !dout || !dq || !dk || !dv) return FA_ERR_NULL;
  std::vector<float> delta((size_t)p->B * p->Hq * p->Sq);
  rc = fa_bwd_preprocess_host(p, o, dout, delta.data(), nthreads);
  if (!rc) rc = fa_bwd_dkdv_host(p, q, k, v, dout, lse, delta.data(), dk, dv, nthreads);
  if (!rc) rc = fa_bwd_dq_host(p, q, k, v, dout, lse, delta.data(), dq, nthreads);
  return rc;
}

}  // extern "C"
