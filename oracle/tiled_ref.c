/*
 * Oracle / CPU baseline: a C + OpenMP restatement of the reference's tiled
 * Pallas flash-attention kernels (src/pallas_flexattn/flash_attn.py).
 * TEST INFRASTRUCTURE ONLY — never linked into the product library.
 *
 * Restated behaviour (file:line in flash_attn.py):
 *   fwd            :59-108 program (b*h, q-block); fori_loop over ALL kv blocks
 *                  (:101-104, no block skipping), S = q k^T (fp32 accumulate, :83)
 *                  * 1/sqrt(D) (:129), mask -> -inf (:85-88), online softmax with
 *                  NaN->0 guards (:90-99), P cast to the V dtype before P V (:94),
 *                  LSE = m + log(l) (:105), O = O / l (:106), outputs cast to the
 *                  input dtype (:107-108; LSE is stored in q's dtype, :144).
 *   bwd preprocess :168-173 Delta = sum_d float32(o * do) with the product formed
 *                  in the input dtype (:172), stored in o's dtype (:190).
 *   bwd dK/dV      :206-253 program (b*h, kv-block), loop over ALL q blocks (:251):
 *                  P = exp(S - LSE) (:241), dP = dO V^T (:242),
 *                  dS = P (dP - Delta) * scale (:243), dV += P^T dO with P cast (:244),
 *                  dK += dS^T Q with dS cast (:245).
 *   bwd dQ         :313-356 program (b*h, q-block), loop over ALL kv blocks (:355):
 *                  dQ += dS K with dS cast (:349).
 * "cast" means round-to-nearest-even to bfloat16 when bf16 != 0, identity for fp32.
 * ds_scale_after != 0 moves the softmax scale of dS after its cast (dS rounded
 * as P (dP - Delta), then multiplied by the scale in fp32): the cast point of
 * the MI355X kernels, which apply the scale once to the dQ / dK accumulators.
 * Inputs are float32 arrays holding values already representable in the input
 * dtype.  Tiles that run past T are masked past the end (the reference has no
 * defined behaviour there).  Masks: window (left, right; -1 = unlimited, as
 * mask_mod.py:25-43; causal = (-1, 0)) optionally AND same-document ids.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

static inline float rnd_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return x; /* NaN */
  u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  float r;
  memcpy(&r, &u, 4);
  return r;
}

static inline float cast_in(float x, int bf16) { return bf16 ? rnd_bf16(x) : x; }

typedef struct {
  int use_mask, left, right;
  const int *doc; /* (B, T) or NULL */
} mask_t;

static inline int allowed(const mask_t *m, int b, int T, int qi, int ki) {
  if (ki >= T) return 0;
  if (!m->use_mask) return 1;
  int delta = qi - ki;
  if (m->left >= 0 && !(delta <= m->left)) return 0;
  if (m->right >= 0 && !(-delta <= m->right)) return 0;
  if (m->doc && m->doc[(size_t)b * T + qi] != m->doc[(size_t)b * T + ki]) return 0;
  return 1;
}

static inline float dotf(const float *a, const float *b, int D) {
  float acc = 0.f;
  for (int d = 0; d < D; ++d) acc += a[d] * b[d];
  return acc;
}

int ref_fwd(const float *q, const float *k, const float *v, int B, int H, int T, int D,
            int block_r, int block_c, int use_mask, int left, int right, const int *doc,
            int bf16, int stats_in_dtype, float *o, float *lse, int nthreads, int bh_begin,
            int bh_end) {
  if (block_r <= 0 || block_c <= 0 || D <= 0 || T <= 0) return -1;
  mask_t m = {use_mask, left, right, doc};
  const float scale = 1.0f / sqrtf((float)D);
  const int nqb = (T + block_r - 1) / block_r, nkb = (T + block_c - 1) / block_c;
  if (bh_end > B * H) bh_end = B * H;
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
  {
    float *s = malloc(sizeof(float) * block_r * block_c);
    float *acc = malloc(sizeof(float) * block_r * D);
    float *mx = malloc(sizeof(float) * block_r), *l = malloc(sizeof(float) * block_r);
#pragma omp for schedule(dynamic)
    for (long prog = (long)bh_begin * nqb; prog < (long)bh_end * nqb; ++prog) {
      const int bh = (int)(prog / nqb), qb = (int)(prog % nqb), b = bh / H;
      const float *qh = q + (size_t)bh * T * D, *kh = k + (size_t)bh * T * D, *vh = v + (size_t)bh * T * D;
      const int q0 = qb * block_r, nr = (q0 + block_r <= T) ? block_r : T - q0;
      memset(acc, 0, sizeof(float) * block_r * D);
      for (int r = 0; r < nr; ++r) { mx[r] = -INFINITY; l[r] = 0.f; }
      for (int t = 0; t < nkb; ++t) {
        const int k0 = t * block_c;
        for (int r = 0; r < nr; ++r) {
          const float *qr = qh + (size_t)(q0 + r) * D;
          float mb = mx[r];
          for (int c = 0; c < block_c; ++c) {
            const int ki = k0 + c;
            float sv = (ki < T) ? dotf(qr, kh + (size_t)ki * D, D) * scale : 0.f;
            if (!allowed(&m, b, T, q0 + r, ki)) sv = -INFINITY;
            s[r * block_c + c] = sv;
            if (sv > mb) mb = sv;
          }
          float lb = 0.f;
          float *ar = acc + (size_t)r * D;
          float alpha = expf(mx[r] - mb);
          if (isnan(alpha)) alpha = 0.f;
          for (int d = 0; d < D; ++d) ar[d] *= alpha;
          for (int c = 0; c < block_c; ++c) {
            float p = expf(s[r * block_c + c] - mb);
            if (isnan(p)) p = 0.f;
            lb += p;
            const float pc = cast_in(p, bf16);
            if (pc != 0.f) {
              const float *vr = vh + (size_t)(k0 + c) * D;
              for (int d = 0; d < D; ++d) ar[d] += pc * vr[d];
            }
          }
          l[r] = l[r] * alpha + lb;
          mx[r] = mb;
        }
      }
      for (int r = 0; r < nr; ++r) {
        const size_t row = (size_t)bh * T + q0 + r;
        for (int d = 0; d < D; ++d) o[row * D + d] = cast_in(acc[(size_t)r * D + d] / l[r], bf16);
        const float ls = mx[r] + logf(l[r]);
        lse[row] = stats_in_dtype ? cast_in(ls, bf16) : ls;
      }
    }
    free(s); free(acc); free(mx); free(l);
  }
  return 0;
}

int ref_bwd(const float *q, const float *k, const float *v, const float *o, const float *lse,
            const float *dout, int B, int H, int T, int D, int block_r, int block_c, int use_mask,
            int left, int right, const int *doc, int bf16, int stats_in_dtype, int ds_scale_after,
            float *dq, float *dk,
            float *dv, int nthreads, int bh_begin, int bh_end) {
  if (block_r <= 0 || block_c <= 0 || D <= 0 || T <= 0) return -1;
  mask_t m = {use_mask, left, right, doc};
  const float scale = 1.0f / sqrtf((float)D);
  const int nqb = (T + block_r - 1) / block_r, nkb = (T + block_c - 1) / block_c;
  if (bh_end > B * H) bh_end = B * H;
  if (nthreads > 0) omp_set_num_threads(nthreads);
  const size_t nrows = (size_t)(bh_end - bh_begin) * T;
  float *delta = malloc(sizeof(float) * (nrows ? nrows : 1));
  /* preprocess: Delta = rowsum(float32(o*do)), product in the input dtype */
#pragma omp parallel for schedule(static)
  for (long i = 0; i < (long)nrows; ++i) {
    const size_t row = (size_t)bh_begin * T + i;
    float acc = 0.f;
    for (int d = 0; d < D; ++d) acc += cast_in(o[row * D + d] * dout[row * D + d], bf16);
    delta[i] = stats_in_dtype ? cast_in(acc, bf16) : acc;
  }
#pragma omp parallel
  {
    float *p = malloc(sizeof(float) * block_r * block_c);
    float *ds = malloc(sizeof(float) * block_r * block_c);
    float *acc1 = malloc(sizeof(float) * block_c * D), *acc2 = malloc(sizeof(float) * block_c * D);
    float *accq = malloc(sizeof(float) * block_r * D);
    /* dK / dV: program per (bh, kv block), loop over all q blocks */
#pragma omp for schedule(dynamic)
    for (long prog = (long)bh_begin * nkb; prog < (long)bh_end * nkb; ++prog) {
      const int bh = (int)(prog / nkb), kb = (int)(prog % nkb), b = bh / H;
      const float *qh = q + (size_t)bh * T * D, *kh = k + (size_t)bh * T * D, *vh = v + (size_t)bh * T * D;
      const float *doh = dout + (size_t)bh * T * D, *lh = lse + (size_t)bh * T;
      const float *dh = delta + (size_t)(bh - bh_begin) * T;
      const int k0 = kb * block_c, nc = (k0 + block_c <= T) ? block_c : T - k0;
      memset(acc1, 0, sizeof(float) * block_c * D);
      memset(acc2, 0, sizeof(float) * block_c * D);
      for (int t = 0; t < nqb; ++t) {
        const int q0 = t * block_r, nr = (q0 + block_r <= T) ? block_r : T - q0;
        for (int r = 0; r < nr; ++r) {
          const float *qr = qh + (size_t)(q0 + r) * D, *dor = doh + (size_t)(q0 + r) * D;
          for (int c = 0; c < nc; ++c) {
            const int ki = k0 + c;
            float sv = dotf(qr, kh + (size_t)ki * D, D) * scale;
            if (!allowed(&m, b, T, q0 + r, ki)) sv = -INFINITY;
            const float pv = expf(sv - lh[q0 + r]);
            const float dp = dotf(dor, vh + (size_t)ki * D, D);
            p[r * block_c + c] = cast_in(pv, bf16);
            ds[r * block_c + c] = ds_scale_after ? cast_in(pv * (dp - dh[q0 + r]), bf16) * scale
                                                 : cast_in(pv * (dp - dh[q0 + r]) * scale, bf16);
          }
        }
        for (int c = 0; c < nc; ++c) {
          float *dvr = acc1 + (size_t)c * D, *dkr = acc2 + (size_t)c * D;
          for (int r = 0; r < nr; ++r) {
            const float pv = p[r * block_c + c], dsv = ds[r * block_c + c];
            const float *dor = doh + (size_t)(q0 + r) * D, *qr = qh + (size_t)(q0 + r) * D;
            if (pv != 0.f) for (int d = 0; d < D; ++d) dvr[d] += pv * dor[d];
            if (dsv != 0.f) for (int d = 0; d < D; ++d) dkr[d] += dsv * qr[d];
          }
        }
      }
      for (int c = 0; c < nc; ++c) {
        const size_t row = (size_t)bh * T + k0 + c;
        for (int d = 0; d < D; ++d) {
          dv[row * D + d] = cast_in(acc1[(size_t)c * D + d], bf16);
          dk[row * D + d] = cast_in(acc2[(size_t)c * D + d], bf16);
        }
      }
    }
    /* dQ: program per (bh, q block), loop over all kv blocks */
#pragma omp for schedule(dynamic)
    for (long prog = (long)bh_begin * nqb; prog < (long)bh_end * nqb; ++prog) {
      const int bh = (int)(prog / nqb), qb = (int)(prog % nqb), b = bh / H;
      const float *qh = q + (size_t)bh * T * D, *kh = k + (size_t)bh * T * D, *vh = v + (size_t)bh * T * D;
      const float *doh = dout + (size_t)bh * T * D, *lh = lse + (size_t)bh * T;
      const float *dh = delta + (size_t)(bh - bh_begin) * T;
      const int q0 = qb * block_r, nr = (q0 + block_r <= T) ? block_r : T - q0;
      memset(accq, 0, sizeof(float) * block_r * D);
      for (int t = 0; t < nkb; ++t) {
        const int k0 = t * block_c, nc = (k0 + block_c <= T) ? block_c : T - k0;
        for (int r = 0; r < nr; ++r) {
          const float *qr = qh + (size_t)(q0 + r) * D, *dor = doh + (size_t)(q0 + r) * D;
          float *aq = accq + (size_t)r * D;
          for (int c = 0; c < nc; ++c) {
            const int ki = k0 + c;
            float sv = dotf(qr, kh + (size_t)ki * D, D) * scale;
            if (!allowed(&m, b, T, q0 + r, ki)) sv = -INFINITY;
            const float pv = expf(sv - lh[q0 + r]);
            const float dp = dotf(dor, vh + (size_t)ki * D, D);
            const float dsv = ds_scale_after ? cast_in(pv * (dp - dh[q0 + r]), bf16) * scale
                                             : cast_in(pv * (dp - dh[q0 + r]) * scale, bf16);
            if (dsv != 0.f) {
              const float *kr = kh + (size_t)ki * D;
              for (int d = 0; d < D; ++d) aq[d] += dsv * kr[d];
            }
          }
        }
      }
      for (int r = 0; r < nr; ++r) {
        const size_t row = (size_t)bh * T + q0 + r;
        for (int d = 0; d < D; ++d) dq[row * D + d] = cast_in(accq[(size_t)r * D + d], bf16);
      }
    }
    free(p); free(ds); free(acc1); free(acc2); free(accq);
  }
  free(delta);
  return 0;
}
