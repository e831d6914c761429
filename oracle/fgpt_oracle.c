/* fgpt_oracle.c -- CPU restatement of the fortran_gpt forward path.
 *
 * TEST INFRASTRUCTURE ONLY (the oracle results are checked against). Loaded
 * by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg;
 * never by the product library.
 *
 * Arithmetic is fp32 throughout, built with -ffp-contract=off so that every
 * `acc = acc + a*b` rounds the product and the sum separately, as the
 * reference's Fortran loops do when compiled without FMA contraction. Each
 * routine keeps the reference's summation order per output element; OpenMP
 * only distributes independent output elements, so the thread count never
 * changes a result.
 *
 * Parity pinning (which checks fix each routine) is listed in the header of
 * tests/test_oracle.py; every routine here has at least one pin there.
 */
#include "fgpt_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* malloc that stops the program when memory runs out */
static void *xmalloc(size_t n) {
  void *p = malloc(n ? n : 1);
  if (!p) {
    fprintf(stderr, "oracle: cannot allocate %zu bytes\n", n);
    abort();
  }
  return p;
}

int32_t or_num_threads(void) {
#ifdef _OPENMP
  return (int32_t)omp_get_max_threads();
#else
  return 1;
#endif
}

/* src/test/test_kernels.f90:115-119
 *   seed = mod(seed * 1103515245 + 12345, 2147483647)
 *   r = real(mod(seed / 65536, 32768)) / 32768 - 0.5
 * on a default (32-bit) integer that wraps on overflow; Fortran mod and
 * integer division truncate toward zero, as C's % and / do. */
void or_frand_fill(int32_t *seed, float *x, int32_t n, float scale) {
  int32_t s = *seed;
  for (int32_t i = 0; i < n; ++i) {
    uint32_t prod = (uint32_t)s * 1103515245u;
    uint32_t sum = prod + 12345u;
    int32_t a = (int32_t)sum;
    s = a % 2147483647;
    float r = (float)((s / 65536) % 32768) / 32768.0f - 0.5f;
    x[i] = r * scale;
  }
  *seed = s;
}

/* src/app/chat_text.f90:225-235 (identical in src/app/eval_bpb.f90:117-126):
 *   theta = 10000 ** (-2 (j-1) / hd);  ang = (i-1) * theta  (fp32 host math) */
void or_rope_tables(float *cosb, float *sinb, int32_t T, int32_t hd) {
  int32_t d2 = hd / 2;
  for (int32_t i = 1; i <= T; ++i) {
    for (int32_t j = 1; j <= d2; ++j) {
      float theta = powf(10000.0f, -2.0f * (float)(j - 1) / (float)hd);
      float ang = (float)(i - 1) * theta;
      cosb[(int64_t)(i - 1) * d2 + (j - 1)] = cosf(ang);
      sinb[(int64_t)(i - 1) * d2 + (j - 1)] = sinf(ang);
    }
  }
}

/* src/lib/fortran_linear.f90:62-78: out(b,t,:) = wte(idx(b,t), :), 0-based ids */
void or_wte_lookup(const int32_t *idx, const float *wte, float *out,
                   int32_t B, int32_t T, int32_t D) {
  int64_t rows = (int64_t)B * T;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r)
    memcpy(out + r * D, wte + (int64_t)idx[r] * D, sizeof(float) * (size_t)D);
}

/* src/lib/fortran_rmsnorm.f90:40-60:
 *   ss = sum_j x_j^2 (sequential); inv = 1/sqrt(ss/C + eps); y = x*inv */
void or_rmsnorm0(const float *x, float *y, int64_t N, int32_t C, float eps) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < N; ++i) {
    const float *xr = x + i * C;
    float ss = 0.0f;
    for (int32_t j = 0; j < C; ++j) ss = ss + xr[j] * xr[j];
    float inv = 1.0f / sqrtf(ss / (float)C + eps);
    for (int32_t j = 0; j < C; ++j) y[i * C + j] = xr[j] * inv;
  }
}

/* src/lib/fortran_linear.f90:18-36: y(bt,o) = sum_i x(bt,i) * w(o,i), the
 * sum over i taken in increasing i. The loop is blocked over (bt, o) and runs
 * i innermost-per-element through a transposed copy of w so that it
 * vectorises over o; each y(bt,o) still sees the same sequence of roundings
 * as the naive loop. */
#define LIN_RB 8   /* rows of x per block */
#define LIN_OB 256 /* outputs per block   */

/* Transposed weight copies kept between calls while or_wt_cache(1) is in
 * force, keyed by (w, IF, OF). The caller that turns it on promises the
 * weight arrays neither move nor change until it turns it off again (which
 * frees the copies); with it off (the default) every call transposes. */
#define WT_MAX 512
static struct { const float *w; int32_t IF, OF; float *wt; } g_wt[WT_MAX];
static int g_wt_n = 0, g_wt_on = 0;

void or_wt_cache(int32_t on) {
  for (int i = 0; i < g_wt_n; ++i) free(g_wt[i].wt);
  g_wt_n = 0;
  g_wt_on = on != 0;
}

static float *transposed(const float *w, int32_t IF, int32_t OF, int *owned) {
  if (g_wt_on)
    for (int i = 0; i < g_wt_n; ++i)
      if (g_wt[i].w == w && g_wt[i].IF == IF && g_wt[i].OF == OF) {
        *owned = 0;
        return g_wt[i].wt;
      }
  float *wt = (float *)xmalloc(sizeof(float) * (size_t)IF * (size_t)OF);
#pragma omp parallel for schedule(static)
  for (int32_t i = 0; i < IF; ++i)
    for (int32_t o = 0; o < OF; ++o) wt[(int64_t)i * OF + o] = w[(int64_t)o * IF + i];
  *owned = 1;
  if (g_wt_on && g_wt_n < WT_MAX) {
    g_wt[g_wt_n].w = w;
    g_wt[g_wt_n].IF = IF;
    g_wt[g_wt_n].OF = OF;
    g_wt[g_wt_n].wt = wt;
    ++g_wt_n;
    *owned = 0;
  }
  return wt;
}

void or_linear(const float *x, const float *w, float *y, int64_t BT,
               int32_t IF, int32_t OF) {
  int owned;
  float *wt = transposed(w, IF, OF, &owned);
  int64_t nrb = (BT + LIN_RB - 1) / LIN_RB;
  int64_t nob = (OF + LIN_OB - 1) / LIN_OB;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int64_t rb = 0; rb < nrb; ++rb) {
    for (int64_t ob = 0; ob < nob; ++ob) {
      float acc[LIN_RB][LIN_OB];
      int64_t r0 = rb * LIN_RB, o0 = ob * LIN_OB;
      int nr = (int)((BT - r0) < LIN_RB ? (BT - r0) : LIN_RB);
      int no = (int)((OF - o0) < LIN_OB ? (OF - o0) : LIN_OB);
      for (int r = 0; r < nr; ++r)
        for (int o = 0; o < no; ++o) acc[r][o] = 0.0f;
      for (int32_t i = 0; i < IF; ++i) {
        const float *wr = wt + (int64_t)i * OF + o0;
        for (int r = 0; r < nr; ++r) {
          float xv = x[(r0 + r) * IF + i];
          float *ar = acc[r];
          for (int o = 0; o < no; ++o) ar[o] = ar[o] + xv * wr[o];
        }
      }
      for (int r = 0; r < nr; ++r)
        memcpy(y + (r0 + r) * OF + o0, acc[r], sizeof(float) * (size_t)no);
    }
  }
  if (owned) free(wt);
}

/* src/lib/fortran_rope.f90:25-52, half-split rotation:
 *   y_d = x_d c + x_{d+D/2} s;  y_{d+D/2} = x_d (-s) + x_{d+D/2} c */
void or_rope(const float *x, const float *cosb, const float *sinb, float *y,
             int32_t B, int32_t T, int32_t H, int32_t D) {
  int32_t d2 = D / 2;
#pragma omp parallel for collapse(3) schedule(static)
  for (int32_t a = 0; a < B; ++a)
    for (int32_t t = 0; t < T; ++t)
      for (int32_t h = 0; h < H; ++h) {
        int64_t base = (((int64_t)a * T + t) * H + h) * D;
        for (int32_t d = 0; d < d2; ++d) {
          float x1 = x[base + d], x2 = x[base + d + d2];
          float c = cosb[(int64_t)t * d2 + d], s = sinb[(int64_t)t * d2 + d];
          y[base + d] = x1 * c + x2 * s;
          y[base + d + d2] = x1 * (-s) + x2 * c;
        }
      }
}

/* One softmax-attention row shared by the three attention routines below;
 * the op order is the one all three reference routines use (and that
 * src/lib/fortran_attn.f90:316 requires to agree bit-exactly):
 *   s_j = (sum_d q_d k_jd) * scale, m = running max (strict >),
 *   p_j = exp(s_j - m), sm = sum_j p_j, inv = 1/sm,
 *   y_d = sum_j (p_j * inv) * v_jd.
 * k and v advance by kstride floats per position. */
static void attn_row(const float *q, const float *k, const float *v,
                     int64_t kstride, int32_t n, int32_t D, float scale,
                     float *sc, float *y) {
  float m = -3.40282347e+38f; /* -huge(1.0_wp) */
  for (int32_t s = 0; s < n; ++s) {
    const float *kr = k + s * kstride;
    float acc = 0.0f;
    for (int32_t d = 0; d < D; ++d) acc = acc + q[d] * kr[d];
    sc[s] = acc * scale;
    if (sc[s] > m) m = sc[s];
  }
  float sm = 0.0f;
  for (int32_t s = 0; s < n; ++s) {
    sc[s] = expf(sc[s] - m);
    sm = sm + sc[s];
  }
  float inv = 1.0f / sm;
  for (int32_t d = 0; d < D; ++d) {
    float acc = 0.0f;
    for (int32_t s = 0; s < n; ++s) acc = acc + sc[s] * inv * v[s * kstride + d];
    y[d] = acc;
  }
}

/* src/lib/fortran_attn.f90:30-117 with cap = 0 and softmax (the defaults):
 * q (B,T,H,D), k/v (B,T,KH,D), query head h reads kv head h/(H/KH). */
void or_causal_attn(const float *q, const float *k, const float *v, float *y,
                    int32_t B, int32_t T, int32_t H, int32_t KH, int32_t D) {
  float scale = 1.0f / sqrtf((float)D);
  int32_t rep = H / KH;
#pragma omp parallel
  {
    float *sc = (float *)xmalloc(sizeof(float) * (size_t)T);
#pragma omp for collapse(3) schedule(dynamic, 16)
    for (int32_t a = 0; a < B; ++a)
      for (int32_t h = 0; h < H; ++h)
        for (int32_t t = 0; t < T; ++t) {
          int32_t kb = h / rep;
          const float *qr = q + (((int64_t)a * T + t) * H + h) * D;
          const float *kr = k + ((int64_t)a * T * KH + kb) * D;
          const float *vr = v + ((int64_t)a * T * KH + kb) * D;
          attn_row(qr, kr, vr, (int64_t)KH * D, t + 1, D, scale, sc,
                   y + (((int64_t)a * T + t) * H + h) * D);
        }
    free(sc);
  }
}

/* src/lib/fortran_attn.f90:317-362: q (B,H,D) vs cache K/V (B,TC,KH,D). */
void or_attn_step(const float *q, const float *K, const float *V, float *y,
                  int32_t B, int32_t H, int32_t KH, int32_t D, int32_t TC) {
  float scale = 1.0f / sqrtf((float)D);
  int32_t rep = H / KH;
#pragma omp parallel
  {
    float *sc = (float *)xmalloc(sizeof(float) * (size_t)(TC > 0 ? TC : 1));
#pragma omp for collapse(2) schedule(static)
    for (int32_t a = 0; a < B; ++a)
      for (int32_t h = 0; h < H; ++h) {
        int32_t kb = h / rep;
        attn_row(q + ((int64_t)a * H + h) * D,
                 K + ((int64_t)a * TC * KH + kb) * D,
                 V + ((int64_t)a * TC * KH + kb) * D, (int64_t)KH * D, TC, D,
                 scale, sc, y + ((int64_t)a * H + h) * D);
      }
    free(sc);
  }
}

/* src/lib/fortran_attn.f90:376-425: TB queries against the cache positions
 * 1..TC_PREV+iq (B=1 cache layout: the batch stride is not carried). */
void or_attn_chunk(const float *q, const float *K, const float *V, float *y,
                   int32_t B, int32_t H, int32_t KH, int32_t D,
                   int32_t TC_PREV, int32_t TB) {
  float scale = 1.0f / sqrtf((float)D);
  int32_t rep = H / KH;
#pragma omp parallel
  {
    float *sc = (float *)xmalloc(sizeof(float) * (size_t)(TC_PREV + TB));
#pragma omp for collapse(3) schedule(dynamic, 4)
    for (int32_t a = 0; a < B; ++a)
      for (int32_t iq = 0; iq < TB; ++iq)
        for (int32_t h = 0; h < H; ++h) {
          int32_t kb = h / rep;
          int64_t qo = (((int64_t)a * TB + iq) * H + h) * D;
          attn_row(q + qo, K + (int64_t)kb * D, V + (int64_t)kb * D,
                   (int64_t)KH * D, TC_PREV + iq + 1, D, scale, sc, y + qo);
        }
    free(sc);
  }
}

/* src/lib/fortran_attn.f90:247-300 (attn_sgemm's statistic, counted in its
 * causal loop :249-254 before the cap and the softmax): per (b, h), npos =
 * the number of scores s = (q . k) * scale, key t' <= query t, that are
 * > 0 (strict). The score is the dot product in attn_row's order. namb
 * (nullable) receives, per (b, h), how many of those scores have
 * |q . k| <= rel_tol * sum_d |q_d k_d|: their sign is within rounding and
 * can differ in another summation order. */
void or_attn_pos_count(const float *q, const float *k, int32_t B, int32_t T,
                       int32_t H, int32_t KH, int32_t D, float rel_tol,
                       int32_t *npos, int32_t *namb) {
  float scale = 1.0f / sqrtf((float)D);
  int32_t rep = H / KH;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int32_t a = 0; a < B; ++a)
    for (int32_t h = 0; h < H; ++h) {
      int32_t kb = h / rep, np = 0, na = 0;
      for (int32_t t = 0; t < T; ++t) {
        const float *qr = q + (((int64_t)a * T + t) * H + h) * D;
        for (int32_t j = 0; j <= t; ++j) {
          const float *kr = k + (((int64_t)a * T + j) * KH + kb) * D;
          float acc = 0.0f, mag = 0.0f;
          for (int32_t d = 0; d < D; ++d) {
            acc = acc + qr[d] * kr[d];
            mag = mag + fabsf(qr[d] * kr[d]);
          }
          if (acc * scale > 0.0f) ++np;
          if (fabsf(acc) <= rel_tol * mag) ++na;
        }
      }
      npos[a * H + h] = np;
      if (namb) namb[a * H + h] = na;
    }
}

/* src/lib/fortran_attn.f90:697-710: x = max(0, x)^2 in place */
void or_relu2(float *x, int64_t N) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < N; ++i) {
    float a = x[i];
    if (a < 0.0f) a = 0.0f;
    x[i] = a * a;
  }
}

static void add_into(float *dst, const float *src, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) dst[i] = dst[i] + src[i];
}

/* src/lib/fortran_gpt.f90:54-199 (default causal_attn path); with npos set,
 * each layer's attention inputs also give or_attn_pos_count's counts
 * (npos / namb [L][B][H]). */
static void forward_body(const int32_t *idx, const float *cosb, const float *sinb,
                         const float *wte, const float *c_q, const float *c_k,
                         const float *c_v, const float *c_proj, const float *c_fc,
                         const float *c_proj2, const float *lm_head, float *outp,
                         int32_t B, int32_t T, int32_t V, int32_t D, int32_t H,
                         int32_t KH, int32_t HD, int32_t L, float eps,
                         float rel_tol, int32_t *npos, int32_t *namb) {
  int64_t bt = (int64_t)B * T;
  int32_t dff = 4 * D, hdd = H * HD, kvd = KH * HD;
  int64_t qsz = (int64_t)hdd * D, ksz = (int64_t)kvd * D, psz = (int64_t)D * hdd;
  int64_t fcsz = (int64_t)dff * D, p2sz = (int64_t)D * dff;
  float *emd = xmalloc(sizeof(float) * bt * D), *xn = xmalloc(sizeof(float) * bt * D);
  float *sub = xmalloc(sizeof(float) * bt * D), *ao = xmalloc(sizeof(float) * bt * D);
  float *q = xmalloc(sizeof(float) * bt * hdd), *qr = xmalloc(sizeof(float) * bt * hdd);
  float *k = xmalloc(sizeof(float) * bt * kvd), *kr = xmalloc(sizeof(float) * bt * kvd);
  float *v = xmalloc(sizeof(float) * bt * kvd), *mlp = xmalloc(sizeof(float) * bt * dff);

  or_wte_lookup(idx, wte, emd, B, T, D);                     /* :136 */
  or_rmsnorm0(emd, xn, bt, D, eps);                          /* :139-142 */
  memcpy(emd, xn, sizeof(float) * bt * D);
  for (int32_t l = 0; l < L; ++l) {                          /* :145-186 */
    or_rmsnorm0(emd, xn, bt, D, eps);
    or_linear(xn, c_q + l * qsz, q, bt, D, hdd);
    or_linear(xn, c_k + l * ksz, k, bt, D, kvd);
    or_linear(xn, c_v + l * ksz, v, bt, D, kvd);
    or_rope(q, cosb, sinb, qr, B, T, H, HD);
    or_rope(k, cosb, sinb, kr, B, T, KH, HD);
    if (npos)
      or_attn_pos_count(qr, kr, B, T, H, KH, HD, rel_tol, npos + (int64_t)l * B * H,
                        namb ? namb + (int64_t)l * B * H : NULL);
    or_causal_attn(qr, kr, v, ao, B, T, H, KH, HD);
    or_linear(ao, c_proj + l * psz, sub, bt, D, D);
    add_into(emd, sub, bt * D);
    or_rmsnorm0(emd, xn, bt, D, eps);
    or_linear(xn, c_fc + l * fcsz, mlp, bt, D, dff);
    or_relu2(mlp, bt * dff);
    or_linear(mlp, c_proj2 + l * p2sz, sub, bt, dff, D);
    add_into(emd, sub, bt * D);
  }
  or_rmsnorm0(emd, xn, bt, D, eps);                          /* :189 */
  or_linear(xn, lm_head, outp, bt, D, V);                    /* :192 */
  free(emd); free(xn); free(sub); free(ao); free(q); free(qr);
  free(k); free(kr); free(v); free(mlp);
}

void or_gpt_forward(const int32_t *idx, const float *cosb, const float *sinb,
                    const float *wte, const float *c_q, const float *c_k,
                    const float *c_v, const float *c_proj, const float *c_fc,
                    const float *c_proj2, const float *lm_head, float *outp,
                    int32_t B, int32_t T, int32_t V, int32_t D, int32_t H,
                    int32_t KH, int32_t HD, int32_t L, float eps) {
  forward_body(idx, cosb, sinb, wte, c_q, c_k, c_v, c_proj, c_fc, c_proj2, lm_head, outp,
               B, T, V, D, H, KH, HD, L, eps, 0.0f, NULL, NULL);
}

void or_gpt_forward_pos(const int32_t *idx, const float *cosb, const float *sinb,
                        const float *wte, const float *c_q, const float *c_k,
                        const float *c_v, const float *c_proj, const float *c_fc,
                        const float *c_proj2, const float *lm_head, float *outp,
                        int32_t B, int32_t T, int32_t V, int32_t D, int32_t H,
                        int32_t KH, int32_t HD, int32_t L, float eps, float rel_tol,
                        int32_t *npos, int32_t *namb) {
  forward_body(idx, cosb, sinb, wte, c_q, c_k, c_v, c_proj, c_fc, c_proj2, lm_head, outp,
               B, T, V, D, H, KH, HD, L, eps, rel_tol, npos, namb);
}

/* Shared body of gpt_step / gpt_step_multi (src/lib/fortran_kv.f90:80-147
 * and :219-287): TB tokens at cache positions tc0+1..tc0+TB, B = 1 layout. */
static void kv_pass(const int32_t *idx, const float *cosb, const float *sinb,
                    const float *wte, const float *c_q, const float *c_k,
                    const float *c_v, const float *c_proj, const float *c_fc,
                    const float *c_proj2, const float *lm_head, float *cache_k,
                    float *cache_v, int32_t tc0, int32_t maxT, float *out,
                    int32_t B, int32_t V, int32_t D, int32_t H, int32_t KH,
                    int32_t HD, int32_t L, int32_t TB, float eps, int single) {
  int64_t bt = (int64_t)B * TB;
  int32_t dff = 4 * D, hdd = H * HD, kvd = KH * HD;
  int64_t qsz = (int64_t)hdd * D, ksz = (int64_t)kvd * D, psz = (int64_t)D * hdd;
  int64_t fcsz = (int64_t)dff * D, p2sz = (int64_t)D * dff;
  float *emd = xmalloc(sizeof(float) * bt * D), *xn = xmalloc(sizeof(float) * bt * D);
  float *sub = xmalloc(sizeof(float) * bt * D), *ao = xmalloc(sizeof(float) * bt * D);
  float *q = xmalloc(sizeof(float) * bt * hdd), *qr = xmalloc(sizeof(float) * bt * hdd);
  float *k = xmalloc(sizeof(float) * bt * kvd), *kr = xmalloc(sizeof(float) * bt * kvd);
  float *v = xmalloc(sizeof(float) * bt * kvd), *mlp = xmalloc(sizeof(float) * bt * dff);

  or_wte_lookup(idx, wte, emd, B, TB, D);
  or_rmsnorm0(emd, xn, bt, D, eps);
  memcpy(emd, xn, sizeof(float) * bt * D);
  for (int32_t l = 0; l < L; ++l) {
    float *lk = cache_k + (int64_t)l * maxT * kvd, *lv = cache_v + (int64_t)l * maxT * kvd;
    or_rmsnorm0(emd, xn, bt, D, eps);
    or_linear(xn, c_q + l * qsz, q, bt, D, hdd);
    or_linear(xn, c_k + l * ksz, k, bt, D, kvd);
    or_linear(xn, c_v + l * ksz, v, bt, D, kvd);
    or_rope(q, cosb, sinb, qr, B, TB, H, HD);
    or_rope(k, cosb, sinb, kr, B, TB, KH, HD);
    /* cache_copy (:292-300): rotated k and un-rotated v, BB*TB*dkh floats
     * written contiguously from position tc0+1 */
    memcpy(lk + (int64_t)tc0 * kvd, kr, sizeof(float) * bt * kvd);
    memcpy(lv + (int64_t)tc0 * kvd, v, sizeof(float) * bt * kvd);
    if (single)
      or_attn_step(qr, lk, lv, ao, B, H, KH, HD, tc0 + 1);
    else
      or_attn_chunk(qr, lk, lv, ao, B, H, KH, HD, tc0, TB);
    or_linear(ao, c_proj + l * psz, sub, bt, D, D);
    add_into(emd, sub, bt * D);
    or_rmsnorm0(emd, xn, bt, D, eps);
    or_linear(xn, c_fc + l * fcsz, mlp, bt, D, dff);
    or_relu2(mlp, bt * dff);
    or_linear(mlp, c_proj2 + l * p2sz, sub, bt, dff, D);
    add_into(emd, sub, bt * D);
  }
  or_rmsnorm0(emd, xn, bt, D, eps);
  or_linear(xn, lm_head, out, bt, D, V);
  free(emd); free(xn); free(sub); free(ao); free(q); free(qr);
  free(k); free(kr); free(v); free(mlp);
}

/* src/lib/fortran_kv.f90:26-149 */
int32_t or_gpt_step(const int32_t *idx1, const float *cos1, const float *sin1,
                    const float *wte, const float *c_q, const float *c_k,
                    const float *c_v, const float *c_proj, const float *c_fc,
                    const float *c_proj2, const float *lm_head,
                    float *cache_k, float *cache_v, int32_t *cache_len,
                    int32_t maxT, float *out1, int32_t B, int32_t V, int32_t D,
                    int32_t H, int32_t KH, int32_t HD, int32_t L, float eps) {
  if (*cache_len >= maxT) return 1; /* :74-77 "cache full" */
  kv_pass(idx1, cos1, sin1, wte, c_q, c_k, c_v, c_proj, c_fc, c_proj2, lm_head,
          cache_k, cache_v, *cache_len, maxT, out1, B, V, D, H, KH, HD, L, 1,
          eps, 1);
  *cache_len += 1;
  return 0;
}

/* src/lib/fortran_kv.f90:160-289 */
int32_t or_gpt_step_multi(const int32_t *idx, const float *cosb,
                          const float *sinb, const float *wte,
                          const float *c_q, const float *c_k, const float *c_v,
                          const float *c_proj, const float *c_fc,
                          const float *c_proj2, const float *lm_head,
                          float *cache_k, float *cache_v, int32_t *cache_len,
                          int32_t maxT, float *out, int32_t B, int32_t V,
                          int32_t D, int32_t H, int32_t KH, int32_t HD,
                          int32_t L, int32_t TB, float eps) {
  if (TB < 1) return 1;                      /* :209-212 */
  if (*cache_len + TB > maxT) return 2;      /* :213-216 */
  kv_pass(idx, cosb, sinb, wte, c_q, c_k, c_v, c_proj, c_fc, c_proj2, lm_head,
          cache_k, cache_v, *cache_len, maxT, out, B, V, D, H, KH, HD, L, TB,
          eps, 0);
  *cache_len += TB;
  return 0;
}

/* src/app/eval_bpb.f90:165-181 */
void or_nll(const float *logits, const int32_t *targets, float *nll,
            int64_t rows, int32_t V) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float *l = logits + r * V;
    float m = l[0];
    for (int32_t j = 1; j < V; ++j)
      if (l[j] > m) m = l[j];
    float s = 0.0f;
    for (int32_t j = 0; j < V; ++j) s = s + expf(l[j] - m);
    nll[r] = (m + logf(s)) - l[targets[r]];
  }
}

/* src/lib/sample.f90:271-277 */
int32_t or_argmax(const float *logits, int32_t V) {
  int32_t best = 0;
  for (int32_t i = 1; i < V; ++i)
    if (logits[i] > logits[best]) best = i;
  return best;
}
