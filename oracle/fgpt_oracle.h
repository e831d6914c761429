/* fgpt_oracle.h -- CPU restatement of the fortran_gpt forward path.
 *
 * TEST INFRASTRUCTURE ONLY. The HIP engine's results are checked against this
 * library: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it. The product path (libfgpt.so) never links, loads or calls
 * it.
 *
 * Every routine restates one reference routine in fp32, in the reference's
 * loop and summation order, with row-major flat buffers and 0-based ids.
 * Citations are to files of 14NGiestas/autoresearch.
 */
#ifndef FGPT_ORACLE_H
#define FGPT_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/test/test_kernels.f90:115-119 (frand: LCG on a default-kind integer,
 * wrapping as gfortran does). Fills x[0..n) with frand()*scale. */
void or_frand_fill(int32_t *seed, float *x, int32_t n, float scale);

/* src/app/chat_text.f90:225-235, src/app/eval_bpb.f90:117-126 */
void or_rope_tables(float *cosb, float *sinb, int32_t T, int32_t hd);

/* src/lib/fortran_linear.f90:62-78 */
void or_wte_lookup(const int32_t *idx, const float *wte, float *out,
                   int32_t B, int32_t T, int32_t D);
/* src/lib/fortran_rmsnorm.f90:40-60 */
void or_rmsnorm0(const float *x, float *y, int64_t N, int32_t C, float eps);
/* src/lib/fortran_linear.f90:18-36 (the order linear3d_sgemm is tested
 * against, src/test/test_kernels.f90:2156-2177) */
void or_linear(const float *x, const float *w, float *y, int64_t BT,
               int32_t IF, int32_t OF);
/* src/lib/fortran_rope.f90:25-52 */
void or_rope(const float *x, const float *cosb, const float *sinb, float *y,
             int32_t B, int32_t T, int32_t H, int32_t D);
/* src/lib/fortran_attn.f90:30-117 (cap = 0, softmax) */
void or_causal_attn(const float *q, const float *k, const float *v, float *y,
                    int32_t B, int32_t T, int32_t H, int32_t KH, int32_t D);
/* src/lib/fortran_attn.f90:317-362 */
void or_attn_step(const float *q, const float *K, const float *V, float *y,
                  int32_t B, int32_t H, int32_t KH, int32_t D, int32_t TC);
/* src/lib/fortran_attn.f90:376-425 */
void or_attn_chunk(const float *q, const float *K, const float *V, float *y,
                   int32_t B, int32_t H, int32_t KH, int32_t D,
                   int32_t TC_PREV, int32_t TB);
/* src/lib/fortran_attn.f90:247-300: attn_sgemm's positive-score count per
 * (b, h) over the causal scores (q . k) * scale > 0; namb (nullable): how
 * many have |q . k| <= rel_tol * sum |q_d k_d| (sign within rounding). */
void or_attn_pos_count(const float *q, const float *k, int32_t B, int32_t T,
                       int32_t H, int32_t KH, int32_t D, float rel_tol,
                       int32_t *npos, int32_t *namb);
/* src/lib/fortran_attn.f90:697-710 */
void or_relu2(float *x, int64_t N);

/* src/lib/fortran_gpt.f90:54-199 (default attention path) */
void or_gpt_forward(const int32_t *idx, const float *cosb, const float *sinb,
                    const float *wte, const float *c_q, const float *c_k,
                    const float *c_v, const float *c_proj, const float *c_fc,
                    const float *c_proj2, const float *lm_head, float *outp,
                    int32_t B, int32_t T, int32_t V, int32_t D, int32_t H,
                    int32_t KH, int32_t HD, int32_t L, float eps);

/* or_gpt_forward plus each layer's or_attn_pos_count (npos, namb:
 * [L][B][H]), the statistic gpt_forward collects with attn_blas and
 * pos_frac (src/lib/fortran_gpt.f90:160-162). */
void or_gpt_forward_pos(const int32_t *idx, const float *cosb, const float *sinb,
                        const float *wte, const float *c_q, const float *c_k,
                        const float *c_v, const float *c_proj, const float *c_fc,
                        const float *c_proj2, const float *lm_head, float *outp,
                        int32_t B, int32_t T, int32_t V, int32_t D, int32_t H,
                        int32_t KH, int32_t HD, int32_t L, float eps, float rel_tol,
                        int32_t *npos, int32_t *namb);
/* src/lib/fortran_kv.f90:26-149. Returns 0, or 1 when the cache is full
 * (the reference prints and exits). */
int32_t or_gpt_step(const int32_t *idx1, const float *cos1, const float *sin1,
                    const float *wte, const float *c_q, const float *c_k,
                    const float *c_v, const float *c_proj, const float *c_fc,
                    const float *c_proj2, const float *lm_head,
                    float *cache_k, float *cache_v, int32_t *cache_len,
                    int32_t maxT, float *out1, int32_t B, int32_t V, int32_t D,
                    int32_t H, int32_t KH, int32_t HD, int32_t L, float eps);

/* src/lib/fortran_kv.f90:160-289. Returns 0, 1 (TB < 1) or 2 (cache full). */
int32_t or_gpt_step_multi(const int32_t *idx, const float *cosb,
                          const float *sinb, const float *wte,
                          const float *c_q, const float *c_k, const float *c_v,
                          const float *c_proj, const float *c_fc,
                          const float *c_proj2, const float *lm_head,
                          float *cache_k, float *cache_v, int32_t *cache_len,
                          int32_t maxT, float *out, int32_t B, int32_t V,
                          int32_t D, int32_t H, int32_t KH, int32_t HD,
                          int32_t L, int32_t TB, float eps);

/* src/app/eval_bpb.f90:165-181: nll[r] = logsumexp(logits[r,:]) - logits[r, tgt[r]] */
void or_nll(const float *logits, const int32_t *targets, float *nll,
            int64_t rows, int32_t V);
/* src/lib/sample.f90:271-277: first index of the maximum (strict >), 0-based */
int32_t or_argmax(const float *logits, int32_t V);

/* Number of OpenMP threads the oracle will use (for reporting). */
int32_t or_num_threads(void);
/* on != 0: or_linear keeps the transposed copy of each weight array it sees
 * (the arrays must not move or change meanwhile); 0: frees them, and every
 * call transposes again (the default). */
void or_wt_cache(int32_t on);

#ifdef __cplusplus
}
#endif
#endif
