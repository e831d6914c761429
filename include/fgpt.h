/* fgpt.h -- C ABI of the MI355X (gfx950) engine for the fortran_gpt forward
 * path of 14NGiestas/autoresearch: gpt_forward (prefill), gpt_step and
 * gpt_step_multi (KV-cache decode).
 *
 * The library (autoresearch_amd/libfgpt.so) is bound from Fortran through
 * iso_c_binding (autoresearch_amd/fortran/fgpt_c.f90) exactly as the
 * reference binds its rocBLAS shim (src/lib/fortran_blas_gpu.f90:30-59 ->
 * src/lib/gpu_shim.cpp:98-122), and from Python through ctypes.
 *
 * Conventions
 *  - Every function returns int32_t: FG_OK (0) or a negative FG_E* code;
 *    fg_last_error() returns the message of the calling thread's last error.
 *  - Host buffers are row-major flats, as in the reference (fortran_gpt.f90:
 *    94-96). Ids are 0-based int32 (fortran_linear.f90:59-61). Logits are
 *    fp32, one row of vocab_size per token.
 *  - Weights are the reference loader's eight stacked fp32 buffers
 *    (load_weights.f90:830-874); every value must be exactly bf16
 *    representable. They are uploaded once, as bf16, into one HBM arena.
 *  - A handle is single-stream and not reentrant: a call made while another
 *    thread is inside a call on the same handle fails with FG_EBUSY.
 *  - There is no CPU fallback: without a usable gfx950 device every call that
 *    needs one fails with FG_ENODEV.
 */
#ifndef FGPT_H
#define FGPT_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  FG_OK = 0,
  FG_EARG = -1,     /* bad argument (null pointer, size out of range)      */
  FG_EDIMS = -2,    /* model dims the engine does not support              */
  FG_EWEIGHT = -3,  /* weight file missing/empty/malformed, not bf16-exact */
  FG_EHIP = -4,     /* HIP runtime error                                   */
  FG_EFULL = -5,    /* KV cache full (fortran_kv.f90:74-77, :213-216)      */
  FG_EROPE = -6,    /* RoPE table row not set for a position in use        */
  FG_ENODEV = -7,   /* no usable gfx950 device                             */
  FG_EBUSY = -8,    /* handle in use by another thread                     */
  FG_EARCH = -9,    /* arch.txt or safetensors arch.* metadata disagrees with the
                       dims or with itself (fortran_arch.f90:238-246,
                       load_weights.f90:533-590,799-821) */
  FG_ERANGE = -10   /* FG_OPT_FORWARD_F16: an activation reached fp16's range
                       limit (|x| >= 65520 rounds to inf); the results of that
                       pass are not valid -- run it without the option */
};

typedef struct fg_model fg_model;
typedef struct fg_kv fg_kv;

/* Model dims: the integer arguments of gpt_forward / gpt_step
 * (fortran_gpt.f90:58-64, fortran_kv.f90:31-39). d_ff is 4*d_model. */
typedef struct fg_dims {
  int32_t n_layer, d_model, n_head, n_kv_head, head_dim, vocab_size;
  float eps;
} fg_dims;

/* ABI version (major*100 + minor). */
int32_t fg_version(void);

/* Copies the calling thread's last error message (NUL-terminated,
 * truncated to len) and returns its code. */
int32_t fg_last_error(char *buf, int32_t len);

/* Upload from the reference's eight stacked host buffers (the outputs of
 * load_gpt_weights, src/lib/load_weights.f90:830-874; replaces the per-call
 * weight registration of gpublas_sgemm_fwd, src/lib/gpu_shim.cpp:76-95).
 * The host buffers may be freed after the call. */
int32_t fg_model_create(const fg_dims *dims, const float *wte, const float *c_q,
                        const float *c_k, const float *c_v, const float *c_proj,
                        const float *c_fc, const float *c_proj2,
                        const float *lm_head, fg_model **out);

/* Read a reference weight directory into caller-owned fp32 stacks (the
 * layout fg_model_create takes). As load_gpt_weights does
 * (src/lib/load_weights.f90:830-874), model.safetensors is used when the
 * directory has one: canonical tensor names wte, lm, l{L}.q/.k/.v/.p/.fc/.p2,
 * F32 payloads, declared arch.* metadata checked against dims and for
 * self-consistency (arch.canonical, arch.id; :446-592,
 * src/lib/fortran_arch.f90:200-236). Otherwise the 1-D <f4 .npy files
 * (:853-873), with arch.txt checked when present (require_arch,
 * src/lib/fortran_arch.f90:238-246). Host only: needs no device. */
int32_t fg_weights_read(const fg_dims *dims, const char *weights_dir, float *wte, float *c_q,
                        float *c_k, float *c_v, float *c_proj, float *c_fc, float *c_proj2,
                        float *lm_head);

/* fg_weights_read + fg_model_create. */
int32_t fg_model_load(const fg_dims *dims, const char *weights_dir, fg_model **out);

int32_t fg_model_destroy(fg_model *m);

/* Set RoPE table rows [pos0, pos0+n_pos) from host fp32 (n_pos, head_dim/2)
 * cos/sin tables (src/app/chat_text.f90:225-235): the engine uses the
 * caller's tables rather than recomputing sin/cos on the device. */
int32_t fg_set_rope(fg_model *m, int32_t pos0, int32_t n_pos, const float *cos_buf,
                    const float *sin_buf);

/* gpt_forward (src/lib/fortran_gpt.f90:54-199): B rows of T ids, positions
 * 0..T-1. logits (B*T*V, host) may be NULL. When targets (B*T) is given,
 * nll (B*T, host) receives logsumexp(logits) - logits[target] in nats
 * (src/app/eval_bpb.f90:165-181). RoPE rows 0..T-1 must be set. */
int32_t fg_forward(fg_model *m, const int32_t *ids, int32_t B, int32_t T, float *logits,
                   const int32_t *targets, float *nll);

/* fg_forward with attn_sgemm's positive-score statistic (gpt_forward's
 * optional pos_frac / pos_n with attn_blas, src/lib/fortran_attn.f90:
 * 247-300): npos (n_layer*B*n_head, host; layer-major, then row, then head)
 * receives, per layer, row and head, how many of the T(T+1)/2 causal scores
 * q.k/sqrt(head_dim) are > 0, counted before the softmax as the reference
 * counts them before its cap and relu. The reference's accumulation,
 * pos_frac(h) += npos / (T(T+1)/2) and pos_n(h) += 1 over (layer, row) in
 * that order, is the caller's (the Fortran drop-in does it). T <= 65535. */
int32_t fg_forward_pos(fg_model *m, const int32_t *ids, int32_t B, int32_t T, float *logits,
                       const int32_t *targets, float *nll, int32_t *npos);

/* eval_bpb on the device (src/app/eval_bpb.f90:97-181 with the byte
 * weighting of scripts/eval_driver.py:174-190 / src/app/bpb_agg.f90:130-155):
 * rows holds n_rows rows of T+1 ids (row-major); each row runs inputs
 * ids[0:T] against targets ids[1:T+1], `batch` rows per forward (1..64, as
 * --batch). nll (nullable, n_rows*T): the per-position NLL in nats that
 * eval_bpb prints. Per row (nullable) and in total: nats summed over the
 * positions whose target has token_bytes > 0, and those byte counts; bpb =
 * total_nats / total_bytes / ln 2. Ids outside [0, vocab) or targets outside
 * token_bytes fail with FG_EARG before any work, as bpb_agg aborts. */
int32_t fg_eval_bpb(fg_model *m, const int32_t *rows, int32_t n_rows, int32_t T, int32_t batch,
                    const int32_t *token_bytes, int32_t n_token_bytes, float *nll,
                    double *row_nats, int64_t *row_bytes, double *total_nats,
                    int64_t *total_bytes);

/* Read eval_bpb's rows file: an int32 .npy of logical shape (N, T+1), C or
 * Fortran order (src/app/eval_bpb.f90:51-57,97-115). rows == NULL returns
 * only n_rows and width (= T+1); else rows receives N*width ids, row-major.
 * Host only. */
int32_t fg_rows_npy(const char *path, int32_t *n_rows, int32_t *width, int32_t *rows);

/* fg_forward on device buffers, enqueued on `stream` (a hipStream_t, NULL =
 * the handle's stream) without host synchronisation. d_logits may be NULL
 * (the handle keeps them in its workspace); d_targets/d_nll as above. */
int32_t fg_forward_dev(fg_model *m, const int32_t *d_ids, int32_t B, int32_t T,
                       float *d_logits, const int32_t *d_targets, float *d_nll,
                       void *stream);

/* KV cache for B sequences of up to maxT positions, fp32, resident in HBM
 * (replaces the caller-owned host cache_k/cache_v of fortran_kv.f90:9-12). */
int32_t fg_kv_create(fg_model *m, int32_t B, int32_t maxT, fg_kv **out);
/* The same with flags: FG_KV_BF16 keeps K and V as bf16 (RNE of the fp32
 * values the reference stores), half the bytes of every cached step; the
 * attention of a chunk then also sees the rounded K and V. No counterpart in
 * the reference (whose cache is fp32); fg_kv_create is flags = 0. The B=1
 * persistent decode loop runs on fp32 caches only. */
enum { FG_KV_BF16 = 1 };
int32_t fg_kv_create_ex(fg_model *m, int32_t B, int32_t maxT, int32_t flags, fg_kv **out);
int32_t fg_kv_destroy(fg_kv *kv);
/* cache_len in/out of gpt_step: the number of filled positions. set_len
 * rolls the length back (or forward again) within the positions this cache
 * has computed; a length past them fails with FG_EARG (those rows were
 * never written). */
int32_t fg_kv_len(const fg_kv *kv, int32_t *len);
int32_t fg_kv_set_len(fg_kv *kv, int32_t len);
/* Copy the cache back in the reference layout (L, B, maxT, KVH*hd) fp32
 * (a bf16 cache widened). */
int32_t fg_kv_read(fg_kv *kv, float *k_out, float *v_out);

/* gpt_step (src/lib/fortran_kv.f90:26-149) for B sequences at position
 * cache_len: ids (B), logits (B*V, nullable), next_ids (B, nullable) =
 * greedy argmax (src/lib/sample.f90:271-277). Advances cache_len by 1. */
int32_t fg_step(fg_model *m, fg_kv *kv, const int32_t *ids, float *logits, int32_t *next_ids);

/* fg_step on device buffers that allocates nothing: no counterpart in the
 * reference; for callers that cannot allocate device memory (code under
 * hipGraph capture, tight serving loops, harnesses that forbid hipMalloc).
 * d_ids (B, device) in; d_logits (B*V, device) out; d_next (B, device,
 * nullable) = the argmax of each row. Enqueued on `stream` (NULL = the
 * handle's stream) without host synchronisation; advances cache_len by 1.
 * The kv's B must take the single-row path (B <= 4 at depth-12's dims;
 * FG_EARG otherwise). The step's activations and attention partials live
 * in one 4 MiB device array the library holds per GPU (FG_EARG when B and
 * maxT need more); every call on a GPU shares it. A call on another stream
 * while an earlier call's work may still be queued or running fails with
 * FG_EBUSY (calls on one stream are ordered by it); calls made under graph
 * capture are not tracked, and ordering their replays against other calls
 * on the GPU is the caller's part. The array needs no clearing: each kernel
 * writes what it reads later, and the attention's arrival counters at its
 * start are zero when the library loads and left zero by every launch.
 * Invalid ids are not checked on the host (they embed to NaN). */
int32_t fg_step_dev_noalloc(fg_model *m, fg_kv *kv, const int32_t *d_ids, float *d_logits,
                            int32_t *d_next, void *stream);

/* gpt_step_multi (src/lib/fortran_kv.f90:160-289): TB tokens of each of the
 * B sequences at positions cache_len..cache_len+TB-1; logits (B*TB*V,
 * nullable), next_ids (B, nullable) = argmax of each sequence's last row.
 * Advances cache_len by TB. */
int32_t fg_step_multi(fg_model *m, fg_kv *kv, const int32_t *ids, int32_t TB, float *logits,
                      int32_t *next_ids);

/* The greedy loop of src/app/chat_text.f90:423-462 (plain argmax, no byte
 * mask): n_steps cached steps fed back on the device, starting from ids
 * (B). ids_out (n_steps*B) receives the chosen ids; logits_out
 * (n_steps*B*V) is optional. */
int32_t fg_decode_greedy(fg_model *m, fg_kv *kv, const int32_t *ids, int32_t n_steps,
                         int32_t *ids_out, float *logits_out);

/* Greedy speculative decoding (temperature 0), the --spec loop of
 * src/app/chat_text.f90:293-422: prompt-lookup drafts (lookup_draft,
 * src/lib/fortran_spec.f90:62-92), one verification pass over the pending
 * id and k_eff drafts (gpt_step_multi), the accept rule (accept_prefix,
 * fortran_spec.f90:41-52), and the sliding-window controller that pauses
 * drafting for `probe` plain steps when a window of `probe` passes accepted
 * fewer than min_acc drafts per pass. */
typedef struct fg_spec_cfg {
  int32_t k;     /* drafts per verification pass, 1..15 (--spec)           */
  int32_t match; /* lookup match length in ids, >= 1 (--match)             */
  int32_t probe; /* controller window, passes, >= 1 (--spec-probe)         */
  float min_acc; /* pause threshold, mean accepted drafts (--spec-min-acc) */
} fg_spec_cfg;

typedef struct fg_spec_stats {
  int64_t passes;   /* verification passes                                  */
  int64_t accepted; /* drafts accepted, summed over passes                  */
  int64_t proposed; /* drafts verified (k_eff), summed over passes          */
  int64_t plain;    /* single plain steps (no lookup match, or paused)      */
  int64_t pauses;   /* times the controller paused drafting                 */
} fg_spec_stats;

/* ids holds n_total slots; ids[0:n_known] are known and the cache (B = 1)
 * holds n_known-1 positions (the prompt minus its last id, which is
 * pending). Fills ids[n_known:n_total] with the target's greedy stream,
 * leaves n_total-1 positions cached. Every verification row is computed as
 * fg_step computes that position, so the stream equals fg_decode_greedy's
 * bit for bit. stats is nullable. */
int32_t fg_decode_spec(fg_model *m, fg_kv *kv, int32_t *ids, int32_t n_known, int32_t n_total,
                       const fg_spec_cfg *cfg, fg_spec_stats *stats);

/* accept_prefix (src/lib/fortran_spec.f90:41-52): n_accept = length of the
 * longest prefix of draft[0:k] equal to targmax, correction =
 * targmax[n_accept] (targmax holds k+1 ids). Host only. */
int32_t fg_spec_accept(const int32_t *draft, const int32_t *targmax, int32_t k,
                       int32_t *n_accept, int32_t *correction);

/* lookup_draft (src/lib/fortran_spec.f90:62-92) over the p known ids:
 * the continuation (at most k ids, never past ids[p-1]) of the most recent
 * earlier occurrence of the last min(m, p-1) ids; n_draft = 0 on a miss.
 * Host only. */
int32_t fg_spec_draft(const int32_t *ids, int32_t p, int32_t m, int32_t k, int32_t *draft,
                      int32_t *n_draft);

/* Token sampling, sample_next of src/lib/sample.f90:153-233 with
 * chat_text's options (src/app/chat_text.f90:118-128): presence/frequency
 * penalties over the ids generated so far, or over the last pwin of them
 * with a length penalty on id 0; the repetition penalty; the no-repeat
 * n-gram ban; the byte-level mask; then argmax (temp <= 0) or a nucleus draw
 * from softmax(logits / temp) with the xorshift64* generator
 * (sample.f90:15-28). Vocabularies up to 8192 ids. */
typedef struct fg_sample_cfg {
  float temp;         /* <= 0: first-max argmax, no draw (--temp)             */
  float topp;         /* nucleus mass; >= 1 keeps every id (--topp)           */
  float pres, freq;   /* presence and frequency penalties (--pres, --freq)    */
  float rep;          /* repetition penalty, active above 1 (--rep)           */
  float plen;         /* length penalty on id 0 within the window (--plen)    */
  int32_t pwin;       /* > 0: penalties over the last pwin ids only (--pwin)  */
  int32_t nblock;     /* >= 2: ban ids completing a seen n-gram (--nblock)    */
  int32_t byte_space; /* nonzero: only ids 0..127 and 256..511 (--space byte) */
} fg_sample_cfg;

/* sample_next on the device for one host row logits[0:V]: gen[0:ngen] the
 * ids generated so far, *state the generator state (int64, advanced in
 * place only when a draw is made), *id the 0-based id. */
int32_t fg_sample(fg_model *m, const float *logits, int32_t V, const int32_t *gen, int32_t ngen,
                  const fg_sample_cfg *cfg, int64_t *state, int32_t *id);

/* The plain decode loop of src/app/chat_text.f90:423-462 with sample_next,
 * on the device: ids holds n_total slots, ids[0:n_known] known, the cache
 * (B = 1) holds n_known-1 positions; fills ids[n_known:n_total] (history
 * for the penalties = the ids generated in this call), advances *state,
 * leaves n_total-1 positions cached. With temp <= 0 and no penalties it is
 * fg_decode_greedy's stream. */
int32_t fg_decode_sample(fg_model *m, fg_kv *kv, int32_t *ids, int32_t n_known, int32_t n_total,
                         const fg_sample_cfg *cfg, int64_t *state);

/* Handle options (no counterpart in the reference, which has one CPU path).
 *
 * FG_OPT_FUSED_DECODE: 1 (the default) lets fg_decode_greedy run a B=1 loop
 * on an fp32 cache as ONE persistent launch (all layers, lm_head and the
 * argmax of every step; the weights stream through LDS ahead of their use,
 * activations pass between workgroups through epoch-tagged slots), for the
 * model shapes the library compiles it for (head_dim 128, d_ff = 4
 * d_model), on a device of 256 CUs in 8 XCDs that allows cooperative
 * launches: one KV head per query head with d_model 768, 6 heads and vocab
 * 8192, or d_model 256, 2 heads and vocab 1024, positions below 2048 (from
 * 128 positions on a head's attention is split over 18 workgroups); two KV
 * heads shared by the query heads with d_model 1280, 10 heads and vocab
 * 8192 (positions below 4096) or d_model 512, 4 heads and vocab 1024
 * (below 1024). 0 keeps the captured per-kernel steps. Both paths compute
 * the same functions of the same inputs; their fp32 sums run in different
 * orders.
 *
 * FG_OPT_FORWARD_F16: 1 runs fg_forward / fg_forward_dev / fg_eval_bpb
 * passes of more than 128 token rows as single-term fp16 MFMA work: one
 * fp16 operand plane for the activations instead of the bf16 hi/lo pair,
 * weights from an fp16 copy (each bf16 weight times a power of 2, exact for
 * every weight above ~2^-31 x that scale's headroom), one MFMA per product
 * instead of 2 (linears) or 3 (attention). Logits move by ~4e-4 x max|logit|
 * instead of ~5e-6; passes that fill a KV cache (fg_step_multi) keep the
 * split format. 0 (the default) is the split format everywhere. Enabling it
 * makes the fp16 copy (the weight arena's size again) and fails with
 * FG_EARG when the weights exceed the fp16 range; disabling it waits for
 * the device's queued work (any stream) and frees the copy. */
enum { FG_OPT_FUSED_DECODE = 1, FG_OPT_FORWARD_F16 = 2 };
int32_t fg_set_option(fg_model *m, int32_t key, int32_t value);
/* *value = the option's effective value (for FG_OPT_FUSED_DECODE: 1 when
 * the persistent decode is set up and enabled); why (nullable, len bytes)
 * receives the reason when it is not available. */
int32_t fg_get_option(fg_model *m, int32_t key, int32_t *value, char *why, int32_t len);

/* Block until the handle's queued work is done. Returns FG_ERANGE (once)
 * when a single-term fp16 pass queued through fg_forward_dev since the last
 * report overflowed fp16 (FG_OPT_FORWARD_F16; a pass on a caller stream is
 * covered once that stream has been synchronised). The host-buffer entry
 * points (fg_forward, fg_forward_pos, fg_eval_bpb) report their own pass's
 * overflow as their return code. */
int32_t fg_sync(fg_model *m);

/* Kernel timing, the device-side counterpart of chat_text --stats
 * (src/app/chat_text.f90:250-282,465-468). With timing on, every launch the
 * handle makes outside graph capture (fg_decode_greedy then runs its steps
 * eagerly) is bracketed by HIP events on the stream it runs on, and tagged
 * with its kernel kind and its algorithmic flops and HBM bytes. Enabling or
 * disabling clears the records. fg_timing_read sums one kind. */
enum {
  FG_K_GEMM = 0,        /* MFMA GEMM (prefill, batched decode linears)   */
  FG_K_GEMV = 1,        /* small-M GEMV (B=1 decode linears)             */
  FG_K_ATTN_CHUNK = 2,  /* causal chunk attention (prefill)              */
  FG_K_ATTN_DECODE = 3, /* single-query attention (decode)               */
  FG_K_OTHER = 4,       /* embedding+norm, argmax, NLL                   */
  FG_K_DECODE_FUSED = 5, /* the persistent B=1 greedy loop (one launch)  */
  FG_K_NKINDS = 6
};
int32_t fg_timing(fg_model *m, int32_t enable);
int32_t fg_timing_read(fg_model *m, int32_t kind, int64_t *launches, double *ms, double *flops,
                       double *bytes);

/* Bytes of HBM the handle holds (weights, workspace, tables). Diagnostic,
 * the counterpart of gpublas_count / gpublas_bufs (gpu_shim.cpp:172-186). */
int32_t fg_model_bytes(const fg_model *m, int64_t *weight_bytes, int64_t *work_bytes);

#ifdef __cplusplus
}
#endif
#endif
