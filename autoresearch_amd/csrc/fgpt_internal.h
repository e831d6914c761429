// fgpt_internal.h -- engine-internal types and kernel launchers (not part of
// the C ABI). Everything here is gfx950-only HIP.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <string>

#include "../../include/fgpt.h"

namespace fgpt {

// Kernel timing: while a timed region is open on this thread (the engine's
// fg_timing), the launches in it carry the region's events in their dispatch
// packet (hipExtLaunchKernelGGL): the first launch the start event, every
// launch the stop event. The events then hold the kernels' own begin and end
// timestamps, not the stream's, so a region's time does not include the
// dispatch gap in front of its first kernel.
struct LaunchEvents {
  hipEvent_t start = nullptr, stop = nullptr;
  int n = 0;
};
inline LaunchEvents& launch_events() {
  static thread_local LaunchEvents e;
  return e;
}

// Set the calling thread's error (code + message, see fg_last_error); returns code.
int32_t set_error(int32_t code, const char* msg);

typedef uint16_t bf16_t;  // raw bf16 bits in HBM

struct Dims {
  int L, D, H, KH, hd, V, dff;
  float eps;
  int qd() const { return H * hd; }
  int kvd() const { return KH * hd; }
  int nqkv() const { return (H + 2 * KH) * hd; }
};

// Validate the public dims against what the kernels support and fill Dims.
int32_t check_dims(const fg_dims* in, Dims* d);

// Weight arena in HBM (bf16), one allocation:
//   per layer l: Wqkv[(H+2KH)*hd][D]  rows permuted, see qkv_row_of()
//                Wproj[D][H*hd], Wfc[4D][D], Wproj2[D][4D]
//   then lm_head[V][D], wte[V][D]
struct Weights {
  bf16_t* base = nullptr;
  size_t bytes = 0;
  size_t layer_stride = 0;  // elements
  size_t off_qkv = 0, off_proj = 0, off_fc = 0, off_proj2 = 0;  // within a layer
  bf16_t* lm = nullptr;
  bf16_t* wte = nullptr;
  const bf16_t* qkv(int l) const { return base + l * layer_stride + off_qkv; }
  const bf16_t* proj(int l) const { return base + l * layer_stride + off_proj; }
  const bf16_t* fc(int l) const { return base + l * layer_stride + off_fc; }
  const bf16_t* proj2(int l) const { return base + l * layer_stride + off_proj2; }
};

// Row order of the fused QKV matrix. Within every q or k head the rows are
// interleaved in rotation pairs (d, d+hd/2) so one GEMV unit or one pair of
// adjacent GEMM columns holds both halves RoPE mixes. Stored row s of a
// head maps to head dimension: s even -> s/2, s odd -> hd/2 + s/2.
__host__ __device__ inline int pair_dim(int s, int hd) {
  return (s & 1) ? (hd / 2 + (s >> 1)) : (s >> 1);
}

// Columns of one log-sum-exp partial of lm_head's cross-entropy epilogue
// (one wavefront row of the 128x256 register-epilogue tile).
constexpr int NLL_GROUP_COLS = 128;

// Activation workspace for up to `rows` token rows.
struct Work {
  int64_t rows = 0;
  float* x = nullptr;       // residual stream [rows][D]
  float* q = nullptr;       // rotated queries [rows][H*hd]
  float* ao = nullptr;      // attention output [rows][H*hd]
  float* h = nullptr;       // relu2(fc) [rows][4D]
  float* logits = nullptr;  // [rows][V]
  int32_t* ids = nullptr;   // [rows]
  int32_t* tgt = nullptr;   // [rows]
  float* nll = nullptr;     // [rows]
  float* stat = nullptr;    // [rows] per-row scratch (argmax values etc.)
  int32_t* amax = nullptr;  // [rows]
  // the MFMA path's activations in the split format (hi plane, lo plane
  // rows*width elements later) and the residual's per-row partial sums of
  // squares [rows][D/64]
  uint16_t* xs = nullptr;   // residual [rows][D]
  uint16_t* aos = nullptr;  // attention output [rows][H*hd]
  uint16_t* hs = nullptr;   // relu2(fc) [rows][4D]
  float* ssq = nullptr;
  float* part = nullptr;    // split-K partial sums of the small-M GEMMs
  float* nllp = nullptr;    // lm_head's log-sum-exp partials [rows][V/NLL_GROUP_COLS][2]
};

struct KVCacheDev {
  int B = 0, maxT = 0;
  float* k = nullptr;  // [L][B][maxT][KH*hd]
  float* v = nullptr;
};

// ------------------------------------------------------------ launchers
// All launches go to `s`; shapes are validated by the caller (engine).

// x[r] = rmsnorm(wte[ids[r]]); when xs is set, also the split copy of x
// (hi plane, lo plane `plane` elements later) and ssq[r] = sum_k x[r][k]^2.
// d_rows (nullable): rows live this launch, read on the device.
// dst[i] = fp16(bf16 src[i] * scale) (scale a power of 2), i < n.
void launch_to_f16(hipStream_t s, const bf16_t* src, uint16_t* dst, int64_t n, float scale);
// p[0..n) = 0 by a kernel (capturable, unlike a memset node).
void launch_zero_u32(hipStream_t s, uint32_t* p, int n);

void launch_embed_norm(hipStream_t s, const Dims& d, const bf16_t* wte, const int32_t* ids,
                       int64_t rows, float* x, uint16_t* xs = nullptr, int64_t plane = 0,
                       float* ssq = nullptr, const int32_t* d_rows = nullptr, bool f16 = false);

// GEMV family for M <= GEMV_MAX_ROWS token rows, fp32 activations x bf16
// weights (the MFMA GEMM shares the argument block).
constexpr int GEMV_MAX_ROWS = 16;
enum GemvEpi { GV_QKV = 0, GV_RESID = 1, GV_RELU2 = 2, GV_STORE = 3 };
struct GemvArgs {
  const float* x;   // [M][K] input rows
  const bf16_t* w;  // [N][K]
  int M, N, K;
  const int32_t* d_M;  // GEMV only (nullable): rows live this launch, <= M, read on
                       // the device (rows past it are neither read nor written)
  int norm;         // apply rmsnorm(x) (scale by inv-rms of each x row)
  float eps;
  float* y;         // output [M][N] (RESID: y += ..., in place)
  // QKV epilogue
  const float* cosb;
  const float* sinb;
  int pos0;         // position of row 0 (row m is at pos0 + m % T)
  int T;            // rows per sequence
  float* kc;        // KV cache of this layer, [B][maxT][KH*hd] (nullable); with
  float* vc;        // kv16 its elements are bf16 (the pointers then address uint16_t)
  int kv16;
  int maxT;
  int H, KH, hd;
  // bf16 hi/lo copies for the MFMA chunk attention (nullable):
  // qs [B][H][T][hd], ks [B][KH][npos][hd], vt [B][KH][hd][npos]
  uint16_t* qs;
  uint16_t* ks;
  uint16_t* vt;
  int npos;
  int64_t q_plane, kv_plane;  // elements between the hi and lo planes
  // MFMA GEMM operands in the split format (bf16 hi plane, lo plane
  // `*_plane` elements later). xs: A rows [M][K]. ssq_in: per-row partial
  // sums of squares of A, [M][ssq_n] (the row norm). ys: split output
  // (RESID: the updated residual, RELU2: relu^2). ssq_out: RESID only,
  // per-row partial sums of squares of the updated residual, one per
  // N tile, [M][N / tile_n].
  const uint16_t* xs;
  int64_t xs_plane;
  const float* ssq_in;
  int ssq_n;
  uint16_t* ys;
  int64_t ys_plane;
  float* ssq_out;
  // split-K scratch for small-M GEMMs (nullable): the K-split partial sums,
  // [splits][M][N] fp32, reduced in split order by a second kernel that
  // applies the norm and the epilogue (RESID then writes one ssq partial per
  // row and 512 columns). Sized by gemm_splitk_floats.
  float* part;
  // single-term fp16 pass (MFMA GEMM only, more than 128 rows): A is one fp16
  // plane (xs), W the fp16 copy of the weights scaled by 1 / wscale (a power
  // of 2), the outputs' operand planes fp16 too
  int f16;
  float wscale;
  // lm_head with the cross-entropy to follow (STORE only, nullable): per row
  // and NLL_GROUP_COLS-column group, the group's maximum logit and sum of
  // exp(logit - maximum), [M][N/NLL_GROUP_COLS][2]; the GEMM then runs where
  // it can write them (gemm_store_nll says when)
  float* nll_part;
  // single-term fp16 pass (nullable): set to 1 by any epilogue whose fp16
  // operand store would round a value to inf (|v| >= 65520 or not finite)
  uint32_t* ovf;
};
void launch_gemv(hipStream_t s, GemvEpi epi, const GemvArgs& a);

// MFMA GEMM, C[M][N] = epi(rowscale * (A[M][K] . W[N][K]^T)), A in the
// split format (xs), W bf16, fp32 accumulation. K must be a multiple of 128.
void launch_gemm(hipStream_t s, GemvEpi epi, const GemvArgs& a);
// Number of ssq_out partials per row that a RESID GEMM of M x N x K
// writes (when it is given split-K scratch, if it splits).
int gemm_ssq_parts(int64_t M, int N, int K);
// Floats of split-K scratch an M x N x K GEMM needs (0: it does not split).
int64_t gemm_splitk_floats(int64_t M, int N, int K);

// Causal chunk attention of T queries at positions pos0..pos0+T-1 against
// keys 0..pos0+t, on MFMA from the bf16 hi/lo planes (layouts of
// GemvArgs::qs/ks/vt; npos = padded row stride of the key planes, a
// multiple of 64, with finite values in the padding) -> y [B][T][H*hd]
// (or its split format in ys). Long key ranges are split over workgroups;
// their partial results go through `scratch` (attn_scratch_floats floats)
// and a merge kernel on the same stream.
int64_t attn_scratch_floats(const Dims& d, int B, int T, int pos0);
// Compute units of the current device (cached per device).
int cu_count();
// Raise kernel fn's dynamic LDS limit to `bytes` on the current device. The
// limit is an attribute of the function on each device, so it is set once
// per device (bit d of *done); devices past 63 set it at every launch.
inline void raise_lds_once(const void* fn, size_t bytes, std::atomic<uint64_t>* done) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  const uint64_t bit = dev >= 0 && dev < 64 ? 1ull << dev : 0;
  if (bit && (done->load(std::memory_order_acquire) & bit)) return;
  (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (bit) done->fetch_or(bit, std::memory_order_release);
}
// pos_cnt (nullable): one count per work item, attn_items(d, B, T, pos0) of
// them, item i belonging to (sequence * H + head) = i % (B * H): how many of
// the item's causal scores q.k are > 0 (src/lib/fortran_attn.f90:247-300).
int64_t attn_items(const Dims& d, int B, int T, int pos0);
void launch_attn_mfma(hipStream_t s, const Dims& d, const uint16_t* qs, const uint16_t* ks,
                      const uint16_t* vt, int B, int T, int npos, int pos0, int64_t q_plane,
                      int64_t kv_plane, float* scratch, float* y, uint16_t* ys = nullptr,
                      int64_t ys_plane = 0, bool f16 = false, uint32_t* pos_cnt = nullptr);
// Fill the hi/lo key/value planes for cache positions [0, n) from the cache
// of one layer ([B][maxT][KH*hd], fp32, or bf16 with kv16: lo planes zero).
void launch_split_cache(hipStream_t s, const Dims& d, const void* kc, const void* vc, bool kv16,
                        int B, int maxT, int n, int npos, int64_t kv_plane, uint16_t* ks,
                        uint16_t* vt);

// Variants whose position / cache length comes from device memory (so a
// captured decode step replays at successive positions).
void launch_gemv_pos(hipStream_t s, GemvEpi epi, const GemvArgs& a, const int32_t* d_pos);
void launch_gemm_pos(hipStream_t s, GemvEpi epi, const GemvArgs& a, const int32_t* d_pos);
// Single-query attention over the cache: q [B*qpr][H][hd] -> y [B*qpr][H*hd]
// (or its split format in ys). Query row j of sequence b (row b*qpr + j)
// sits at position len-1+j of cache b and sees positions 0..len-1+j: qpr
// consecutive single steps in one launch. d_len (nullable) holds the cache
// length before the step (the first query is at *d_len), else len is the
// length including the first query. scratch: attn_decode_scratch_floats(d,
// B*qpr, maxT) floats. cnt (nullable): attn_decode_counters(d, B*qpr)
// arrival counters, zero before the first launch and left zero by every
// launch; with them a multi-chunk step merges its chunks in the same launch,
// else a merge kernel follows. d_rows (nullable): query rows live this
// launch (of B*qpr), on the device.
int64_t attn_decode_scratch_floats(const Dims& d, int B, int maxT);
inline int64_t attn_decode_counters(const Dims& d, int rows) { return (int64_t)rows * d.H; }
// The QKV GEMM's split-K partial sums, left for the single-query attention
// to finish (sum in split order, row norm, RoPE, the k/v append) instead of
// a reduce launch: part [splits][rows][N], N = (H + 2 KH) hd in the stored
// column order; the norm from ssq_in [rows][ssq_n] over K inputs.
struct QkvFold {
  const float* part = nullptr;
  int splits = 0, rows = 0, N = 0, K = 0, ssq_n = 0;
  const float* ssq_in = nullptr;
  float eps = 0.f;
  const float* cosb = nullptr;
  const float* sinb = nullptr;
};
// Whether launch_attn_decode_pos for one query row per sequence (no
// d_rows; replayed: d_len set) runs the kernel that takes a QkvFold.
bool attn_decode_takes_qkv(const Dims& d, int B, int maxT, bool replayed, int len, bool kv16);
// The split-K GEMM alone (no reduce): its partial sums into a.part. Returns
// the split count, or 0 (nothing launched) when this GEMM is not split.
int launch_gemm_partials(hipStream_t s, GemvEpi epi, const GemvArgs& a, const int32_t* d_pos);
void launch_attn_decode_pos(hipStream_t s, const Dims& d, const float* q, const void* kc,
                            const void* vc, bool kv16, int B, int maxT, const int32_t* d_len,
                            int len, float* scratch, uint32_t* cnt, float* y,
                            uint16_t* ys = nullptr, int64_t ys_plane = 0, int qpr = 1,
                            const int32_t* d_rows = nullptr, const QkvFold* qf = nullptr);
// argmax into out; with d_len/d_len0 set, also into out2[(len-len0)*rows +
// row] (and the logits row into lgs_out at that slot, when set), then
// *d_len += 1.
void launch_argmax_step(hipStream_t s, const float* logits, int64_t rows, int V, int32_t* out,
                        int32_t* out2, int32_t* d_len, const int32_t* d_len0, float* lgs_out);

// GEMV-path greedy step end (rows <= 4, one block): argmax of each row into
// ids and out2 (and the logits row into lgs_out) as launch_argmax_step does,
// then x[row] = rmsnorm0(wte[id]) for the next step, then *d_len += 1.
void launch_greedy_tail(hipStream_t s, const Dims& d, const float* logits, int rows,
                        const bf16_t* wte, int32_t* ids, int32_t* out2, int32_t* d_len,
                        const int32_t* d_len0, float* lgs_out, float* x);

// Per-row argmax (first max) of logits [rows][V] -> out [rows].
void launch_argmax(hipStream_t s, const float* logits, int64_t rows, int V, int32_t* out);
// Per eval row (rows of T positions): byte-weighted nats and byte count
// with the token byte-length table tbytes (targets already range-checked).
void launch_bpb_rows(hipStream_t s, const float* nll, const int32_t* tgt, int rows, int T,
                     const int32_t* tbytes, double* row_nats, long long* row_bytes);
// Per-row nll = logsumexp - logit[tgt].
void launch_nll(hipStream_t s, const float* logits, const int32_t* tgt, int64_t rows, int V,
                float* out);
// The same from lm_head's per-row partials (GemvArgs::nll_part,
// V/NLL_GROUP_COLS groups a row) and the target's logit.
void launch_nll_parts(hipStream_t s, const float* logits, const float* parts, const int32_t* tgt,
                      int64_t rows, int V, float* out);
// Whether an lm_head GEMM of M rows over a vocabulary of N writes the
// log-sum-exp partials when asked (1025 to 4096 rows, N a multiple of 256).
bool gemm_store_nll(int64_t M, int N);

// ---- greedy speculative decoding
// host side (fgpt_spec.hip)
int spec_accept_prefix(const int32_t* draft, const int32_t* targ, int k, int32_t* correction);
int spec_lookup_draft(const int32_t* ids, int p, int m, int k, int32_t* d);

// Device-resident state of the draft/verify loop for one sequence whose ids
// live in a device array. A round is k_spec_draft (lookup, the pass's ids
// and live row count), the verification pass (rows single steps at cache
// length `len`), then k_spec_commit (argmax of each row, the accept rule,
// the commit, the controller). Rounds after pp reaches n_total do nothing.
struct SpecDev {
  int32_t pp;          // known ids (ids[pp-1] pending, pp-1 positions cached)
  int32_t n_total;     // stop when pp reaches it
  int32_t len;         // cache length before this round's pass (pp-1)
  int32_t rows;        // live rows of this round's pass; 0 once done
  int32_t keff;        // drafts verified this round
  int32_t spec_round;  // this round verifies drafts (else a plain step)
  int32_t mode_spec, plain_left, npass_w, nacc_w;  // the controller window
  int32_t k, match, probe;
  float min_acc;
  int32_t passes, accepted, proposed, plain, pauses;
  int32_t inp[GEMV_MAX_ROWS];  // the pass's ids: pending id, then drafts
};
void launch_spec_draft(hipStream_t s, SpecDev* st, const int32_t* ids);
void launch_spec_commit(hipStream_t s, SpecDev* st, const float* logits, int V, int32_t* ids);

// ---- token sampling (kern_sample.hip): sample_next of src/lib/sample.f90
struct SampleCfg {
  float temp, topp, pres, freq, rep, plen;
  int32_t pwin, nblock, byte_space;
};
constexpr int SAMPLE_MAX_V = 8192;  // the row, its sort keys and sums sit in LDS
// Device state of the sampling loop for one sequence (ids in a device array):
// each step samples ids[pp] from the pass over ids[pp-1] = inp[0].
struct SampleDev {
  int32_t pp, n_total, len, n_known;
  int64_t rng;
  int32_t inp[2];
  SampleCfg cfg;
};
void launch_sample_one(hipStream_t s, const float* logits, int V, const int32_t* gen, int ngen,
                       const SampleCfg& c, int64_t* state, int32_t* out);
void launch_sample_step(hipStream_t s, SampleDev* sd, const float* logits, int V, int32_t* ids);

// ---- B=1 greedy decode as one persistent launch (kern_fused.hip)
// 256 workgroups, one per CU, in 8 groups of 32 (the workgroups of one XCD,
// found from XCC_ID at the start of the launch). XCD g < H computes head g's q/k/v, attention and its share of
// c_proj; every XCD computes 1/8 of c_fc and the matching split of
// c_proj2. Workgroups hand values over through "exchange slots": 8 bytes,
// the fp32 value below a 32-bit epoch that names the hand-over, so a reader
// polls until the epoch it expects is there and never takes a stale value.
// Each workgroup streams its weight slices into LDS one pseudo-layer ahead
// (the 12 layers, then lm_head) from a weight copy laid out per workgroup.
constexpr int FUSED_NWG = 256;  // workgroups (CUs)
constexpr int FUSED_NX = 8;     // XCDs
constexpr int FUSED_NC = 32;    // workgroups per XCD
constexpr int FUSED_MAX_LEN = 2048;  // attention positions a step may see
// From this many positions on, a head's attention is split over
// FUSED_SPLIT_WG workgroups of its XCD (each takes every FUSED_SPLIT_WG-th
// position) and their partial results meet in one more hand-over within the
// XCD; below it every workgroup of the XCD computes the whole attention of
// the head itself.
constexpr int FUSED_SPLIT_MIN = 128;
// 18: one batch of cache rows per position group up to 18 x 8 groups x 8
// = 1 152 positions (chat_text's 1 024-position contexts and a little
// beyond); at 1 032-1 094 positions 154.1 against 162.9 us a token with 16
// (some workgroups then fetched a second batch), 14.6 us a layer with 8;
// more would take the kernel past its 256 VGPRs (the merge gathers
// FUSED_SPLIT_WG partials of hd + 2 slots at once)
constexpr int FUSED_SPLIT_WG = 18;

struct FusedLayout {
  bool ok = false;
  // 0: one KV head per query head (kern_fused.hip); 1: two KV heads, each
  // shared by a group of query heads (kern_fused_gqa.hip)
  int kind = 0;
  int max_len = FUSED_MAX_LEN;  // attention positions a step may see
  int64_t off_xp = 0;           // (kind 1) slot offset of the XCD-level attention partials
  int QR, C, FR, HN, LR;  // rows per workgroup: qkv, proj/proj2 outputs, fc, proj2 K, lm_head
  int64_t wq, wp, wf, w2;   // segment byte offsets within a layer slice
  int64_t slice, lmb;       // bytes of a layer slice and of the lm_head slice
  int64_t wbuf;             // LDS bytes of one weight buffer
  int64_t cu_bytes;         // bytes of one workgroup's region of the fused arena
  int64_t lds_bytes;        // dynamic LDS of the kernel
  int64_t slots;            // exchange slots (8 bytes each)
  int64_t off_ql, off_pp, off_xl, off_hl, off_p2, off_lm, off_ap;  // slot offsets
};
// The layout for dims d; ok = false (with the reason in *why) when the
// fused kernel does not serve them.
FusedLayout fused_layout(const Dims& d, const char** why);
// The same for two KV heads shared by groups of query heads (kind 1).
FusedLayout fused_layout_gqa(const Dims& d, const char** why);
// Copy the main arena's weights (host bf16, the Weights layout) into the
// fused layout (host buffer of FUSED_NWG * cu_bytes bytes).
void fused_pack(const Dims& d, const FusedLayout& f, const Weights& w, const bf16_t* host_main,
                bf16_t* host_fused);
void fused_pack_gqa(const Dims& d, const FusedLayout& f, const Weights& w, const bf16_t* host_main,
                    bf16_t* host_fused);

struct FusedArgs {
  const bf16_t* arena;  // fused weight copy
  const bf16_t* wte;    // [V][D]
  const float* cosb;
  const float* sinb;
  float* kc;            // cache [L][maxT][KH*hd] (B = 1)
  float* vc;
  int maxT, len0, n_steps;
  const int32_t* d_id0;  // the first input id
  int32_t* ids_out;      // [n_steps]
  float* logits_out;     // [n_steps][V] or null
  uint64_t* slots;
  uint32_t ep_base;      // epochs of this launch start here
  uint32_t* err;         // nonzero after the launch: a hand-over timed out (1) or
                         // an XCD held more than 32 workgroups (2); zeroed before
  uint32_t* cnt;         // [8] workgroups placed per XCD so far; zeroed before
  int D, H, KH, L, V, dff;
  float eps;
  uint64_t* trace;       // null, or [256][L+1][32] phase timestamps of step trace_step
  int trace_step;
};
// Epochs one launch of n_steps uses (the next launch starts past them).
uint32_t fused_epochs(const Dims& d, int n_steps);
hipError_t launch_fused_decode(hipStream_t s, const Dims& d, const FusedLayout& f,
                               const FusedArgs& a);
hipError_t launch_fused_gqa(hipStream_t s, const Dims& d, const FusedLayout& f,
                            const FusedArgs& a);

}  // namespace fgpt
