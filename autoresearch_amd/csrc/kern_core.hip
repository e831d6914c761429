// kern_core.hip -- embedding, small-M GEMV, decode attention, chunk
// attention, argmax and NLL kernels for gfx950 (64-wide wavefronts).
//
// Reference semantics (14NGiestas/autoresearch):
//   embedding + first norm  src/lib/fortran_gpt.f90:136-142, fortran_linear.f90:62-78
//   rmsnorm0                src/lib/fortran_rmsnorm.f90:40-60
//   y = x W^T               src/lib/fortran_blas.f90:39-57
//   rope_4d (half split)    src/lib/fortran_rope.f90:25-52
//   cache append            src/lib/fortran_kv.f90:112-116,292-300
//   attn_step / attn_chunk  src/lib/fortran_attn.f90:317-425
//   relu2                   src/lib/fortran_attn.f90:697-710
//   greedy argmax           src/lib/sample.f90:271-277
//   per-position NLL        src/app/eval_bpb.f90:165-181
#include <float.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>

#include "fgpt_internal.h"
#include "kern_common.h"
#include "kern_epi.h"

namespace fgpt {

// ------------------------------------------------------------ block reduce
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < NW; ++i) t += red[i];
  return t;
}

template <int NW>
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) t = fmaxf(t, red[i]);
  return t;
}

// ------------------------------------------------------------ embedding
// x[r] = rmsnorm0(wte[ids[r]]): the embedding lookup and the norm that
// gpt_forward copies back into the residual (fortran_gpt.f90:136-142).
// An id outside [0, V) (possible only through the device-pointer entry
// point, the host ones validate) yields a NaN row instead of a wild read.
// xs (nullable) takes the split copy of x (bf16 hi, lo `plane` later) or,
// for a single-term fp16 pass (P16), one fp16 plane.
template <bool P16>
__global__ __launch_bounds__(256) void k_embed_norm(const bf16_t* __restrict__ wte,
                                                    const int32_t* __restrict__ ids, int D, int V,
                                                    float eps, float* __restrict__ x,
                                                    uint16_t* __restrict__ xs, int64_t plane,
                                                    float* __restrict__ ssq,
                                                    const int32_t* __restrict__ d_rows) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  if (d_rows && r >= *d_rows) return;
  const int id = ids[r];
  if (id < 0 || id >= V) {
    for (int k = threadIdx.x; k < D; k += 256) x[r * D + k] = __builtin_nanf("");
    if (ssq && threadIdx.x == 0) ssq[r] = __builtin_nanf("");
    return;
  }
  const bf16_t* row = wte + (int64_t)id * D;
  float ss = 0.f;
  for (int k = threadIdx.x; k < D; k += 256) {
    float v = bf16_to_f32(row[k]);
    ss += v * v;
  }
  ss = block_sum<4>(ss, red);
  const float inv = 1.0f / sqrtf(ss / (float)D + eps);
  float s2 = 0.f;
  for (int k = threadIdx.x; k < D; k += 256) {
    const float v = bf16_to_f32(row[k]) * inv;
    x[r * D + k] = v;
    if (xs) put1<P16>(v, xs + r * D + k, plane);
    s2 += v * v;
  }
  if (ssq) {
    s2 = block_sum<4>(s2, red);
    if (threadIdx.x == 0) ssq[r] = s2;
  }
}

__global__ __launch_bounds__(256) void k_to_f16(const bf16_t* __restrict__ src,
                                                uint16_t* __restrict__ dst, int64_t n,
                                                float scale) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    dst[i] = f32_to_f16_rne(bf16_to_f32(src[i]) * scale);
}

__global__ __launch_bounds__(64) void k_zero_u32(uint32_t* __restrict__ p, int n) {
  for (int i = threadIdx.x; i < n; i += 64) p[i] = 0u;
}

void launch_zero_u32(hipStream_t s, uint32_t* p, int n) {
  if (n > 0) FG_LAUNCH(k_zero_u32, dim3(1), dim3(64), 0, s, p, n);
}

void launch_to_f16(hipStream_t s, const bf16_t* src, uint16_t* dst, int64_t n, float scale) {
  if (n <= 0) return;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
  FG_LAUNCH(k_to_f16, dim3((unsigned)blocks), dim3(256), 0, s, src, dst, n, scale);
}

void launch_embed_norm(hipStream_t s, const Dims& d, const bf16_t* wte, const int32_t* ids,
                       int64_t rows, float* x, uint16_t* xs, int64_t plane, float* ssq,
                       const int32_t* d_rows, bool f16) {
  if (rows <= 0) return;
  if (f16)
    FG_LAUNCH(k_embed_norm<true>, dim3((unsigned)rows), dim3(256), 0, s, wte, ids, d.D, d.V,
              d.eps, x, xs, plane, ssq, d_rows);
  else
    FG_LAUNCH(k_embed_norm<false>, dim3((unsigned)rows), dim3(256), 0, s, wte, ids, d.D, d.V,
              d.eps, x, xs, plane, ssq, d_rows);
}

// ------------------------------------------------------------ epilogues
// res: the residual y[m][r] (RESID), loaded before the dot product
template <int EPI>
__device__ __forceinline__ void single_store(const GemvArgs& a, int m, int r, float v,
                                             float res) {
  float* y = a.y + (int64_t)m * a.N + r;
  if (EPI == GV_RESID) {
    *y = res + v;
  } else if (EPI == GV_RELU2) {
    const float t = v < 0.f ? 0.f : v;
    *y = t * t;
  } else {
    *y = v;
  }
}

// ------------------------------------------------------------ GEMV
// M <= 4 token rows per wavefront (k_gemv: one group of rows; k_gemv_live:
// up to 16 live rows read on the device, in groups of four). A wavefront
// owns R weight rows at a time (R = 2 for QKV, so a rotation pair stays in
// one wavefront; else 1, for twice the wavefronts): lanes stride the rows in
// 16-byte chunks (8 bf16), so each row is read as whole, coalesced lines,
// and x comes straight from global memory (L2) in matching float4 pairs. No
// LDS and no barrier: the weight loads go out at once, and so do the
// epilogue's own loads (RoPE coefficients, the residual), so none waits
// behind the reduction. The row norm (a.norm)
// is a scale of the dot products, from sum(x^2) the same lanes accumulate
// over the chunks they read. Each (token row, weight row) result is the same
// sequence of operations whatever M is, so a row's value does not depend on
// how many rows share the launch.
// 8-term dot product, one multiply then seven fused multiply-adds in index
// order, spelled out so that every instantiation (any M, any U) rounds alike
// whatever contraction the compiler would choose for a sum of products.
__device__ __forceinline__ float dot8(const float (&u)[8], const float (&v)[8]) {
  float t = u[0] * v[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) t = fmaf(u[e], v[e], t);
  return t;
}

template <int M, int EPI, int R, int U>
__device__ __forceinline__ void gemv_rows(const GemvArgs& a, int pos0) {
  const int K = a.K, lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int nunits = (a.N + R - 1) / R, nch = K >> 3;
  for (int u = blockIdx.x * 4 + wid; u < nunits; u += gridDim.x * 4) {
    const bf16_t* wr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) wr[r] = a.w + (int64_t)min(R * u + r, a.N - 1) * K;
    float acc[R][M], ss[M];
    float e0[R][M], e1[R][M];  // RoPE cos / sin of a pair (QKV), the residual (RESID)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      ss[m] = 0.f;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        acc[r][m] = 0.f;
        e0[r][m] = e1[r][m] = 0.f;
        if (EPI == GV_QKV && (r & 1) == 0 && R * u + r < a.N)
          qkv_pair_coeffs(a, m, pos0, R * u + r, e0[r][m], e1[r][m]);
        if (EPI == GV_RESID && R * u + r < a.N) e0[r][m] = a.y[(int64_t)m * a.N + R * u + r];
      }
    }
    // U chunks per lane in flight: every load of a round goes out before the
    // first is used (a 5120-long row is 10 chunks a lane: one round at U = 10
    // instead of five dependent pairs); the chunks are summed in ascending
    // order whatever U is
    for (int c0 = lane; c0 < nch; c0 += 64 * U) {
      uint4 wv[U][R];
      float4 xa[U][M], xb[U][M];
#pragma unroll
      for (int i = 0; i < U; ++i) {
        const int c = c0 + 64 * i;
        if (c < nch) {
#pragma unroll
          for (int r = 0; r < R; ++r) wv[i][r] = *(const uint4*)(wr[r] + c * 8);
#pragma unroll
          for (int m = 0; m < M; ++m) {
            xa[i][m] = *(const float4*)(a.x + (int64_t)m * K + c * 8);
            xb[i][m] = *(const float4*)(a.x + (int64_t)m * K + c * 8 + 4);
          }
        }
      }
#pragma unroll
      for (int i = 0; i < U; ++i) {
        if (c0 + 64 * i >= nch) break;
        float f[R][8];
#pragma unroll
        for (int r = 0; r < R; ++r) unpack8(wv[i][r], f[r]);
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const float4 p = xa[i][m], q = xb[i][m];
          const float xv[8] = {p.x, p.y, p.z, p.w, q.x, q.y, q.z, q.w};
          ss[m] += dot8(xv, xv);
#pragma unroll
          for (int r = 0; r < R; ++r) acc[r][m] += dot8(f[r], xv);
        }
      }
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float inv = a.norm ? 1.0f / sqrtf(wave_sum(ss[m]) / (float)K + a.eps) : 1.f;
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r][m] = wave_sum(acc[r][m]) * inv;
    }
    if (lane == 0) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        if (EPI == GV_QKV) {
#pragma unroll
          for (int pr = 0; pr < R; pr += 2)
            if (R * u + pr < a.N)
              qkv_pair_store(a, m, pos0, R * u + pr, acc[pr][m], acc[pr + 1][m], e0[pr][m],
                             e1[pr][m]);
        } else {
#pragma unroll
          for (int r = 0; r < R; ++r)
            if (R * u + r < a.N) single_store<EPI>(a, m, R * u + r, acc[r][m], e0[r][m]);
        }
      }
    }
  }
}

template <int M, int EPI, int R, int U>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a, const int32_t* __restrict__ d_pos) {
  gemv_rows<M, EPI, R, U>(a, d_pos ? *d_pos : a.pos0);
}

// Chunks in flight per lane: rows of up to 4 chunks a lane (K <= 2048) in
// one round; longer rows (the MLP's second matrix) in rounds of 10 for one
// token row, fewer as x's registers grow with M. k_gemv and k_gemv_live
// pick U alike (gemv_long), so a row's arithmetic is the same code in both.
template <int M, bool LONG> constexpr int gemv_u() {
  return LONG ? (M == 1 ? 10 : M == 2 ? 5 : 2) : (M <= 2 ? 4 : 2);
}
inline bool gemv_long(int K) { return K > 64 * 8 * 4; }

// Up to 16 rows, the live count *a.d_M read on the device (a captured pass
// whose row count changes between replays). blockIdx.y picks a group of up
// to four rows; each group runs the exact 1-4 row body of k_gemv on its
// rows (offset x, y and positions), groups past the live count exit.
template <int EPI, bool LONG>
__global__ __launch_bounds__(256) void k_gemv_live(GemvArgs a, const int32_t* __restrict__ d_pos) {
  constexpr int R = EPI == GV_QKV ? 2 : 1;
  const int g0 = blockIdx.y * 4, ml = *a.d_M - g0;
  if (ml <= 0) return;
  const int pos0 = (d_pos ? *d_pos : a.pos0) + g0;
  a.x += (int64_t)g0 * a.K;
  a.y += (int64_t)g0 * (EPI == GV_QKV ? a.H * a.hd : a.N);
  if (ml == 1) gemv_rows<1, EPI, R, gemv_u<1, LONG>()>(a, pos0);
  else if (ml == 2) gemv_rows<2, EPI, R, gemv_u<2, LONG>()>(a, pos0);
  else if (ml == 3) gemv_rows<3, EPI, R, gemv_u<3, LONG>()>(a, pos0);
  else gemv_rows<4, EPI, R, gemv_u<4, LONG>()>(a, pos0);
}

template <int M, int EPI, int R>
static void gemv_grid(hipStream_t s, const GemvArgs& a, const int32_t* d_pos) {
  const int nunits = (a.N + R - 1) / R;
  int grid = (nunits + 3) / 4;
  if (grid > 2048) grid = 2048;
  constexpr int US = gemv_u<M, false>(), UL = gemv_u<M, true>();
  if (US != UL && gemv_long(a.K))
    FG_LAUNCH((k_gemv<M, EPI, R, UL>), dim3(grid), dim3(256), 0, s, a, d_pos);
  else
    FG_LAUNCH((k_gemv<M, EPI, R, US>), dim3(grid), dim3(256), 0, s, a, d_pos);
}

template <int EPI>
static void gemv_m(hipStream_t s, const GemvArgs& a, const int32_t* d_pos) {
  constexpr int R = EPI == GV_QKV ? 2 : 1;
  if (a.d_M) {  // a.M = the most rows the launch can be given
    int grid = (a.N / R + 3) / 4;
    if (grid > 2048) grid = 2048;
    if (gemv_long(a.K))
      FG_LAUNCH((k_gemv_live<EPI, true>), dim3(grid, (a.M + 3) / 4), dim3(256), 0, s, a, d_pos);
    else
      FG_LAUNCH((k_gemv_live<EPI, false>), dim3(grid, (a.M + 3) / 4), dim3(256), 0, s, a, d_pos);
  } else if (a.M <= 1) {
    gemv_grid<1, EPI, R>(s, a, d_pos);
  } else if (a.M == 2) {
    gemv_grid<2, EPI, R>(s, a, d_pos);
  } else if (a.M == 3) {
    gemv_grid<3, EPI, R>(s, a, d_pos);
  } else {
    gemv_grid<4, EPI, R>(s, a, d_pos);
  }
}

void launch_gemv_pos(hipStream_t s, GemvEpi epi, const GemvArgs& a, const int32_t* d_pos) {
  switch (epi) {
    case GV_QKV: gemv_m<GV_QKV>(s, a, d_pos); break;
    case GV_RESID: gemv_m<GV_RESID>(s, a, d_pos); break;
    case GV_RELU2: gemv_m<GV_RELU2>(s, a, d_pos); break;
    default: gemv_m<GV_STORE>(s, a, d_pos); break;
  }
}

void launch_gemv(hipStream_t s, GemvEpi epi, const GemvArgs& a) {
  launch_gemv_pos(s, epi, a, nullptr);
}

// ------------------------------------------------------------ decode attention
// Single-query attention over the cache (attn_step,
// src/lib/fortran_attn.f90:317-362): the query at position len-1 against
// cache positions 0..len-1, softmax in the natural domain as the reference
// has it. Work item = (sequence row, KV head, group of GH query heads that
// share it, chunk of DPC positions): each K and V row of the chunk is read
// once for the GH heads of its group (GQA). A lane holds 8 values of the head
// dim, so hd/8 lanes cover one cached row and a wavefront PPW rows per load;
// every K and V row of the chunk is loaded up front (V does not depend on
// the scores), so a chunk costs one memory round trip. A single-chunk call
// writes the result; otherwise each chunk leaves (O, max, sum) per head in
// scratch for k_attn_dec_merge. DPC = 64 positions per chunk; 128 for
// batches of many sequence-heads, where the longer chunks halve the partial
// results (the chunk length sets the merge order, so it depends on the
// sequence count only: every query row of one sequence, and a sequence
// decoded alone, sums alike). The cache holds fp32 (the reference's) or
// bf16 elements (KT).
constexpr int DPC_MIN = 64;
constexpr int DEC_FOLD_MAX_CHUNKS = 8;  // chunks up to which a launch merges its own

struct DecArgs {
  const float* q;  // [rows][H][hd]
  const void* kc;  // [B][maxT][KH*hd], fp32 or bf16
  const void* vc;
  int H, KH, maxT, nchunk;
  int iters;             // DPC-position blocks per workgroup (k_attn_dec_loop), else 1
  const int32_t* d_len;  // cache length before the step (first query at *d_len), or null
  int len_imm;           // cache length including the first query, if d_len is null
  int qpr;               // query rows per sequence: row j sees one position more than j-1
  const int32_t* d_rows; // query rows live (nullable): later rows' blocks exit at once
  float* y;
  uint16_t* ys;
  int64_t ys_plane;
  float* part;  // [rows*H][nchunk][hd + 4]: O, then max and sum (and two unused
                // floats, so every partial row starts 16-byte aligned)
  uint32_t* cnt;  // (nullable) arrival counters, one per head group, zero
                  // between launches: k_attn_dec merges its own chunks
  int fold;       // k_attn_dec_loop: q, k, v from qf's split-K sums (qpr == 1)
  QkvFold qf;
};

// Floats per partial row of the single-query attention: O (HD), max, sum,
// padded to a multiple of 4 so the row's float4 accesses are aligned.
__host__ __device__ constexpr int dec_pstride(int hd) { return hd + 4; }

template <int HD>
__device__ __forceinline__ void dec_store(const DecArgs& a, int64_t o, int d, float4 v) {
  if (a.ys) {  // d % 4 == 0: one 8-byte store per plane
    const float w[4] = {v.x, v.y, v.z, v.w};
    split_bf16x4(w, a.ys + o + d, a.ys_plane);
  } else {
    *(float4*)(a.y + o + d) = v;
  }
}

// 8 consecutive cache elements: raw loads (issued together) and their values.
template <class KT> struct Row8;
template <> struct Row8<float> {
  float4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = *(const float4*)p;
    b = *(const float4*)(p + 4);
  }
  __device__ __forceinline__ void get(float (&x)[8]) const {
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  }
};
template <> struct Row8<uint16_t> {
  uint4 u;
  __device__ __forceinline__ void load(const uint16_t* p) { u = *(const uint4*)p; }
  __device__ __forceinline__ void get(float (&x)[8]) const { unpack8(u, x); }
};

// Sum over the LPP lanes of each cached row (rows of 8 or 16 lanes): quad
// permutes, then the half-row (and row) mirror, which pair the same values
// as strides 4 (and 8) once the smaller groups are uniform.
template <int LPP>
__device__ __forceinline__ float row_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  if constexpr (LPP == 16) v += dpp_f<0x140>(v);
  return v;
}

// A partial's pair of floats, written through to memory (agent scope), and
// read back the same way by the merging workgroup.
__device__ __forceinline__ void part_put(float* p, float x, float y) {
  const uint64_t v = (uint64_t)__float_as_uint(x) | ((uint64_t)__float_as_uint(y) << 32);
  __hip_atomic_store((uint64_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 part_get(const float* p) {
  const uint64_t v = __hip_atomic_load((const uint64_t*)p, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32)));
}

// The merge of nch chunk partials of GH heads, run by the workgroup that
// arrived last. 256 / (HD/8) lane groups, NGH per head: group k of head j
// takes chunks k, k + NGH, ... ascending with a running maximum (old sums
// rescaled when it moves); the NGH groups of a head then meet at their
// common maximum, in group order. sO: NG x HD floats of LDS, gml: the
// groups' maxima and sums.
template <int HD, int GH>
__device__ void dec_fold_merge(const DecArgs& a, int row, int h0, int nch, float* sO,
                               float (*gml)[256 / (HD / 8)]) {
  constexpr int LPC = HD / 8, NG = 256 / LPC, NGH = NG / GH, CPG = 4;
  const int tid = threadIdx.x, g = tid / LPC, dl = tid % LPC;
  const int j = g / NGH, k = g % NGH;
  const bool act = j < GH && k < nch;
  float m = -FLT_MAX, l = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (act) {
    const float* P = a.part + ((int64_t)row * a.H + h0 + j) * a.nchunk * dec_pstride(HD);
    for (int c0 = k; c0 < nch; c0 += NGH * CPG) {
      float2 ml[CPG], ov[CPG][4];
#pragma unroll
      for (int i = 0; i < CPG; ++i) {  // this round's loads go out together
        const int c = min(c0 + i * NGH, nch - 1);
        const float* pc = P + (int64_t)c * dec_pstride(HD);
        ml[i] = part_get(pc + HD);
#pragma unroll
        for (int e = 0; e < 4; ++e) ov[i][e] = part_get(pc + 8 * dl + 2 * e);
      }
#pragma unroll
      for (int i = 0; i < CPG; ++i) {
        if (c0 + i * NGH >= nch) break;
        const float mn = fmaxf(m, ml[i].x);
        const float s0 = expf(m - mn), w = expf(ml[i].x - mn);
        l = l * s0 + w * ml[i].y;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          o[2 * e] = o[2 * e] * s0 + w * ov[i][e].x;
          o[2 * e + 1] = o[2 * e + 1] * s0 + w * ov[i][e].y;
        }
        m = mn;
      }
    }
  }
  *(float4*)&sO[g * HD + 8 * dl] = make_float4(o[0], o[1], o[2], o[3]);
  *(float4*)&sO[g * HD + 8 * dl + 4] = make_float4(o[4], o[5], o[6], o[7]);
  if (dl == 0) {
    gml[0][g] = m;
    gml[1][g] = l;
  }
  __syncthreads();
  for (int q4 = tid; q4 < GH * HD / 4; q4 += 256) {
    const int jj = q4 / (HD / 4), d = 4 * (q4 % (HD / 4)), g0 = jj * NGH;
    const int ngr = min(NGH, nch);
    float mx = gml[0][g0];
    for (int i = 1; i < ngr; ++i) mx = fmaxf(mx, gml[0][g0 + i]);
    float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
    float L = 0.f;
    for (int i = 0; i < ngr; ++i) {
      const float w = expf(gml[0][g0 + i] - mx);
      const float4 u = *(const float4*)&sO[(g0 + i) * HD + d];
      t.x += w * u.x; t.y += w * u.y; t.z += w * u.z; t.w += w * u.w;
      L += w * gml[1][g0 + i];
    }
    const float inv = 1.0f / L;
    dec_store<HD>(a, ((int64_t)row * a.H + h0 + jj) * HD, d,
                  make_float4(t.x * inv, t.y * inv, t.z * inv, t.w * inv));
  }
}

template <int HD, int DPC, int GH, class KT>
__global__ __launch_bounds__(256) void k_attn_dec(DecArgs a) {
  constexpr int LPP = HD / 8;        // lanes per cached row
  constexpr int PPW = 64 / LPP;      // rows per wavefront load
  constexpr int IT = DPC / 4 / PPW;  // loads per lane and tensor
  static_assert(LPP == 8 || LPP == 16, "head dim 64 or 128");
  __shared__ float red[2][4][GH];
  __shared__ float so[4 * PPW][GH][HD];
  __shared__ float gml[2][256 / LPP];
  const int G = a.H / a.KH, ng = G / GH;
  const int gi = blockIdx.x, c = blockIdx.y;
  const int row = gi / (a.KH * ng), kvh = (gi / ng) % a.KH, h0 = kvh * G + (gi % ng) * GH;
  if (a.d_rows && row >= *a.d_rows) return;
  const int len = (a.d_len ? *a.d_len + 1 : a.len_imm) + row % a.qpr;
  const int p0 = c * DPC;
  if (p0 >= len) return;
  const int nch = (len + DPC - 1) / DPC;
  const int b = row / a.qpr;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int sub = lane / LPP, dl = lane % LPP;
  const int64_t kd = (int64_t)a.KH * HD;
  const KT* K = (const KT*)a.kc + (int64_t)b * a.maxT * kd + kvh * HD + 8 * dl;
  const KT* V = (const KT*)a.vc + (int64_t)b * a.maxT * kd + kvh * HD + 8 * dl;
  Row8<KT> kr[IT], vr[IT];
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int p = min(p0 + wv * (DPC / 4) + i * PPW + sub, len - 1);
    kr[i].load(K + p * kd);
    vr[i].load(V + p * kd);
  }
  float qv[GH][8];
#pragma unroll
  for (int j = 0; j < GH; ++j) {
    const float* qp = a.q + ((int64_t)row * a.H + h0 + j) * HD + 8 * dl;
    const float4 u = *(const float4*)qp, w = *(const float4*)(qp + 4);
    qv[j][0] = u.x; qv[j][1] = u.y; qv[j][2] = u.z; qv[j][3] = u.w;
    qv[j][4] = w.x; qv[j][5] = w.y; qv[j][6] = w.z; qv[j][7] = w.w;
  }
  const float scale = 1.0f / sqrtf((float)HD);
  float sc[GH][IT], mx[GH];
#pragma unroll
  for (int j = 0; j < GH; ++j) mx[j] = -FLT_MAX;
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    float x[8];
    kr[i].get(x);
    const int p = p0 + wv * (DPC / 4) + i * PPW + sub;
#pragma unroll
    for (int j = 0; j < GH; ++j) {
      float v = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) v += qv[j][e] * x[e];
      v = row_sum<LPP>(v);
      sc[j][i] = p < len ? v * scale : -INFINITY;
      mx[j] = fmaxf(mx[j], sc[j][i]);
    }
  }
  // maxima over the wavefront's rows, then over the four wavefronts
#pragma unroll
  for (int j = 0; j < GH; ++j) {
    const int iv = __builtin_bit_cast(int, mx[j]);
    float t = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0));
#pragma unroll
    for (int r = 1; r < PPW; ++r)
      t = fmaxf(t, __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, r * LPP)));
    if (lane == 0) red[0][wv][j] = t;
  }
  __syncthreads();
  float m[GH], l[GH], o[GH][8];
#pragma unroll
  for (int j = 0; j < GH; ++j) {
    m[j] = fmaxf(fmaxf(red[0][0][j], red[0][1][j]), fmaxf(red[0][2][j], red[0][3][j]));
    l[j] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[j][e] = 0.f;
  }
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    float x[8];
    vr[i].get(x);
#pragma unroll
    for (int j = 0; j < GH; ++j) {
      const float w = expf(sc[j][i] - m[j]);
      l[j] += w;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[j][e] += w * x[e];
    }
  }
  // per-row partial O to LDS; row sums of the weights (equal in a row's lanes)
#pragma unroll
  for (int j = 0; j < GH; ++j) {
    float4* dst = (float4*)&so[wv * PPW + sub][j][8 * dl];
    dst[0] = make_float4(o[j][0], o[j][1], o[j][2], o[j][3]);
    dst[1] = make_float4(o[j][4], o[j][5], o[j][6], o[j][7]);
    const int iv = __builtin_bit_cast(int, l[j]);
    float t = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0));
#pragma unroll
    for (int r = 1; r < PPW; ++r)
      t += __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, r * LPP));
    if (lane == 0) red[1][wv][j] = t;
  }
  __syncthreads();
  const bool fold = a.cnt && nch > 1;
  // O of each head: the 4*PPW row partials summed in a fixed order
  for (int q4 = tid; q4 < GH * HD / 4; q4 += 256) {
    const int j = q4 / (HD / 4), d = 4 * (q4 % (HD / 4));
    float4 t = *(const float4*)&so[0][j][d];
#pragma unroll
    for (int r = 1; r < 4 * PPW; ++r) {
      const float4 u = *(const float4*)&so[r][j][d];
      t.x += u.x; t.y += u.y; t.z += u.z; t.w += u.w;
    }
    const float lj = (red[1][0][j] + red[1][1][j]) + (red[1][2][j] + red[1][3][j]);
    const int64_t bh = (int64_t)row * a.H + h0 + j;
    if (nch == 1) {
      const float inv = 1.0f / lj;
      dec_store<HD>(a, bh * HD, d, make_float4(t.x * inv, t.y * inv, t.z * inv, t.w * inv));
    } else {
      float* P = a.part + (bh * a.nchunk + c) * dec_pstride(HD);
      const float mj = fmaxf(fmaxf(red[0][0][j], red[0][1][j]), fmaxf(red[0][2][j], red[0][3][j]));
      if (fold) {  // written through to memory: the merging workgroup may sit on another XCD
        part_put(P + d, t.x, t.y);
        part_put(P + d + 2, t.z, t.w);
        if (d == 0) part_put(P + HD, mj, lj);
      } else {
        *(float4*)(P + d) = t;
        if (d == 0) *(float2*)(P + HD) = make_float2(mj, lj);
      }
    }
  }
  if (!fold) return;
  // Arrival: each lane's partial stores are complete before the workgroup
  // is counted; the last of the nch chunk workgroups merges them.
  __shared__ uint32_t last;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0)
    last = __hip_atomic_fetch_add(a.cnt + gi, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           (uint32_t)(nch - 1);
  __syncthreads();
  if (!last) return;
  if (tid == 0)  // every chunk has arrived: ready for the next launch
    __hip_atomic_store(a.cnt + gi, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  dec_fold_merge<HD, GH>(a, row, h0, nch, &so[0][0][0], gml);
}

// The QKV projection's tail for one query row, done by the attention that
// consumes it (a batched cached step whose QKV GEMM split K): the split
// partial sums added in split order, eight at a time, the row's rmsnorm
// scale, RoPE at position pos, as k_splitk_reduce and the QKV epilogue have
// it (stored column pair 2i, 2i+1 of a head holds dims i and i + hd/2).
// Thread t takes item t: pair t of the GH query heads h0.., then, with kv
// set, pair t - GH*HD/2 of the KV head's k and then v (at most (GH+2)*HD/2
// items, no more than the workgroup's threads). fold_load issues every load
// the item needs at once (the first eight splits, four of the row's
// sum-of-squares partials, the RoPE pair), ahead of the kernel's first K
// rows; fold_pin, after those, marks where the values must have arrived;
// fold_finish adds them (and any further splits and partials), and leaves q
// in sq and the new k and v (their cached values: bf16-rounded for a bf16
// cache) in skv, and with put set also in the cache at pos.
struct FoldIn {
  float2 pv[8];
  float ss[4];
  float cs, sn;
};

template <int HD, int GH>
__device__ __forceinline__ int fold_col(const DecArgs& a, int h0, int kvh, bool kv, int& grp,
                                        int& i) {
  constexpr int NP = HD / 2;  // rotation pairs per head
  const int it = threadIdx.x;
  grp = it / NP;  // q heads 0..GH-1, then k, then v
  i = it % NP;
  if (it >= (GH + (kv ? 2 : 0)) * NP) return -1;
  return grp < GH ? (h0 + grp) * HD + 2 * i
                  : a.H * HD + (grp - GH) * a.KH * HD + kvh * HD + 2 * i;
}

// (Every load goes out, from a clamped and valid address; the unused
// values are dropped later: conditional loads would become branches that
// each wait for their load.)
template <int HD, int GH>
__device__ __forceinline__ void fold_load(const DecArgs& a, int row, int h0, int kvh, bool kv,
                                          int pos, FoldIn& in) {
  const QkvFold& f = a.qf;
  int grp, i;
  const int n = fold_col<HD, GH>(a, h0, kvh, kv, grp, i);
  const float* P = f.part + (int64_t)row * f.N + max(n, 0);
  const int64_t stride = (int64_t)f.rows * f.N;
#pragma unroll
  for (int k = 0; k < 8; ++k)
    in.pv[k] = *reinterpret_cast<const float2*>(P + min(k, f.splits - 1) * stride);
#pragma unroll
  for (int t = 0; t < 4; ++t) in.ss[t] = f.ssq_in[(int64_t)row * f.ssq_n + min(t, f.ssq_n - 1)];
  const int64_t at = (int64_t)pos * (HD / 2) + i;
  in.cs = f.cosb[at];
  in.sn = f.sinb[at];
}

__device__ __forceinline__ void fold_pin(FoldIn& in) {
#pragma unroll
  for (int k = 0; k < 8; ++k) asm volatile("" : "+v"(in.pv[k].x), "+v"(in.pv[k].y) : : "memory");
  asm volatile("" : "+v"(in.ss[0]), "+v"(in.ss[1]), "+v"(in.ss[2]), "+v"(in.ss[3]),
               "+v"(in.cs), "+v"(in.sn) : : "memory");
}

template <int HD, int GH, class KT>
__device__ void fold_finish(const DecArgs& a, int row, int h0, int kvh, int pos, bool kv,
                            bool put, const FoldIn& in, float (*sq)[HD], float (*skv)[HD]) {
  const QkvFold& f = a.qf;
  constexpr int NP = HD / 2;
  int grp, i;
  const int n = fold_col<HD, GH>(a, h0, kvh, kv, grp, i);
  if (n < 0) return;
  float v0 = 0.f, v1 = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) {  // split order (a zero adds nothing)
    const float2 x = k < f.splits ? in.pv[k] : make_float2(0.f, 0.f);
    v0 += x.x;
    v1 += x.y;
  }
  const float* P = f.part + (int64_t)row * f.N + n;
  const int64_t stride = (int64_t)f.rows * f.N;
  for (int s0 = 8; s0 < f.splits; s0 += 8) {
    float2 pv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k)
      pv[k] = s0 + k < f.splits ? *reinterpret_cast<const float2*>(P + (s0 + k) * stride)
                                : make_float2(0.f, 0.f);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      v0 += pv[k].x;
      v1 += pv[k].y;
    }
  }
  float ssum = 0.f;
#pragma unroll
  for (int t = 0; t < 4; ++t)
    if (t < f.ssq_n) ssum += in.ss[t];
  for (int t = 4; t < f.ssq_n; ++t) ssum += f.ssq_in[(int64_t)row * f.ssq_n + t];
  const float inv = 1.0f / sqrtf(ssum / (float)f.K + f.eps);
  v0 *= inv;
  v1 *= inv;
  float y1 = v0, y2 = v1;
  if (grp <= GH) {  // q and k: rotated
    const float cs = in.cs, sn = in.sn;
    y1 = v0 * cs + v1 * sn;
    y2 = v0 * (-sn) + v1 * cs;
  }
  if (grp < GH) {
    sq[grp][i] = y1;
    sq[grp][i + NP] = y2;
    return;
  }
  const int t = grp - GH;  // 0: k, 1: v
  // (row = sequence: one query row each; the cache operands are read-only
  // to every other kernel of the launch)
  const int64_t at = (int64_t)(row * a.maxT + pos) * a.KH * HD + kvh * HD;
  if constexpr (sizeof(KT) == 2) {
    const uint16_t h1 = f32_to_bf16_rne(y1), h2 = f32_to_bf16_rne(y2);
    skv[t][i] = bf16_to_f32(h1);
    skv[t][i + NP] = bf16_to_f32(h2);
    if (put) {
      uint16_t* c = (uint16_t*)(t ? a.vc : a.kc) + at;
      c[i] = h1;
      c[i + NP] = h2;
    }
  } else {
    skv[t][i] = y1;
    skv[t][i + NP] = y2;
    if (put) {
      float* c = (float*)(t ? a.vc : a.kc) + at;
      c[i] = y1;
      c[i + NP] = y2;
    }
  }
}

// k_attn_dec over a.iters consecutive blocks of DPC positions per
// workgroup (NWV wavefronts, DPC / NWV positions each per block), for
// batches with rows x KV heads enough to fill the chip without splitting
// the positions finely (at B=64 one workgroup takes a whole sequence and
// head, and no merge follows). Each wavefront keeps an online softmax of
// its own positions across the blocks (running maximum, sum and O, rescaled
// when the maximum moves); the wavefronts' results meet at the end, each
// rescaled to the workgroup maximum, and leave as
// k_attn_dec's do (the output, or a partial for k_attn_dec_merge). While a
// block's scores are formed its V rows load, and the next block's K rows
// load while its V rows are weighed. With FOLD the kernel also finishes the
// step's QKV projection (fold_load / fold_finish): the query comes from the
// split-K partials, and the new position, not cached yet, is added by the
// last chunk from the k and v it computed (and appended to the cache).
template <int HD, int DPC, int GH, class KT, int NWV = 4, bool FOLD = false>
__global__ __launch_bounds__(64 * NWV) void k_attn_dec_loop(DecArgs a) {
  constexpr int LPP = HD / 8;        // lanes per cached row
  constexpr int PPW = 64 / LPP;      // rows per wavefront load
  constexpr int IT = DPC / NWV / PPW;  // loads per lane and tensor per block
  static_assert(LPP == 8 || LPP == 16, "head dim 64 or 128");
  __shared__ float red[3][NWV][GH];
  __shared__ float so[NWV * PPW][GH][HD];
  __shared__ float sq[FOLD ? GH : 1][HD], skv[FOLD ? 2 : 1][HD];  // (FOLD) q; new k, v
  const int G = a.H / a.KH, ng = G / GH;
  const int gi = blockIdx.x, c = blockIdx.y;
  const int row = gi / (a.KH * ng), kvh = (gi / ng) % a.KH, h0 = kvh * G + (gi % ng) * GH;
  if (a.d_rows && row >= *a.d_rows) return;
  const int len = (a.d_len ? *a.d_len + 1 : a.len_imm) + row % a.qpr;
  const int span = DPC * a.iters;
  const int p0 = c * span;
  if (p0 >= len) return;
  const int nch = (len + span - 1) / span;
  // With FOLD the new position len-1 is not in the cache yet: the cached
  // positions stop at lenc, and the last chunk adds the new one from skv.
  const int lenc = FOLD ? len - 1 : len;
  const int plast = max(lenc - 1, 0);  // (loads past lenc repeat a cached row)
  const int nblk = min(a.iters, (lenc - p0 + DPC - 1) / DPC);  // blocks with positions < lenc
  const bool last = c == nch - 1;
  const int b = row / a.qpr;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int sub = lane / LPP, dl = lane % LPP;
  const int64_t kd = (int64_t)a.KH * HD;
  // cached rows: the sequence's head base (workgroup-uniform) plus a 32-bit
  // byte offset, row x row bytes as a 24-bit multiply (rows and row bytes
  // below 2^24, a sequence's cache below 2^31 bytes: the cache's creation
  // checks it)
  const char* Kb = (const char*)((const KT*)a.kc + (int64_t)b * a.maxT * kd + kvh * HD);
  const char* Vb = (const char*)((const KT*)a.vc + (int64_t)b * a.maxT * kd + kvh * HD);
  const uint32_t rowb = (uint32_t)kd * sizeof(KT), laneb = 8 * dl * sizeof(KT);
  auto rowp = [&](const char* base, int p) {
    return (const KT*)(base + (__umul24((uint32_t)min(p, plast), rowb) + laneb));
  };
  auto pos = [&](int blk, int i) { return p0 + blk * DPC + wv * (DPC / NWV) + i * PPW + sub; };
  Row8<KT> kr[IT], vr[IT];
  FoldIn fin;
  if constexpr (FOLD) {
    fold_load<HD, GH>(a, row, h0, kvh, last, len - 1, fin);
    asm volatile("" ::: "memory");  // (those loads go out before the K rows')
  }
#pragma unroll
  for (int i = 0; i < IT; ++i) kr[i].load(rowp(Kb, pos(0, i)));
  float qv[GH][8];
  if constexpr (FOLD) {
    fold_pin(fin);
    fold_finish<HD, GH, KT>(a, row, h0, kvh, len - 1, last, last && gi % ng == 0, fin, sq, skv);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < GH; ++j) {
      const float4 u = *(const float4*)&sq[j][8 * dl], w = *(const float4*)&sq[j][8 * dl + 4];
      qv[j][0] = u.x; qv[j][1] = u.y; qv[j][2] = u.z; qv[j][3] = u.w;
      qv[j][4] = w.x; qv[j][5] = w.y; qv[j][6] = w.z; qv[j][7] = w.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < GH; ++j) {
      const float* qp = a.q + ((int64_t)row * a.H + h0 + j) * HD + 8 * dl;
      const float4 u = *(const float4*)qp, w = *(const float4*)(qp + 4);
      qv[j][0] = u.x; qv[j][1] = u.y; qv[j][2] = u.z; qv[j][3] = u.w;
      qv[j][4] = w.x; qv[j][5] = w.y; qv[j][6] = w.z; qv[j][7] = w.w;
    }
  }
  // scores in log2 units (scale x log2(e)): each weight is one v_exp_f32 of
  // a difference; the maximum handed to the merge is converted back
  const float scale = 1.44269504088896341f / sqrtf((float)HD);
  float m[GH], l[GH], o[GH][8];
#pragma unroll
  for (int j = 0; j < GH; ++j) {
    m[j] = -FLT_MAX;
    l[j] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[j][e] = 0.f;
  }
  for (int blk = 0; blk < nblk; ++blk) {
#pragma unroll
    for (int i = 0; i < IT; ++i) vr[i].load(rowp(Vb, pos(blk, i)));
    float sc[GH][IT], mx[GH];
#pragma unroll
    for (int j = 0; j < GH; ++j) mx[j] = -FLT_MAX;
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      float x[8];
      kr[i].get(x);
      const int p = pos(blk, i);
#pragma unroll
      for (int j = 0; j < GH; ++j) {
        float v = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) v += qv[j][e] * x[e];
        v = row_sum<LPP>(v);
        sc[j][i] = p < lenc ? v * scale : -INFINITY;
        mx[j] = fmaxf(mx[j], sc[j][i]);
      }
    }
    if (blk + 1 < nblk) {
#pragma unroll
      for (int i = 0; i < IT; ++i) kr[i].load(rowp(Kb, pos(blk + 1, i)));
    }
#pragma unroll
    for (int j = 0; j < GH; ++j) {
      const float mn = fmaxf(m[j], wave_max(mx[j]));  // (>= -FLT_MAX: finite)
      const float alpha = __builtin_amdgcn_exp2f(m[j] - mn);
      m[j] = mn;
      l[j] *= alpha;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[j][e] *= alpha;
    }
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      float x[8];
      vr[i].get(x);
#pragma unroll
      for (int j = 0; j < GH; ++j) {
        const float w = __builtin_amdgcn_exp2f(sc[j][i] - m[j]);
        l[j] += w;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[j][e] += w * x[e];
      }
    }
  }
  if (FOLD && last && wv == 0) {  // the new position, one row of wavefront 0
    float kx[8], vx[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      kx[e] = skv[0][8 * dl + e];
      vx[e] = skv[1][8 * dl + e];
    }
#pragma unroll
    for (int j = 0; j < GH; ++j) {
      float v = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) v += qv[j][e] * kx[e];
      const float sc = row_sum<LPP>(v) * scale;
      const float mn = fmaxf(m[j], sc);
      const float alpha = __builtin_amdgcn_exp2f(m[j] - mn);
      m[j] = mn;
      l[j] *= alpha;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[j][e] *= alpha;
      if (sub == 0) {
        const float w = __builtin_amdgcn_exp2f(sc - mn);
        l[j] += w;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[j][e] += w * vx[e];
      }
    }
  }
  // the wavefronts' maxima, then each wavefront's O and row sums rescaled
  // to the workgroup's
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < GH; ++j) red[0][wv][j] = m[j];
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < GH; ++j) {
    float mw = red[0][0][j];
#pragma unroll
    for (int w = 1; w < NWV; ++w) mw = fmaxf(mw, red[0][w][j]);
    const float f = __builtin_amdgcn_exp2f(m[j] - mw);
    float4* dst = (float4*)&so[wv * PPW + sub][j][8 * dl];
    dst[0] = make_float4(o[j][0] * f, o[j][1] * f, o[j][2] * f, o[j][3] * f);
    dst[1] = make_float4(o[j][4] * f, o[j][5] * f, o[j][6] * f, o[j][7] * f);
    const int iv = __builtin_bit_cast(int, l[j]);
    float t = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0));
#pragma unroll
    for (int r = 1; r < PPW; ++r)
      t += __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, r * LPP));
    if (lane == 0) red[1][wv][j] = t * f;
    if (lane == 0) red[2][wv][j] = mw;
  }
  __syncthreads();
  for (int q4 = tid; q4 < GH * HD / 4; q4 += 64 * NWV) {
    const int j = q4 / (HD / 4), d = 4 * (q4 % (HD / 4));
    float4 t = *(const float4*)&so[0][j][d];
#pragma unroll
    for (int r = 1; r < NWV * PPW; ++r) {
      const float4 u = *(const float4*)&so[r][j][d];
      t.x += u.x; t.y += u.y; t.z += u.z; t.w += u.w;
    }
    float lj = red[1][0][j];
#pragma unroll
    for (int w = 1; w < NWV; ++w) lj += red[1][w][j];
    const int64_t bh = (int64_t)row * a.H + h0 + j;
    if (nch == 1) {
      const float inv = 1.0f / lj;
      dec_store<HD>(a, bh * HD, d, make_float4(t.x * inv, t.y * inv, t.z * inv, t.w * inv));
    } else {
      float* P = a.part + (bh * a.nchunk + c) * dec_pstride(HD);
      *(float4*)(P + d) = t;
      if (d == 0) *(float2*)(P + HD) = make_float2(red[2][0][j] * 0.693147180559945309f, lj);
    }
  }
}

// Combine the chunks of a multi-chunk step: the maximum over chunks, then
// 256/(hd/8) chunk groups (group g takes chunks g, g + NG, ..., ascending)
// whose weighted partial sums are added in group order. Every chunk's loads
// are issued before the maximum is known.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_dec_merge(DecArgs a, int dpc) {
  constexpr int LPC = HD / 8, NG = 256 / LPC, CPG = 4;
  __shared__ float wmax[4];
  __shared__ float sO[NG][HD];
  __shared__ float sl[NG];
  const int bh = blockIdx.x, tid = threadIdx.x;
  if (a.d_rows && bh / a.H >= *a.d_rows) return;
  const int len = (a.d_len ? *a.d_len + 1 : a.len_imm) + (bh / a.H) % a.qpr;
  const int nch = (len + dpc - 1) / dpc;
  if (nch == 1) return;
  const float* P = a.part + (int64_t)bh * a.nchunk * dec_pstride(HD);
  const int g = tid / LPC, dl = tid % LPC;
  float mx = -FLT_MAX;
  for (int c = tid; c < nch; c += 256) mx = fmaxf(mx, P[(int64_t)c * dec_pstride(HD) + HD]);
  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, l = 0.f, m = 0.f;
  float2 ml[CPG];
  float4 ov[CPG][2];
  auto load = [&](int c0) {
#pragma unroll
    for (int k = 0; k < CPG; ++k) {
      const int c = c0 + k * NG;
      const float* pc = P + (int64_t)(c < nch ? c : 0) * dec_pstride(HD);
      ml[k] = *(const float2*)(pc + HD);
      ov[k][0] = *(const float4*)(pc + 8 * dl);
      ov[k][1] = *(const float4*)(pc + 8 * dl + 4);
    }
  };
  auto accumulate = [&](int c0) {
#pragma unroll
    for (int k = 0; k < CPG; ++k) {
      if (c0 + k * NG >= nch) break;
      const float w = expf(ml[k].x - m);
      l += w * ml[k].y;
      o[0] += w * ov[k][0].x; o[1] += w * ov[k][0].y; o[2] += w * ov[k][0].z; o[3] += w * ov[k][0].w;
      o[4] += w * ov[k][1].x; o[5] += w * ov[k][1].y; o[6] += w * ov[k][1].z; o[7] += w * ov[k][1].w;
    }
  };
  load(g);  // this group's first chunks, in flight during the maximum's reduction
  mx = wave_max(mx);
  if ((tid & 63) == 0) wmax[tid >> 6] = mx;
  __syncthreads();
  m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  accumulate(g);
  for (int c0 = g + NG * CPG; c0 < nch; c0 += NG * CPG) {
    load(c0);
    accumulate(c0);
  }
  *(float4*)&sO[g][8 * dl] = make_float4(o[0], o[1], o[2], o[3]);
  *(float4*)&sO[g][8 * dl + 4] = make_float4(o[4], o[5], o[6], o[7]);
  if (dl == 0) sl[g] = l;
  __syncthreads();
  if (tid >= HD / 4) return;
  float4 t = *(const float4*)&sO[0][4 * tid];
  float L = sl[0];
  for (int k = 1; k < NG; ++k) {
    const float4 u = *(const float4*)&sO[k][4 * tid];
    t.x += u.x; t.y += u.y; t.z += u.z; t.w += u.w;
    L += sl[k];
  }
  const float inv = 1.0f / L;
  dec_store<HD>(a, (int64_t)bh * HD, 4 * tid, make_float4(t.x * inv, t.y * inv, t.z * inv, t.w * inv));
}

int attn_decode_chunks(int maxT) { return (maxT + DPC_MIN - 1) / DPC_MIN; }

int64_t attn_decode_scratch_floats(const Dims& d, int B, int maxT) {
  return (int64_t)B * d.H * attn_decode_chunks(maxT) * dec_pstride(d.hd);
}

namespace {

// Largest head group that divides the query heads per KV head and keeps the
// kernel's registers in bounds (8 values x GH heads of q and O per lane).
int dec_group(int G, int dpc) {
  static const int opts64[] = {5, 4, 2, 1}, opts128[] = {2, 1};
  const int* opts = dpc == 128 ? opts128 : opts64;
  const int n = dpc == 128 ? 2 : 4;
  for (int i = 0; i < n; ++i)
    if (G % opts[i] == 0) return opts[i];
  return 1;
}

template <int HD, int DPC, class KT>
void launch_dec_gh(hipStream_t s, const DecArgs& a, int rows, int gh) {
  const int ng = a.H / a.KH / gh;
  const dim3 grid((unsigned)(rows * a.KH * ng), (unsigned)a.nchunk);
  if constexpr (sizeof(KT) == 2 && DPC == 128) {
    // a bf16 cache walked in pairs of blocks: 8 wavefronts over blocks of
    // 256 positions, the same span per workgroup (and chunk count) with
    // twice the K/V rows in flight per workgroup (B=64: 384 workgroups,
    // all resident at two per CU; 1.9 % of the step faster than 4 x 128)
    if (a.iters > 1 && a.iters % 2 == 0) {
      DecArgs b2 = a;
      b2.iters = a.iters / 2;
      if (a.fold) {
        if (gh == 2)
          FG_LAUNCH((k_attn_dec_loop<HD, 256, 2, KT, 8, true>), grid, dim3(512), 0, s, b2);
        else
          FG_LAUNCH((k_attn_dec_loop<HD, 256, 1, KT, 8, true>), grid, dim3(512), 0, s, b2);
      } else {
        if (gh == 2)
          FG_LAUNCH((k_attn_dec_loop<HD, 256, 2, KT, 8>), grid, dim3(512), 0, s, b2);
        else
          FG_LAUNCH((k_attn_dec_loop<HD, 256, 1, KT, 8>), grid, dim3(512), 0, s, b2);
      }
      return;
    }
  }
  if (a.iters > 1) {  // (DPC 128 only: dec_group's options for it)
    if constexpr (DPC == 128) {
      if (a.fold) {
        if (gh == 2)
          FG_LAUNCH((k_attn_dec_loop<HD, DPC, 2, KT, 4, true>), grid, dim3(256), 0, s, a);
        else
          FG_LAUNCH((k_attn_dec_loop<HD, DPC, 1, KT, 4, true>), grid, dim3(256), 0, s, a);
        return;
      }
    }
    if (gh == 2)
      FG_LAUNCH((k_attn_dec_loop<HD, DPC, 2, KT>), grid, dim3(256), 0, s, a);
    else
      FG_LAUNCH((k_attn_dec_loop<HD, DPC, 1, KT>), grid, dim3(256), 0, s, a);
    return;
  }
  switch (gh) {
    case 5:
      if constexpr (DPC == 64) { FG_LAUNCH((k_attn_dec<HD, DPC, 5, KT>), grid, dim3(256), 0, s, a); return; }
      break;
    case 4:
      if constexpr (DPC == 64) { FG_LAUNCH((k_attn_dec<HD, DPC, 4, KT>), grid, dim3(256), 0, s, a); return; }
      break;
    case 2: FG_LAUNCH((k_attn_dec<HD, DPC, 2, KT>), grid, dim3(256), 0, s, a); return;
    default: break;
  }
  FG_LAUNCH((k_attn_dec<HD, DPC, 1, KT>), grid, dim3(256), 0, s, a);
}

template <int HD, class KT>
void launch_dec_hd(hipStream_t s, const DecArgs& a, int rows, int dpc, int gh) {
  if (dpc == 128)
    launch_dec_gh<HD, 128, KT>(s, a, rows, gh);
  else
    launch_dec_gh<HD, DPC_MIN, KT>(s, a, rows, gh);
  if (a.nchunk > 1 && !(a.cnt && a.iters == 1))  // k_attn_dec with counters merges itself
    FG_LAUNCH((k_attn_dec_merge<HD>), dim3((unsigned)(rows * a.H)), dim3(256), 0, s, a,
              dpc * a.iters);
}

}  // namespace

namespace {

// Positions per chunk, head group and blocks per workgroup of a launch.
struct DecPlan {
  int dpc, gh, iters, live;
};
DecPlan dec_plan(const Dims& d, int B, int maxT, bool replayed, int len, int qpr, bool kv16) {
  DecPlan p;
  // chunks that can be live: all of maxT for a replayed step, else those of
  // the last query row
  p.dpc = B * d.H >= 192 ? 128 : DPC_MIN;
  p.live = replayed ? maxT : len + qpr - 1;
  const int rows = B * qpr;
  p.gh = dec_group(d.H / d.KH, p.dpc);
  // blocks of dpc positions per workgroup (k_attn_dec_loop: fewer chunks to
  // merge): as many as keep 1.5 workgroups per CU on a bf16 cache (B=64: a
  // sequence and head each, no merge; 1.8 % of the step faster than one
  // block), 6 on an fp32 one (its workgroups hold twice the bytes in flight
  // and half the occupancy; 1.2 %), else one
  const int nblk = (p.live + p.dpc - 1) / p.dpc, wg_rows = rows * d.KH * (d.H / d.KH / p.gh);
  const int64_t want2 = (kv16 ? 3 : 12) * (int64_t)cu_count();  // twice the workgroups wanted
  p.iters = 1;
  if (p.dpc == 128)
    for (int it = nblk; it > 1; --it)
      if ((int64_t)wg_rows * ((nblk + it - 1) / it) * 2 >= want2) {
        p.iters = it;
        break;
      }
  return p;
}

}  // namespace

bool attn_decode_takes_qkv(const Dims& d, int B, int maxT, bool replayed, int len, bool kv16) {
  return dec_plan(d, B, maxT, replayed, len, 1, kv16).iters > 1;  // k_attn_dec_loop
}

void launch_attn_decode_pos(hipStream_t s, const Dims& d, const float* q, const void* kc,
                            const void* vc, bool kv16, int B, int maxT, const int32_t* d_len,
                            int len, float* scratch, uint32_t* cnt, float* y, uint16_t* ys,
                            int64_t ys_plane, int qpr, const int32_t* d_rows,
                            const QkvFold* qf) {
  DecArgs a;
  a.q = q;
  a.kc = kc;
  a.vc = vc;
  a.H = d.H;
  a.KH = d.KH;
  a.maxT = maxT;
  const DecPlan pl = dec_plan(d, B, maxT, d_len != nullptr, len, qpr, kv16);
  const int dpc = pl.dpc, live = pl.live, gh = pl.gh, iters = pl.iters;
  const int rows = B * qpr;
  // a caller passes qf only where attn_decode_takes_qkv holds for the same
  // arguments; the QKV's sums would go unfinished otherwise
  if (qf && (iters <= 1 || qpr != 1 || d_rows)) {
    std::fprintf(stderr, "fgpt: internal error: QKV fold for a launch that cannot take it\n");
    std::abort();
  }
  a.fold = qf ? 1 : 0;
  if (qf) a.qf = *qf;
  a.iters = iters;
  a.nchunk = (live + dpc * iters - 1) / (dpc * iters);
  a.d_len = d_len;
  a.len_imm = len;
  a.qpr = qpr;
  a.d_rows = d_rows;
  a.y = y;
  a.ys = ys;
  a.ys_plane = ys_plane;
  a.part = scratch;
  // The in-launch merge costs the chunk workgroups a write-through, an
  // agent-scope count and the last one's reads, a chain of device-scope
  // round trips that beats a merge launch only for a few chunks (B=1, 2 KV
  // heads x 5, 36 chunks of 64: 6.2 + 3.2 us as two launches, 11.8 us as
  // one; at up to 6 chunks one launch is the faster)
  if (a.nchunk > DEC_FOLD_MAX_CHUNKS) cnt = nullptr;
  a.cnt = cnt;
  if (d.hd == 128) {
    if (kv16) launch_dec_hd<128, uint16_t>(s, a, rows, dpc, gh);
    else launch_dec_hd<128, float>(s, a, rows, dpc, gh);
  } else {
    if (kv16) launch_dec_hd<64, uint16_t>(s, a, rows, dpc, gh);
    else launch_dec_hd<64, float>(s, a, rows, dpc, gh);
  }
}

// ------------------------------------------------------------ argmax / nll
// First index of the maximum, as sample_token's strict > scan returns it.
__device__ __forceinline__ void amax_merge(float& v, int& i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

// One block per row. With a step record (d_len/d_len0 set), the chosen id
// also goes to out2[(len - len0) * rows + row] and, when lgs_out is set, the
// whole logits row is copied to lgs_out at the same slot: a replayed greedy
// graph then needs no per-step pointers.
__global__ __launch_bounds__(256) void k_argmax(const float* __restrict__ logits, int V,
                                                int32_t* __restrict__ out,
                                                int32_t* __restrict__ out2,
                                                const int32_t* __restrict__ d_len,
                                                const int32_t* __restrict__ d_len0,
                                                float* __restrict__ lgs_out) {
  __shared__ float rv[4];
  __shared__ int ri[4];
  const int64_t row = blockIdx.x, rows = gridDim.x;
  const float* l = logits + row * V;
  const int64_t slot = d_len ? (int64_t)(*d_len - *d_len0) * rows + row : 0;
  float* cp = (d_len && lgs_out) ? lgs_out + slot * V : nullptr;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  auto take = [&](float v, int j) {
    if (v > bv) {
      bv = v;
      bi = j;
    }
  };
  if ((V & 3) == 0 && ((reinterpret_cast<uintptr_t>(l) | reinterpret_cast<uintptr_t>(cp)) & 15) == 0) {
    // 16-byte loads, eight in flight per thread before any compare; each
    // thread still sees its indices in increasing order
    const float4* l4 = reinterpret_cast<const float4*>(l);
    float4* c4 = reinterpret_cast<float4*>(cp);
    const int V4 = V >> 2;
    for (int j0 = threadIdx.x; j0 < V4; j0 += 256 * 8) {
      float4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        v[u] = j0 + 256 * u < V4 ? l4[j0 + 256 * u] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int j = j0 + 256 * u;
        if (j < V4) {
          if (c4) c4[j] = v[u];
          take(v[u].x, 4 * j);
          take(v[u].y, 4 * j + 1);
          take(v[u].z, 4 * j + 2);
          take(v[u].w, 4 * j + 3);
        }
      }
    }
  } else {
    for (int j = threadIdx.x; j < V; j += 256) {
      const float v = l[j];
      if (cp) cp[j] = v;
      take(v, j);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = __shfl_xor(bv, o, 64);
    const int i2 = __shfl_xor(bi, o, 64);
    amax_merge(bv, bi, v2, i2);
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) {
    rv[w] = bv;
    ri[w] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < 4; ++k) amax_merge(bv, bi, rv[k], ri[k]);
    if (bi == 0x7fffffff) bi = 0;  // all -inf / NaN: position 1, as the scan starts there
    out[row] = bi;
    if (out2 && d_len) out2[slot] = bi;
  }
}

// Advance the device-side cache length after a replayed step.
__global__ void k_advance(int32_t* d_len) {
  if (threadIdx.x == 0) *d_len = *d_len + 1;
}

void launch_argmax_step(hipStream_t s, const float* logits, int64_t rows, int V, int32_t* out,
                        int32_t* out2, int32_t* d_len, const int32_t* d_len0, float* lgs_out) {
  FG_LAUNCH(k_argmax, dim3((unsigned)rows), dim3(256), 0, s, logits, V, out, out2, d_len,
                     d_len0, lgs_out);
  if (d_len) FG_LAUNCH(k_advance, dim3(1), dim3(64), 0, s, d_len);
}

// The end of a GEMV-path greedy step in one single-block launch: for each of
// the (<= 4) rows, the first-max argmax of its logits (sample_token's
// strict > scan), the id into ids[row] and out2[(len-len0)*rows + row],
// the logits row into lgs_out at that slot (when set), then the next
// step's input x[row] = rmsnorm0(wte[id]); finally len += 1. One block, so
// every read of len precedes the increment.
__global__ __launch_bounds__(1024) void k_greedy_tail(const float* __restrict__ logits, int rows,
                                                      int V, int D, float eps,
                                                      const bf16_t* __restrict__ wte,
                                                      int32_t* __restrict__ ids,
                                                      int32_t* __restrict__ out2,
                                                      int32_t* __restrict__ d_len,
                                                      const int32_t* __restrict__ d_len0,
                                                      float* __restrict__ lgs_out,
                                                      float* __restrict__ x) {
  __shared__ float rv[16];
  __shared__ int ri[16];
  __shared__ float red[16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t slot = (int64_t)(*d_len - *d_len0);
  for (int r = 0; r < rows; ++r) {
    const float* l = logits + (int64_t)r * V;
    float* cp = lgs_out ? lgs_out + (slot * rows + r) * V : nullptr;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    // eight values a thread in flight at once (one round trip for V <= 8192),
    // then scanned in index order
    for (int j0 = tid; j0 < V; j0 += 8 * 1024) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = j0 + 1024 * u < V ? l[j0 + 1024 * u] : -INFINITY;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int j = j0 + 1024 * u;
        if (j < V) {
          if (cp) cp[j] = v[u];
          if (v[u] > bv) {
            bv = v[u];
            bi = j;
          }
        }
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) amax_merge(bv, bi, __shfl_xor(bv, o, 64), __shfl_xor(bi, o, 64));
    if (lane == 0) {
      rv[w] = bv;
      ri[w] = bi;
    }
    __syncthreads();
    bv = rv[0];
    bi = ri[0];
    for (int k = 1; k < 16; ++k) amax_merge(bv, bi, rv[k], ri[k]);
    if (bi == 0x7fffffff) bi = 0;  // all -inf / NaN: position 1, as the scan starts there
    if (tid == 0) {
      ids[r] = bi;
      out2[slot * rows + r] = bi;
    }
    // next input row, its sum of squares in k_embed_norm's order (four
    // waves of 256-strided partials), so an id embeds to the same bits here
    // as in any other pass
    const bf16_t* row = wte + (int64_t)bi * D;
    float ss = 0.f;
    if (tid < 256)
      for (int k = tid; k < D; k += 256) {
        const float v = bf16_to_f32(row[k]);
        ss += v * v;
      }
    ss = wave_sum(ss);
    __syncthreads();  // rv/ri reads above are done before red is reused
    if (lane == 0) red[w] = ss;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) t += red[k];
    const float inv = 1.0f / sqrtf(t / (float)D + eps);
    for (int k = tid; k < D; k += 1024) x[(int64_t)r * D + k] = bf16_to_f32(row[k]) * inv;
    __syncthreads();
  }
  if (tid == 0) *d_len = *d_len + 1;
}

void launch_greedy_tail(hipStream_t s, const Dims& d, const float* logits, int rows,
                        const bf16_t* wte, int32_t* ids, int32_t* out2, int32_t* d_len,
                        const int32_t* d_len0, float* lgs_out, float* x) {
  FG_LAUNCH(k_greedy_tail, dim3(1), dim3(1024), 0, s, logits, rows, d.V, d.D, d.eps, wte,
                     ids, out2, d_len, d_len0, lgs_out, x);
}

// ------------------------------------------------------------ speculative loop
// Start of a round of the draft/verify loop (src/app/chat_text.f90:
// 297-318): when the controller is in spec mode, the prompt-lookup drafter
// (lookup_draft, src/lib/fortran_spec.f90:62-92) searches the ids for the
// most recent earlier window equal to the last mm = min(match, pp-1) ids
// (1-based window ends s from pp-mm down to mm; each thread scans its own
// stride from the top, so its first hit is its largest, and the block keeps
// the largest) and proposes what followed it; then the pass's ids (pending
// id + drafts), its cache length and its live row count. No match, or plain
// mode: a one-row pass (a plain step).
__global__ __launch_bounds__(256) void k_spec_draft(SpecDev* __restrict__ st,
                                                    const int32_t* __restrict__ ids) {
  __shared__ int best;
  const int tid = threadIdx.x;
  const int pp = st->pp, nt = st->n_total;
  if (pp >= nt) {
    if (tid == 0) st->rows = 0;
    return;
  }
  const bool spec = st->mode_spec != 0;
  const int mm = min(st->match, pp - 1);
  if (tid == 0) best = 0;
  __syncthreads();
  if (spec && mm >= 1) {
    int mine = 0;
    for (int s = pp - mm - tid; s >= mm; s -= 256) {
      int j = 0;
      while (j < mm && ids[s - mm + j] == ids[pp - mm + j]) ++j;
      if (j == mm) {
        mine = s;
        break;
      }
    }
    if (mine) atomicMax(&best, mine);
  }
  __syncthreads();
  const int s = best;
  int keff = s > 0 ? min(st->k, pp - s) : 0;
  const bool round_spec = keff > 0;
  if (round_spec && pp + keff > nt) keff = nt - pp;
  if (round_spec && tid < keff) st->inp[1 + tid] = ids[s + tid];
  if (tid == 0) {
    st->inp[0] = ids[pp - 1];
    st->keff = round_spec ? keff : 0;
    st->spec_round = round_spec ? 1 : 0;
    st->len = pp - 1;
    st->rows = round_spec ? keff + 1 : 1;
  }
}

// End of a round (src/app/chat_text.f90:319-420): the first-max argmax of
// each live row of the pass's logits (sample_token's strict > scan), the
// accept rule (accept_prefix, src/lib/fortran_spec.f90:41-52) with the
// clamp at n_total, the commit into ids, and the sliding-window controller:
// every `probe` passes in spec mode, fewer than min_acc accepted drafts per
// pass (compared in single precision) pauses drafting for `probe` rounds.
__global__ __launch_bounds__(1024) void k_spec_commit(SpecDev* __restrict__ st,
                                                      const float* __restrict__ logits, int V,
                                                      int32_t* __restrict__ ids) {
  __shared__ float rv[16];
  __shared__ int ri[16];
  __shared__ int targ[GEMV_MAX_ROWS];
  const int rows = st->rows;
  if (rows == 0) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int r = 0; r < rows; ++r) {
    const float* l = logits + (int64_t)r * V;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int j0 = tid; j0 < V; j0 += 8 * 1024) {  // eight loads in flight, then in index order
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = j0 + 1024 * u < V ? l[j0 + 1024 * u] : -INFINITY;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (v[u] > bv) {  // (padding is -inf: never taken)
          bv = v[u];
          bi = j0 + 1024 * u;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) amax_merge(bv, bi, __shfl_xor(bv, o, 64), __shfl_xor(bi, o, 64));
    if (lane == 0) {
      rv[w] = bv;
      ri[w] = bi;
    }
    __syncthreads();
    if (tid == 0) {
      for (int k = 1; k < 16; ++k) amax_merge(bv, bi, rv[k], ri[k]);
      targ[r] = bi == 0x7fffffff ? 0 : bi;  // all -inf / NaN: position 1
    }
    __syncthreads();
  }
  if (tid != 0) return;
  const int pp = st->pp, nt = st->n_total;
  int na = 0;
  if (st->spec_round) {
    const int keff = st->keff;
    while (na < keff && st->inp[1 + na] == targ[na]) ++na;
    int corr = targ[na];
    if (pp + na + 1 > nt) {
      na = nt - pp - 1;
      corr = targ[na];
    }
    for (int j = 0; j < na; ++j) ids[pp + j] = st->inp[1 + j];
    ids[pp + na] = corr;
    st->passes += 1;
    st->accepted += na;
    st->proposed += keff;
  } else {
    ids[pp] = targ[0];
    st->plain += 1;
  }
  st->pp = pp + na + 1;
  if (st->mode_spec) {
    if (st->spec_round) {
      st->npass_w += 1;
      st->nacc_w += na;
    }
    if (st->npass_w >= st->probe) {
      if ((float)st->nacc_w < st->min_acc * (float)st->npass_w) {
        st->mode_spec = 0;
        st->plain_left = st->probe;
        st->pauses += 1;
      }
      st->npass_w = 0;
      st->nacc_w = 0;
    }
  } else {
    st->plain_left -= 1;
    if (st->plain_left <= 0) {
      st->mode_spec = 1;
      st->npass_w = 0;
      st->nacc_w = 0;
    }
  }
}

void launch_spec_draft(hipStream_t s, SpecDev* st, const int32_t* ids) {
  FG_LAUNCH(k_spec_draft, dim3(1), dim3(256), 0, s, st, ids);
}

void launch_spec_commit(hipStream_t s, SpecDev* st, const float* logits, int V, int32_t* ids) {
  FG_LAUNCH(k_spec_commit, dim3(1), dim3(1024), 0, s, st, logits, V, ids);
}

void launch_argmax(hipStream_t s, const float* logits, int64_t rows, int V, int32_t* out) {
  launch_argmax_step(s, logits, rows, V, out, nullptr, nullptr, nullptr, nullptr);
}

// One block per row. Rows of up to 256*4*NV4 logits are read once, as
// float4s held in registers (all loads in flight together); longer rows take
// the two-pass loop.
template <int NV4>
__global__ __launch_bounds__(256) void k_nll(const float* __restrict__ logits,
                                             const int32_t* __restrict__ tgt, int V,
                                             float* __restrict__ out) {
  __shared__ float red[8];
  const int64_t row = blockIdx.x;
  const float* l = logits + row * V;
  float m = -FLT_MAX, s = 0.f;
  if (NV4 > 0) {
    float4 v[NV4 > 0 ? NV4 : 1];
#pragma unroll
    for (int i = 0; i < NV4; ++i) {
      const int j = 4 * (threadIdx.x + 256 * i);
      v[i] = j < V ? *(const float4*)(l + j) : make_float4(-FLT_MAX, -FLT_MAX, -FLT_MAX, -FLT_MAX);
      m = fmaxf(m, fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w)));
    }
    m = block_max<4>(m, red);
#pragma unroll
    for (int i = 0; i < NV4; ++i)
      s += expf(v[i].x - m) + expf(v[i].y - m) + expf(v[i].z - m) + expf(v[i].w - m);
  } else {
    for (int j = threadIdx.x; j < V; j += 256) m = fmaxf(m, l[j]);
    m = block_max<4>(m, red);
    for (int j = threadIdx.x; j < V; j += 256) s += expf(l[j] - m);
  }
  s = block_sum<4>(s, red + 4);
  const int t = tgt[row];
  if (threadIdx.x == 0) out[row] = (t >= 0 && t < V) ? (m + logf(s)) - l[t] : __builtin_nanf("");
}

// The per-row nll of src/app/eval_bpb.f90:165-181 from lm_head's
// log-sum-exp partials (one (max, sum of exp(logit - max)) per
// NLL_GROUP_COLS-column group, written by the GEMM's epilogue): one wavefront per row, the row
// maximum and the rescaled sums reduced in a fixed order.
__global__ __launch_bounds__(256) void k_nll_parts(const float* __restrict__ logits,
                                                   const float* __restrict__ parts,
                                                   const int32_t* __restrict__ tgt, int64_t rows,
                                                   int V, float* __restrict__ out) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // (whole wavefronts)
  const int lane = threadIdx.x & 63, ng = V / NLL_GROUP_COLS;
  const float2* P = reinterpret_cast<const float2*>(parts) + row * ng;
  float m = -FLT_MAX;
  for (int g = lane; g < ng; g += 64) m = fmaxf(m, P[g].x);
  m = wave_max(m);
  float sum = 0.f;
  for (int g = lane; g < ng; g += 64) sum += P[g].y * expf(P[g].x - m);
  sum = wave_sum(sum);
  if (lane == 0) {
    const int t = tgt[row];
    out[row] = (t >= 0 && t < V) ? (m + logf(sum)) - logits[row * V + t] : __builtin_nanf("");
  }
}

void launch_nll_parts(hipStream_t s, const float* logits, const float* parts, const int32_t* tgt,
                      int64_t rows, int V, float* out) {
  if (rows <= 0) return;
  FG_LAUNCH(k_nll_parts, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, logits, parts, tgt,
            rows, V, out);
}

// Byte-weighted sums of one eval row (scripts/eval_driver.py:174-190,
// src/app/bpb_agg.f90:130-152): nats = sum of nll[t] over positions whose
// target has a nonzero byte length, bytes = sum of those lengths. One block
// per row; double accumulation in a fixed order (strided partial sums, then
// a tree), so repeated runs give identical sums. Targets were range-checked
// against the table on the host.
__global__ __launch_bounds__(256) void k_bpb_rows(const float* __restrict__ nll,
                                                  const int32_t* __restrict__ tgt, int T,
                                                  const int32_t* __restrict__ tbytes,
                                                  double* __restrict__ row_nats,
                                                  long long* __restrict__ row_bytes) {
  __shared__ double sn[256];
  __shared__ long long sb[256];
  const int r = blockIdx.x, tid = threadIdx.x;
  double n = 0.0;
  long long b = 0;
  for (int t = tid; t < T; t += 256) {
    const int64_t i = (int64_t)r * T + t;
    const int tb = tbytes[tgt[i]];
    if (tb > 0) {
      n += (double)nll[i];
      b += tb;
    }
  }
  sn[tid] = n;
  sb[tid] = b;
  __syncthreads();
  for (int off = 128; off > 0; off >>= 1) {
    if (tid < off) {
      sn[tid] += sn[tid + off];
      sb[tid] += sb[tid + off];
    }
    __syncthreads();
  }
  if (tid == 0) {
    row_nats[r] = sn[0];
    row_bytes[r] = sb[0];
  }
}

void launch_bpb_rows(hipStream_t s, const float* nll, const int32_t* tgt, int rows, int T,
                     const int32_t* tbytes, double* row_nats, long long* row_bytes) {
  if (rows <= 0) return;
  FG_LAUNCH(k_bpb_rows, dim3((unsigned)rows), dim3(256), 0, s, nll, tgt, T, tbytes,
                     row_nats, row_bytes);
}

void launch_nll(hipStream_t s, const float* logits, const int32_t* tgt, int64_t rows, int V,
                float* out) {
  if (rows <= 0) return;
  // V % 64 == 0, so a row is whole float4s
  if (V <= 256 * 4 * 8)
    FG_LAUNCH(k_nll<8>, dim3((unsigned)rows), dim3(256), 0, s, logits, tgt, V, out);
  else if (V <= 256 * 4 * 16)
    FG_LAUNCH(k_nll<16>, dim3((unsigned)rows), dim3(256), 0, s, logits, tgt, V, out);
  else
    FG_LAUNCH(k_nll<0>, dim3((unsigned)rows), dim3(256), 0, s, logits, tgt, V, out);
}

}  // namespace fgpt
