// kern_attn.hip -- causal chunk attention on MFMA (gfx950).
//
// Computes, for T queries at positions pos0..pos0+T-1 of each of B
// sequences, softmax(q k^T / sqrt(hd)) v over the keys 0..pos0+t with GQA
// head mapping h -> h / (H/KH): causal_attn (src/lib/fortran_attn.f90:30-117)
// when pos0 = 0 and attn_chunk (:376-425) in general.
//
// Formulation: each 64-wide wavefront owns 32 queries and forms S^T = K Q^T
// with v_mfma_f32_32x32x16_bf16 (keys as MFMA rows, queries as columns), so
// the probabilities come out in the register layout the B operand of
// O^T = V^T P^T needs: no LDS round trip for P. The key rows of each 32-key
// tile are permuted (bits 2 and 3 of the row index swapped) so that the 8
// probabilities a lane holds per 16-key step belong to 8 consecutive keys,
// and the matching V^T operand is one 16-byte LDS read. Online softmax
// (running max and sum per query, log2 domain) replaces the reference's two
// passes; the result differs from it only by rounding.
//
// Work split: a workgroup (8 wavefronts: 4 query groups x 2 key parities)
// takes 128 queries against one chunk of at most ck keys, so a T=2048
// prefill gives ~40 items per head instead of 16 uneven query blocks at
// ck = 512. ck is chosen per launch (attn_chunk_keys): the longest chunk
// that still leaves two items per CU, since splitting costs the merge
// (B=1 T=2048: 512; eight such rows: no split). K and
// V^T tiles (64 keys per step) stream memory -> LDS by global_load_lds into
// two XOR-swizzled buffers, the next step loading while the current one is
// consumed. When a query block spans several chunks, each item leaves its
// unnormalised (O, max, sum) in scratch and a second kernel merges them in
// chunk order (a device-scope fence per workgroup, needed to merge in the
// same kernel, costs more than the extra launch).
//
// Precision: q, k, v and p are fp32 quantities carried as bf16 hi + lo
// pairs; each product uses hi*hi + lo*hi + hi*lo (the lo*lo term is below
// fp32 rounding), so scores and outputs keep ~16 mantissa bits rather than
// bf16's 8. A single bf16 term is not enough to keep greedy decodes that
// follow a long prefill identical to the fp32 reference.
#include <float.h>

#include "fgpt_internal.h"
#include "kern_common.h"
#include "kern_epi.h"

namespace fgpt {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

namespace {

constexpr int QB = 128;  // queries per workgroup (4 groups of 32 MFMA columns)
constexpr int CK_MIN = 512;  // shortest key chunk of a work item (sizes the scratch)
constexpr int SK = 64;   // keys per pipeline step (two 32-key tiles)
constexpr float LOG2E = 1.4426950408889634f;

struct AttnArgs {
  const uint16_t* qs;
  const uint16_t* ks;
  const uint16_t* vt;
  int H, KH, T, npos, nvalid, pos0;
  int nbh;  // B * H
  int nqb;  // query blocks per (sequence, head)
  int iph;  // work items per (sequence, head)
  int ck;   // keys per chunk (a multiple of CK_MIN)
  int64_t q_plane, kv_plane;
  float* y;
  uint16_t* ys;
  int64_t ys_plane;
  float* part;
  // (nullable) per work item (blockIdx.x): how many of its causal scores
  // q.k are > 0 -- attn_sgemm's positive-score statistic
  // (src/lib/fortran_attn.f90:247-300), counted before the softmax
  uint32_t* pos_cnt;
};

// key chunks of query block j (queries j*QB .. j*QB+QB-1)
__host__ __device__ inline int chunk_count(int j, int T, int pos0, int nvalid, int ck) {
  const int tl = (j + 1) * QB < T ? (j + 1) * QB : T;
  const int kend = nvalid < pos0 + tl ? nvalid : pos0 + tl;
  return (kend + ck - 1) / ck;
}

// key offset held by row i of a 32-key tile: bits 2 and 3 swapped
__device__ __forceinline__ int tile_key(int i) { return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1); }

// 16-byte chunk slot of logical chunk c in LDS row r: K rows (HD*2 bytes)
// and V^T rows (64 keys = 128 bytes), swizzled so that 16 consecutive rows
// read at one logical chunk hit distinct banks
template <int HD>
__device__ __forceinline__ int kslot(int r, int c) {
  return HD == 128 ? c ^ (r & 15) : c ^ ((r >> 1) & 7);
}
__device__ __forceinline__ int vslot(int d, int c) { return c ^ ((d >> 1) & 7); }

__device__ __forceinline__ void split8(const float* v, bf16x8_t& h, bf16x8_t& l) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const __bf16 hb = (__bf16)v[e];
    h[e] = hb;
    l[e] = (__bf16)(v[e] - (float)hb);
  }
}

// four consecutive output dims (d % 4 == 0): fp32, or the bf16 hi/lo planes
// the next GEMM reads, one 8-byte store per plane
template <int HD, bool P16>
__device__ __forceinline__ void store_out(const AttnArgs& p, int64_t yo, int d, const float (&v)[4]) {
  if (p.ys) {
    put4<P16>(v, p.ys + yo + d, p.ys_plane);
  } else {
    *(float4*)(p.y + yo + d) = make_float4(v[0], v[1], v[2], v[3]);
  }
}

template <int HD, bool P16>
__global__ __launch_bounds__(512) void k_attn_mfma(AttnArgs p) {
  constexpr int NS = HD / 16;          // k-steps over the head dim
  constexpr int ND = HD / 32;          // 32-row blocks of O^T
  constexpr int RBK = HD * 2;          // bytes per K row in LDS
  constexpr int REG = SK * RBK;        // bytes per region (K hi, K lo, V^T hi, V^T lo; P16: K, V^T)
  constexpr int NKR = P16 ? 1 : 2;     // K regions (then as many V^T regions)
  constexpr int STAGE = 2 * NKR * REG;
  constexpr int GPR = REG / 1024;      // 1 KB DMA groups per region
  constexpr int GPW = 2 * NKR * GPR / 8;  // groups per wavefront per stage
  constexpr int PSTR = QB * (HD + 2);  // floats per scratch item: O, then (max, sum)
  static_assert(GPR >= 8 && GPR % 8 == 0, "region / wavefront mismatch");
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int qg = wv & 3, kp = wv >> 2, g = lane >> 5, qi = lane & 31;

  // work item: (sequence*head, query block j, key chunk c); items of one
  // index across heads are adjacent, heaviest query blocks first
  const int bh = blockIdx.x % p.nbh;
  int it = blockIdx.x / p.nbh, j = p.nqb - 1, base = 0, nch;
  for (;;) {
    nch = chunk_count(j, p.T, p.pos0, p.nvalid, p.ck);
    if (it < nch) break;
    it -= nch;
    base += nch;
    --j;
  }
  const int c = it;
  const int b = bh / p.H, h = bh % p.H, kvh = h / (p.H / p.KH);
  const int64_t bk = (int64_t)b * p.KH + kvh;
  const int tq0 = j * QB;
  const int kend = min(p.nvalid, p.pos0 + min(tq0 + QB, p.T));
  const int kbeg = c * p.ck, kstop = min(kend, kbeg + p.ck);
  const int nsteps = (kstop - kbeg + SK - 1) / SK;

  const int t = tq0 + qg * 32 + qi;  // this lane's query (column)
  const bool tok = t < p.T;
  const int qpos = p.pos0 + t;
  const int klim = min(qpos + 1, p.nvalid);  // keys below this are visible
  const bool wact = tq0 + qg * 32 < p.T;  // the wavefront has queries
  const int wq0 = p.pos0 + tq0 + qg * 32;
  const int wq1 = p.pos0 + min(tq0 + qg * 32 + 32, p.T) - 1;

  bf16x8_t qh[NS], ql[NS];  // (P16: qh holds fp16 bits, ql is unused)
  {
    const uint16_t* qp = p.qs + ((int64_t)bh * p.T + (tok ? t : 0)) * HD + 8 * g;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      uint4 vh = *(const uint4*)(qp + 16 * s);
      uint4 vl = P16 ? make_uint4(0, 0, 0, 0) : *(const uint4*)(qp + 16 * s + p.q_plane);
      if (!tok) vh = vl = make_uint4(0, 0, 0, 0);
      qh[s] = __builtin_bit_cast(bf16x8_t, vh);
      ql[s] = __builtin_bit_cast(bf16x8_t, vl);
    }
  }

  // DMA sources of this lane, one per 1 KB group the wavefront fills:
  // group G = wv + 8q lies in region G / GPR = 8q / GPR (compile time)
  const uint16_t* src[GPW];
  int koff[GPW];
#pragma unroll
  for (int q = 0; q < GPW; ++q) {
    const int region = 8 * q / GPR, gi = (wv + 8 * q) % GPR;
    if (region < NKR) {  // K rows: 1024 / RBK rows per group
      const int row = gi * (1024 / RBK) + lane / (HD / 8), slot = lane % (HD / 8);
      koff[q] = 32 * (row >> 5) + tile_key(row & 31);
      src[q] = p.ks + (region ? p.kv_plane : 0) + bk * p.npos * HD + kslot<HD>(row, slot) * 8;
    } else {  // V^T rows (dims): 8 rows of 64 keys per group
      const int d = gi * 8 + lane / 8, slot = lane & 7;
      koff[q] = 0;
      src[q] = p.vt + (region == 3 ? p.kv_plane : 0) + (bk * HD + d) * p.npos + vslot(d, slot) * 8;
    }
  }
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_off(lds) + wv * 1024);
  auto fill = [&](int stg, int k0) {
#pragma unroll
    for (int q = 0; q < GPW; ++q) {
      const int region = 8 * q / GPR;
      const uint16_t* g0 =
          region < NKR ? src[q] + (int64_t)min(k0 + koff[q], p.nvalid - 1) * HD : src[q] + k0;
      dma16(g0, lds0 + stg * STAGE + 8 * q * 1024);
    }
  };

  f32x16_t o[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[i][r] = 0.f;
  float m_run = -FLT_MAX, l_run = 0.f;  // in the log2 domain
  uint32_t npos = 0;  // this lane's positive causal scores (p.pos_cnt)
  __shared__ float wpos[8];
  const float cs = LOG2E / sqrtf((float)HD);

  fill(0, kbeg);
  for (int st = 0; st < nsteps; ++st) {
    // this step's buffer has landed and every wavefront is done with the other
    stage_sync<0>();
    if (st + 1 < nsteps) fill((st + 1) & 1, kbeg + (st + 1) * SK);
    const int kt0 = kbeg + st * SK + 32 * kp;  // this wavefront's tile
    if (!wact || kt0 > wq1 || kt0 >= kstop) continue;
    const uint8_t* S = lds + (st & 1) * STAGE;

    // S^T (32 keys x 32 queries) = K Q^T with hi*hi + lo*hi + hi*lo
    f32x16_t sc;
#pragma unroll
    for (int r = 0; r < 16; ++r) sc[r] = 0.f;
    {
      const int row = 32 * kp + qi;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int off = row * RBK + kslot<HD>(row, 2 * s + g) * 16;
        const bf16x8_t ah = *(const bf16x8_t*)(S + off);
        if constexpr (P16) {
          sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, ah),
                                                     __builtin_bit_cast(f16x8_t, qh[s]), sc, 0, 0, 0);
        } else {
          const bf16x8_t al = *(const bf16x8_t*)(S + REG + off);
          sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, qh[s], sc, 0, 0, 0);
          sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, qh[s], sc, 0, 0, 0);
          sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, ql[s], sc, 0, 0, 0);
        }
      }
    }
    // accumulator r of this lane is key kt0 + 16(r/8) + 8g + (r%8); mask
    // (select, no branch) only tiles that reach the diagonal or the end of
    // the valid keys
    if ((kt0 + 31 > wq0) || (kt0 + 32 > p.nvalid)) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        sc[r] = kt0 + 16 * (r >> 3) + 8 * g + (r & 7) < klim ? sc[r] : -INFINITY;
    }
    if (p.pos_cnt) {  // (masked scores are -inf; a query past T has q = 0, so s = 0)
#pragma unroll
      for (int r = 0; r < 16; ++r) npos += sc[r] > 0.f ? 1u : 0u;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * cs;  // log2 domain (cs > 0)
    // lazy rescale: the running max moves only when a score passes it by
    // 2^8, so most tiles skip rescaling O; probabilities stay below 2^8
    if (__any(mx > m_run + 8.f)) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int i = 0; i < ND; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[i][r] *= alpha;
      m_run = m_new;
    }
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float pr = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], cs, -m_run));
      sc[r] = pr;
      ps += pr;
    }
    l_run += ps + __shfl_xor(ps, 32, 64);

    // O^T += V^T P^T over two 16-key steps: this lane's 8 probabilities are
    // keys 16s + 8g .. +7, one 16-byte chunk of each V^T row
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[e] = sc[8 * s + e];
      if constexpr (P16) {
        f16x8_t p8;
#pragma unroll
        for (int e = 0; e < 8; ++e) p8[e] = (_Float16)pv[e];
#pragma unroll
        for (int i = 0; i < ND; ++i) {
          const int d = 32 * i + qi;
          const int off = NKR * REG + d * 128 + vslot(d, 4 * kp + 2 * s + g) * 16;
          const f16x8_t av = *(const f16x8_t*)(S + off);
          o[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, p8, o[i], 0, 0, 0);
        }
      } else {
        bf16x8_t bh8, bl8;
        split8(pv, bh8, bl8);
#pragma unroll
        for (int i = 0; i < ND; ++i) {
          const int d = 32 * i + qi;
          const int off = NKR * REG + d * 128 + vslot(d, 4 * kp + 2 * s + g) * 16;
          const bf16x8_t avh = *(const bf16x8_t*)(S + off);
          const bf16x8_t avl = *(const bf16x8_t*)(S + REG + off);
          o[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(avh, bh8, o[i], 0, 0, 0);
          o[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(avl, bh8, o[i], 0, 0, 0);
          o[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(avh, bl8, o[i], 0, 0, 0);
        }
      }
    }
  }

  if (p.pos_cnt) {  // (a wavefront's count is below 2^24: its float sum is exact)
    const float wc = wave_sum((float)npos);
    if (lane == 0) wpos[wv] = wc;
  }
  // merge the two key parities of each query group through LDS (no DMA is
  // in flight: the last step issued none and waited for its own)
  __syncthreads();
  if (p.pos_cnt && tid == 0) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < 8; ++w) t += wpos[w];
    p.pos_cnt[blockIdx.x] = (uint32_t)t;
  }
  float* xo = reinterpret_cast<float*>(lds) + qg * (ND * 16 * 64 + 128);
  if (kp == 1) {
#pragma unroll
    for (int i = 0; i < ND; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) xo[(i * 16 + r) * 64 + lane] = o[i][r];
    xo[ND * 16 * 64 + lane] = m_run;
    xo[ND * 16 * 64 + 64 + lane] = l_run;
  }
  __syncthreads();
  const int64_t yrow = (int64_t)p.H * HD;
  if (kp == 0 && wact) {
    const float m1 = xo[ND * 16 * 64 + lane], l1 = xo[ND * 16 * 64 + 64 + lane];
    const float m = fmaxf(m_run, m1);
    const float a0 = exp2f(m_run - m), a1 = exp2f(m1 - m);
    const float l = l_run * a0 + l1 * a1;
    if (nch == 1) {
      if (tok) {
        const float inv = 1.0f / l;
        const int64_t yo = ((int64_t)b * p.T + t) * yrow + h * HD;
#pragma unroll
        for (int i = 0; i < ND; ++i)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
              v[e] = (o[i][4 * r4 + e] * a0 + xo[(i * 16 + 4 * r4 + e) * 64 + lane] * a1) * inv;
            store_out<HD, P16>(p, yo, 32 * i + 8 * r4 + 4 * g, v);
          }
      }
    } else {
      float* P = p.part + ((int64_t)bh * p.iph + base + c) * PSTR;
      const int q = qg * 32 + qi;
#pragma unroll
      for (int i = 0; i < ND; ++i)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            v[e] = o[i][4 * r4 + e] * a0 + xo[(i * 16 + 4 * r4 + e) * 64 + lane] * a1;
          *(float4*)(P + q * HD + 32 * i + 8 * r4 + 4 * g) = make_float4(v[0], v[1], v[2], v[3]);
        }
      if (g == 0) *(float2*)(P + QB * HD + 2 * q) = make_float2(m, l);
    }
  }
}

// Query blocks that span several key chunks: combine the chunks' partial
// (O, max, sum) in chunk order. One workgroup per (sequence*head, block,
// group of 1024/HD queries); a thread owns 4 dims of one query. Up to 8 chunks
// (keys < 4096 at 512 a chunk) take one round trip: every chunk's (max,
// sum) and O are loaded at once, the maximum is taken over the loaded
// values, then the weighted sums; longer blocks take the maximum in a pass
// of its own first. The arithmetic is the same either way.
template <int HD>
constexpr int merge_queries() { return 1024 / HD; }  // per workgroup: 256 threads x 4 dims

template <int HD, bool P16>
__global__ __launch_bounds__(256) void k_attn_merge(AttnArgs p) {
  constexpr int PSTR = QB * (HD + 2), D4 = HD / 4, MQ = merge_queries<HD>();
  static_assert(MQ * D4 == 256 && QB % MQ == 0, "one item per thread");
  const int bh = blockIdx.x % p.nbh, rest = blockIdx.x / p.nbh;
  const int j = p.nqb - 1 - rest / (QB / MQ), part = rest % (QB / MQ);  // heaviest blocks first
  const int nch = chunk_count(j, p.T, p.pos0, p.nvalid, p.ck);
  if (nch == 1) return;  // written by the attention kernel itself
  const int q = part * MQ + threadIdx.x / D4, d = 4 * (threadIdx.x % D4), tt = j * QB + q;
  if (tt >= p.T) return;
  int base = 0;
  for (int i = p.nqb - 1; i > j; --i) base += chunk_count(i, p.T, p.pos0, p.nvalid, p.ck);
  const int b = bh / p.H, h = bh % p.H;
  const int64_t yrow = (int64_t)p.H * HD;
  const float* P0 = p.part + ((int64_t)bh * p.iph + base) * PSTR;
  float m = -FLT_MAX;
  if (nch > 8) {
    for (int k0 = 0; k0 < nch; k0 += 8) {
      float mk[8];
#pragma unroll
      for (int k = 0; k < 8; ++k)
        mk[k] = k0 + k < nch ? P0[(k0 + k) * PSTR + QB * HD + 2 * q] : -FLT_MAX;
#pragma unroll
      for (int k = 0; k < 8; ++k) m = fmaxf(m, mk[k]);
    }
  }
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  float l = 0.f;
  for (int k0 = 0; k0 < nch; k0 += 8) {
    float2 ml[8];
    float4 ov[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const bool ok = k0 + k < nch;
      ml[k] = ok ? *(const float2*)(P0 + (k0 + k) * PSTR + QB * HD + 2 * q) : make_float2(-FLT_MAX, 0.f);
      ov[k] = ok ? *(const float4*)(P0 + (k0 + k) * PSTR + q * HD + d) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (nch <= 8) {
#pragma unroll
      for (int k = 0; k < 8; ++k) m = fmaxf(m, ml[k].x);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (k0 + k >= nch) break;
      const float w = exp2f(ml[k].x - m);
      l += w * ml[k].y;
      acc.x += w * ov[k].x;
      acc.y += w * ov[k].y;
      acc.z += w * ov[k].z;
      acc.w += w * ov[k].w;
    }
  }
  const float inv = 1.0f / l;
  const float v[4] = {acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv};
  store_out<HD, P16>(p, ((int64_t)b * p.T + tt) * yrow + h * HD, d, v);
}

// Cache positions [0, n) of one layer, [B][maxT][KH*hd] -> hi/lo planes
// (a bf16 cache: hi = the element, lo = 0).
__device__ __forceinline__ float cache_elem(const float* c, int64_t i) { return c[i]; }
__device__ __forceinline__ float cache_elem(const uint16_t* c, int64_t i) { return bf16_to_f32(c[i]); }

template <class KT>
__global__ __launch_bounds__(256) void k_split_cache(const KT* __restrict__ kc,
                                                     const KT* __restrict__ vc, int KH, int hd,
                                                     int maxT, int n, int npos, int64_t kv_plane,
                                                     uint16_t* __restrict__ ks,
                                                     uint16_t* __restrict__ vt) {
  const int p = blockIdx.x, b = blockIdx.y, kd = KH * hd;
  if (p >= n) return;
  for (int i = threadIdx.x; i < kd; i += 256) {
    const int kvh = i / hd, d = i % hd;
    const int64_t src = ((int64_t)b * maxT + p) * kd + i;
    const int64_t bk = (int64_t)b * KH + kvh;
    const float kv = cache_elem(kc, src), vv = cache_elem(vc, src);
    uint16_t h = f32_to_bf16_rne(kv);
    const int64_t ko = (bk * npos + p) * hd + d;
    ks[ko] = h;
    ks[ko + kv_plane] = f32_to_bf16_rne(kv - bf16_to_f32(h));
    h = f32_to_bf16_rne(vv);
    const int64_t vo = (bk * hd + d) * npos + p;
    vt[vo] = h;
    vt[vo + kv_plane] = f32_to_bf16_rne(vv - bf16_to_f32(h));
  }
}

}  // namespace

int attn_items_per_head(int T, int pos0, int ck) {
  const int nqb = (T + QB - 1) / QB, nvalid = pos0 + T;
  int n = 0;
  for (int j = 0; j < nqb; ++j) n += chunk_count(j, T, pos0, nvalid, ck);
  return n;
}

// Keys per chunk: the longest of 512, 1024, 2048, ... (the last one covering
// every key, no split) whose items still number at least two per CU, else
// 512. A split query block costs its partials' round trip through memory and
// the merge; fewer, longer items cost nothing while every CU still has two.
int attn_chunk_keys(int BH, int T, int pos0) {
  const int64_t want = 2 * (int64_t)cu_count();
  int best = CK_MIN;
  for (int ck = CK_MIN;; ck *= 2) {
    if ((int64_t)BH * attn_items_per_head(T, pos0, ck) >= want) best = ck;
    if (ck >= pos0 + T) break;
  }
  return best;
}

int64_t attn_items(const Dims& d, int B, int T, int pos0) {
  const int nbh = B * d.H;
  return (int64_t)nbh * attn_items_per_head(T, pos0, attn_chunk_keys(nbh, T, pos0));
}

int64_t attn_scratch_floats(const Dims& d, int B, int T, int pos0) {
  // sized for the shortest chunks (the most items)
  return (int64_t)B * d.H * attn_items_per_head(T, pos0, CK_MIN) * QB * (d.hd + 2);
}

// LDS of a chunk attention launch: two stages, or the key-parity merge
// buffer after the loop (4 query groups x (O^T + max and sum)) if larger
template <int HD, bool P16>
constexpr int attn_lds() {
  constexpr int stages = 2 * 2 * (P16 ? 1 : 2) * SK * HD * 2;
  constexpr int merge = 4 * (HD / 32 * 16 * 64 + 128) * 4;
  return stages > merge ? stages : merge;
}

template <int HD, bool P16>
void launch_attn_hd(hipStream_t s, const AttnArgs& p, dim3 grid, bool split) {
  constexpr int lds = attn_lds<HD, P16>();
  static std::atomic<uint64_t> lds_set{0};
  raise_lds_once((const void*)k_attn_mfma<HD, P16>, lds, &lds_set);
  FG_LAUNCH((k_attn_mfma<HD, P16>), grid, dim3(512), lds, s, p);
  if (!split) return;
  // the merge takes query blocks from the last one down, and a block's chunk
  // count never falls as its index grows: the grid ends before the blocks
  // that fit in one chunk (written by the attention kernel itself)
  int nm = 0;
  while (nm < p.nqb && chunk_count(p.nqb - 1 - nm, p.T, p.pos0, p.nvalid, p.ck) > 1) ++nm;
  const dim3 mgrid((unsigned)(p.nbh * nm * (QB / merge_queries<HD>())));
  if (nm > 0) FG_LAUNCH((k_attn_merge<HD, P16>), mgrid, dim3(256), 0, s, p);
}

void launch_attn_mfma(hipStream_t s, const Dims& d, const uint16_t* qs, const uint16_t* ks,
                      const uint16_t* vt, int B, int T, int npos, int pos0, int64_t q_plane,
                      int64_t kv_plane, float* scratch, float* y, uint16_t* ys,
                      int64_t ys_plane, bool f16, uint32_t* pos_cnt) {
  AttnArgs p;
  p.qs = qs;
  p.ks = ks;
  p.vt = vt;
  p.H = d.H;
  p.KH = d.KH;
  p.T = T;
  p.npos = npos;
  p.nvalid = pos0 + T;
  p.pos0 = pos0;
  p.nbh = B * d.H;
  p.nqb = (T + QB - 1) / QB;
  p.ck = attn_chunk_keys(p.nbh, T, pos0);
  p.iph = attn_items_per_head(T, pos0, p.ck);
  p.q_plane = q_plane;
  p.kv_plane = kv_plane;
  p.y = y;
  p.ys = ys;
  p.ys_plane = ys_plane;
  p.part = scratch;
  p.pos_cnt = pos_cnt;
  const dim3 grid((unsigned)(p.nbh * p.iph));
  const bool split = p.iph > p.nqb;  // some query block spans several chunks
  if (d.hd == 128) {
    if (f16) launch_attn_hd<128, true>(s, p, grid, split);
    else launch_attn_hd<128, false>(s, p, grid, split);
  } else {
    if (f16) launch_attn_hd<64, true>(s, p, grid, split);
    else launch_attn_hd<64, false>(s, p, grid, split);
  }
}

void launch_split_cache(hipStream_t s, const Dims& d, const void* kc, const void* vc, bool kv16,
                        int B, int maxT, int n, int npos, int64_t kv_plane, uint16_t* ks,
                        uint16_t* vt) {
  if (n <= 0) return;
  if (kv16)
    FG_LAUNCH(k_split_cache<uint16_t>, dim3(n, B), dim3(256), 0, s, (const uint16_t*)kc,
              (const uint16_t*)vc, d.KH, d.hd, maxT, n, npos, kv_plane, ks, vt);
  else
    FG_LAUNCH(k_split_cache<float>, dim3(n, B), dim3(256), 0, s, (const float*)kc,
              (const float*)vc, d.KH, d.hd, maxT, n, npos, kv_plane, ks, vt);
}

}  // namespace fgpt
