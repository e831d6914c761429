// kern_attn.hip -- causal chunk attention on MFMA (gfx950).
//
// Computes, for T queries at positions pos0..pos0+T-1 of each of B
// sequences, softmax(q k^T / sqrt(hd)) v over the keys 0..pos0+t with GQA
// head mapping h -> h / (H/KH): causal_attn (src/lib/fortran_attn.f90:30-117)
// when pos0 = 0 and attn_chunk (:376-425) in general.
//
// Formulation: each 64-wide wavefront owns 32 queries and walks 64-key
// tiles staged in LDS (keys and transposed values, shared by the block's two
// wavefronts). It forms S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (keys as
// MFMA rows, queries as columns), so the probabilities come out in exactly
// the register layout the B operand of O^T = V^T P^T needs: no LDS round
// trip for P. Online softmax (running max and sum per query) replaces the
// reference's two passes; the result differs from it only by rounding.
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
typedef float f32x16_t __attribute__((ext_vector_type(16)));

namespace {

constexpr int QG = 32;   // queries per wavefront (MFMA columns)
constexpr int KT = 32;   // keys per tile (MFMA rows)
constexpr float LOG2E = 1.4426950408889634f;

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) {
  return (uint32_t)lo | ((uint32_t)hi << 16);
}

// hi/lo bf16 halves of 8 floats, packed as the 8-element MFMA operand.
__device__ __forceinline__ void split8(const float* v, bf16x8_t& h, bf16x8_t& l) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const __bf16 hb = (__bf16)v[e];
    h[e] = hb;
    l[e] = (__bf16)(v[e] - (float)hb);
  }
}

// Block = 4 wavefronts = 2 query groups (32 queries each) x 2 key parities.
// Each step stages two 32-key tiles (one per parity) in LDS; the wavefront
// of parity p takes tile p, so both query groups share every tile and the
// key range is walked two tiles at a time. The two parities' running
// (max, sum, O) are merged through LDS at the end.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_mfma(const uint16_t* __restrict__ qs,
                                                   const uint16_t* __restrict__ ks,
                                                   const uint16_t* __restrict__ vt, int H, int KH,
                                                   int T, int npos, int nvalid, int pos0,
                                                   int64_t q_plane, int64_t kv_plane,
                                                   float* __restrict__ y,
                                                   uint16_t* __restrict__ ys, int64_t ys_plane) {
  constexpr int KSTR = HD + 8;  // bf16 per LDS key row
  constexpr int VSTR = KT + 8;  // bf16 per LDS value-dim row
  constexpr int NS = HD / 16;   // k-steps over the head dim
  constexpr int ND = HD / 32;   // 32-row blocks of O^T
  constexpr int PAR = 2 * KT * KSTR + 2 * HD * VSTR;  // bf16 per parity
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, g = lane >> 5, qi = lane & 31;
  const int qg = wv & 1, kp = wv >> 1;
  uint16_t* sKh = lds + kp * PAR;
  uint16_t* sKl = sKh + KT * KSTR;
  uint16_t* sVh = sKl + KT * KSTR;
  uint16_t* sVl = sVh + HD * VSTR;

  const int nqb = (T + 2 * QG - 1) / (2 * QG);
  const int qb = nqb - 1 - (int)blockIdx.x;  // longest causal rows first
  const int bh = blockIdx.y, b = bh / H, h = bh % H, kvh = h / (H / KH);
  const int64_t bk = (int64_t)b * KH + kvh;
  const int t = qb * 2 * QG + qg * QG + qi;  // this lane's query (column)
  const bool tok = t < T;
  const int qpos = pos0 + t;

  bf16x8_t qh[NS], ql[NS];
  {
    const uint16_t* qp = qs + ((int64_t)bh * T + (tok ? t : 0)) * HD + 8 * g;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      uint4 vh = *(const uint4*)(qp + 16 * s);
      uint4 vl = *(const uint4*)(qp + 16 * s + q_plane);
      if (!tok) vh = vl = make_uint4(0, 0, 0, 0);
      qh[s] = as_bf16x8(vh);
      ql[s] = as_bf16x8(vl);
    }
  }

  f32x16_t o[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[i][r] = 0.f;
  float m_run = -FLT_MAX, l_run = 0.f;           // in the log2 domain
  const float c = LOG2E / sqrtf((float)HD);

  const int t_last = min(qb * 2 * QG + 2 * QG, T) - 1;
  const int kend = min(nvalid, pos0 + t_last + 1);
  const int wq0 = pos0 + qb * 2 * QG + qg * QG;              // first query position of the wave
  const int wq1 = pos0 + min(qb * 2 * QG + qg * QG + QG, T) - 1;  // last

  for (int k0 = 0; k0 < kend; k0 += 2 * KT) {
    __syncthreads();
    // both parities' K tiles (KT keys x HD) and V^T tiles (HD x KT)
#pragma unroll
    for (int i = 0; i < 2 * KT * HD / 8 / 256; ++i) {
      const int cc = tid + 256 * i, p = cc / (KT * HD / 8), rem = cc % (KT * HD / 8);
      const int row = rem / (HD / 8), col = (rem % (HD / 8)) * 8;
      const int key = k0 + p * KT + row;
      uint4 vh = make_uint4(0, 0, 0, 0), vl = vh;
      if (key < nvalid) {
        const uint16_t* src = ks + (bk * npos + key) * HD + col;
        vh = *(const uint4*)src;
        vl = *(const uint4*)(src + kv_plane);
      }
      uint16_t* dh = lds + p * PAR + row * KSTR + col;
      *(uint4*)dh = vh;
      *(uint4*)(dh + KT * KSTR) = vl;
    }
#pragma unroll
    for (int i = 0; i < 2 * HD * KT / 8 / 256; ++i) {
      const int cc = tid + 256 * i, p = cc / (HD * KT / 8), rem = cc % (HD * KT / 8);
      const int d = rem / (KT / 8), col = (rem % (KT / 8)) * 8;
      const int key = k0 + p * KT + col;
      const uint16_t* src = vt + (bk * HD + d) * npos + key;
      uint4 vh, vl;
      if (key + 8 <= nvalid) {
        vh = *(const uint4*)src;
        vl = *(const uint4*)(src + kv_plane);
      } else {
        uint16_t eh[8], el[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const bool ok = key + e < nvalid;
          eh[e] = ok ? src[e] : 0;
          el[e] = ok ? src[e + kv_plane] : 0;
        }
        vh = make_uint4(pack2(eh[0], eh[1]), pack2(eh[2], eh[3]), pack2(eh[4], eh[5]),
                        pack2(eh[6], eh[7]));
        vl = make_uint4(pack2(el[0], el[1]), pack2(el[2], el[3]), pack2(el[4], el[5]),
                        pack2(el[6], el[7]));
      }
      uint16_t* dh = lds + p * PAR + 2 * KT * KSTR + d * VSTR + col;
      *(uint4*)dh = vh;
      *(uint4*)(dh + HD * VSTR) = vl;
    }
    __syncthreads();
    const int kt0 = k0 + kp * KT;       // this wavefront's tile
    if (kt0 > wq1 || kt0 >= kend) continue;

    // S^T (32 keys x 32 queries) = K Q^T with hi*hi + lo*hi + hi*lo
    f32x16_t sc;
#pragma unroll
    for (int r = 0; r < 16; ++r) sc[r] = 0.f;
    {
      const uint16_t* kh = sKh + qi * KSTR + 8 * g;
      const uint16_t* kl = sKl + qi * KSTR + 8 * g;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const bf16x8_t ah = as_bf16x8(*(const uint4*)(kh + 16 * s));
        const bf16x8_t al = as_bf16x8(*(const uint4*)(kl + 16 * s));
        sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, qh[s], sc, 0, 0, 0);
        sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, qh[s], sc, 0, 0, 0);
        sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, ql[s], sc, 0, 0, 0);
      }
    }
    // scores in the log2 domain; mask only tiles that reach the diagonal or
    // the end of the valid keys
    const bool need_mask = (kt0 + KT - 1 > wq0) || (kt0 + KT > nvalid);
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float v = sc[r] * c;
      if (need_mask) {
        const int key = kt0 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (key > qpos || key >= nvalid) v = -INFINITY;
      }
      sc[r] = v;
      mx = fmaxf(mx, v);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    if (__any(m_new > m_run)) {
      const float alpha = exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int i = 0; i < ND; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[i][r] *= alpha;
    }
    m_run = m_new;
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = exp2f(sc[r] - m_new);
      sc[r] = p;
      ps += p;
    }
    l_run += ps + __shfl_xor(ps, 32, 64);

    // O^T += V^T P^T over two 16-key steps
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[e] = sc[8 * s + e];
      bf16x8_t bh8, bl8;
      split8(pv, bh8, bl8);
      // A operand: V^T row d, keys 16s + {4g..4g+3, 8+4g..8+4g+3}, the key
      // order the S^T accumulator hands to this lane group
#pragma unroll
      for (int i = 0; i < ND; ++i) {
        const int d = 32 * i + qi;
        const uint16_t* vh = sVh + d * VSTR + 16 * s + 4 * g;
        const uint16_t* vl = sVl + d * VSTR + 16 * s + 4 * g;
        const uint2 h0 = *(const uint2*)vh, h1 = *(const uint2*)(vh + 8);
        const uint2 l0 = *(const uint2*)vl, l1 = *(const uint2*)(vl + 8);
        const bf16x8_t avh = as_bf16x8(make_uint4(h0.x, h0.y, h1.x, h1.y));
        const bf16x8_t avl = as_bf16x8(make_uint4(l0.x, l0.y, l1.x, l1.y));
        o[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(avh, bh8, o[i], 0, 0, 0);
        o[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(avl, bh8, o[i], 0, 0, 0);
        o[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(avh, bl8, o[i], 0, 0, 0);
      }
    }
  }

  // merge the two key parities of each query group through LDS
  __syncthreads();
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
  if (kp == 0 && tok) {
    const float m1 = xo[ND * 16 * 64 + lane], l1 = xo[ND * 16 * 64 + 64 + lane];
    const float m = fmaxf(m_run, m1);
    const float a0 = exp2f(m_run - m), a1 = exp2f(m1 - m);
    const float inv = 1.0f / (l_run * a0 + l1 * a1);
    const int64_t yo = ((int64_t)b * T + t) * ((int64_t)H * HD) + h * HD;
#pragma unroll
    for (int i = 0; i < ND; ++i)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = 32 * i + 8 * r4 + 4 * g;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = (o[i][4 * r4 + e] * a0 + xo[(i * 16 + 4 * r4 + e) * 64 + lane] * a1) * inv;
        if (ys) {
#pragma unroll
          for (int e = 0; e < 4; ++e) split_bf16(v[e], ys + yo + d + e, ys_plane);
        } else {
          *(float4*)(y + yo + d) = make_float4(v[0], v[1], v[2], v[3]);
        }
      }
  }
}

// Cache positions [0, n) of one layer, fp32 [B][maxT][KH*hd] -> hi/lo planes.
__global__ __launch_bounds__(256) void k_split_cache(const float* __restrict__ kc,
                                                     const float* __restrict__ vc, int KH, int hd,
                                                     int maxT, int n, int npos, int64_t kv_plane,
                                                     uint16_t* __restrict__ ks,
                                                     uint16_t* __restrict__ vt) {
  const int p = blockIdx.x, b = blockIdx.y, kd = KH * hd;
  if (p >= n) return;
  for (int i = threadIdx.x; i < kd; i += 256) {
    const int kvh = i / hd, d = i % hd;
    const int64_t src = ((int64_t)b * maxT + p) * kd + i;
    const int64_t bk = (int64_t)b * KH + kvh;
    const float kv = kc[src], vv = vc[src];
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

void launch_attn_mfma(hipStream_t s, const Dims& d, const uint16_t* qs, const uint16_t* ks,
                      const uint16_t* vt, int B, int T, int npos, int pos0, int64_t q_plane,
                      int64_t kv_plane, float* y, uint16_t* ys, int64_t ys_plane) {
  static bool lds_set = false;
  if (!lds_set) {
    (void)hipFuncSetAttribute((const void*)k_attn_mfma<128>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    (void)hipFuncSetAttribute((const void*)k_attn_mfma<64>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    lds_set = true;
  }
  const int nvalid = pos0 + T;
  dim3 grid((T + 2 * QG - 1) / (2 * QG), B * d.H);
  if (d.hd == 128) {
    const size_t lds = 2 * (2 * KT * (128 + 8) + 2 * 128 * (KT + 8)) * sizeof(uint16_t);
    hipLaunchKernelGGL(k_attn_mfma<128>, grid, dim3(256), lds, s, qs, ks, vt, d.H, d.KH, T,
                       npos, nvalid, pos0, q_plane, kv_plane, y, ys, ys_plane);
  } else {
    const size_t lds = 2 * (2 * KT * (64 + 8) + 2 * 64 * (KT + 8)) * sizeof(uint16_t);
    hipLaunchKernelGGL(k_attn_mfma<64>, grid, dim3(256), lds, s, qs, ks, vt, d.H, d.KH, T, npos,
                       nvalid, pos0, q_plane, kv_plane, y, ys, ys_plane);
  }
}

void launch_split_cache(hipStream_t s, const Dims& d, const float* kc, const float* vc, int B,
                        int maxT, int n, int npos, int64_t kv_plane, uint16_t* ks, uint16_t* vt) {
  if (n <= 0) return;
  hipLaunchKernelGGL(k_split_cache, dim3(n, B), dim3(256), 0, s, kc, vc, d.KH, d.hd, maxT, n, npos,
                     kv_plane, ks, vt);
}

}  // namespace fgpt
