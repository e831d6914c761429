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

namespace fgpt {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

namespace {

constexpr int QW = 32;   // queries per wavefront
constexpr int NW = 2;    // wavefronts per block
constexpr int KT = 64;   // keys per LDS tile

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) {
  return (uint32_t)lo | ((uint32_t)hi << 16);
}

template <int HD>
__global__ __launch_bounds__(NW * 64) void k_attn_mfma(const uint16_t* __restrict__ qs,
                                                       const uint16_t* __restrict__ ks,
                                                       const uint16_t* __restrict__ vt, int H,
                                                       int KH, int T, int npos, int nvalid,
                                                       int pos0, int64_t q_plane,
                                                       int64_t kv_plane, float* __restrict__ y) {
  constexpr int KSTR = HD + 8;  // bf16 per LDS key row (16-byte pad)
  constexpr int VSTR = KT + 8;  // bf16 per LDS value-dim row
  constexpr int NS = HD / 16;   // k-steps over the head dim
  constexpr int ND = HD / 32;   // 32-row blocks of O^T
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  uint16_t* sKh = lds;
  uint16_t* sKl = sKh + KT * KSTR;
  uint16_t* sVh = sKl + KT * KSTR;
  uint16_t* sVl = sVh + HD * VSTR;

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, g = lane >> 5, qi = lane & 31;
  const int nqt = (T + NW * QW - 1) / (NW * QW);
  const int qt = nqt - 1 - (int)blockIdx.x;  // longest causal rows first
  const int bh = blockIdx.y, b = bh / H, h = bh % H, kvh = h / (H / KH);
  const int64_t bk = (int64_t)b * KH + kvh;
  const int t = qt * NW * QW + wv * QW + qi;  // this lane's query (column)
  const bool tok = t < T;
  const int qpos = pos0 + t;

  // B operand (Q^T): lane holds q[t][16s + 8g .. +7], hi and lo
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
  float m_run = -FLT_MAX, l_run = 0.f;
  const float scale = 1.0f / sqrtf((float)HD);

  const int t_last = min(qt * NW * QW + NW * QW, T) - 1;
  const int kend = min(nvalid, pos0 + t_last + 1);
  const int wave_last_t = min(qt * NW * QW + wv * QW + QW, T) - 1;
  const int wave_kmax = pos0 + wave_last_t;  // highest key any query of this wave sees

  for (int k0 = 0; k0 < kend; k0 += KT) {
    __syncthreads();
    // K tile: KT keys x HD, both planes; zero beyond the valid keys
    for (int c = tid; c < KT * HD / 8; c += NW * 64) {
      const int row = c / (HD / 8), col = (c % (HD / 8)) * 8;
      uint4 vh = make_uint4(0, 0, 0, 0), vl = vh;
      if (k0 + row < nvalid) {
        const uint16_t* src = ks + (bk * npos + k0 + row) * HD + col;
        vh = *(const uint4*)src;
        vl = *(const uint4*)(src + kv_plane);
      }
      *(uint4*)(sKh + row * KSTR + col) = vh;
      *(uint4*)(sKl + row * KSTR + col) = vl;
    }
    // V^T tile: HD dims x KT keys
    for (int c = tid; c < HD * KT / 8; c += NW * 64) {
      const int d = c / (KT / 8), col = (c % (KT / 8)) * 8;
      const uint16_t* src = vt + (bk * HD + d) * npos + k0 + col;
      uint4 vh, vl;
      if (k0 + col + 8 <= nvalid) {
        vh = *(const uint4*)src;
        vl = *(const uint4*)(src + kv_plane);
      } else {
        uint16_t eh[8], el[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const bool ok = k0 + col + e < nvalid;
          eh[e] = ok ? src[e] : 0;
          el[e] = ok ? src[e + kv_plane] : 0;
        }
        vh = make_uint4(pack2(eh[0], eh[1]), pack2(eh[2], eh[3]), pack2(eh[4], eh[5]),
                        pack2(eh[6], eh[7]));
        vl = make_uint4(pack2(el[0], el[1]), pack2(el[2], el[3]), pack2(el[4], el[5]),
                        pack2(el[6], el[7]));
      }
      *(uint4*)(sVh + d * VSTR + col) = vh;
      *(uint4*)(sVl + d * VSTR + col) = vl;
    }
    __syncthreads();
    if (k0 > wave_kmax) continue;  // every key of this tile is in this wave's future

    // S^T blocks: 32 keys x 32 queries each
    f32x16_t sc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[kb][r] = 0.f;
      const uint16_t* kr_h = sKh + (32 * kb + qi) * KSTR + 8 * g;
      const uint16_t* kr_l = sKl + (32 * kb + qi) * KSTR + 8 * g;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const bf16x8_t ah = as_bf16x8(*(const uint4*)(kr_h + 16 * s));
        const bf16x8_t al = as_bf16x8(*(const uint4*)(kr_l + 16 * s));
        sc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, qh[s], sc[kb], 0, 0, 0);
        sc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, qh[s], sc[kb], 0, 0, 0);
        sc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, ql[s], sc[kb], 0, 0, 0);
      }
    }
    // scale, causal / range mask, running max and sum per query
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + 32 * kb + 8 * (r >> 2) + 4 * g + (r & 3);
        float v = sc[kb][r] * scale;
        if (key > qpos || key >= nvalid) v = -INFINITY;
        sc[kb][r] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = expf(m_run - m_new);
    float ps = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = expf(sc[kb][r] - m_new);
        sc[kb][r] = p;
        ps += p;
      }
    ps += __shfl_xor(ps, 32, 64);
    l_run = l_run * alpha + ps;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < ND; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[i][r] *= alpha;

    // O^T += V^T P^T over four 16-key steps
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int kb = s >> 1, rb = (s & 1) * 8;
      uint16_t ph[8], pl[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float p = sc[kb][rb + e];
        ph[e] = f32_to_bf16_rne(p);
        pl[e] = f32_to_bf16_rne(p - bf16_to_f32(ph[e]));
      }
      const bf16x8_t bh8 = as_bf16x8(make_uint4(pack2(ph[0], ph[1]), pack2(ph[2], ph[3]),
                                                pack2(ph[4], ph[5]), pack2(ph[6], ph[7])));
      const bf16x8_t bl8 = as_bf16x8(make_uint4(pack2(pl[0], pl[1]), pack2(pl[2], pl[3]),
                                                pack2(pl[4], pl[5]), pack2(pl[6], pl[7])));
      // A operand: V^T row d, keys 16s + {4g..4g+3, 8+4g..8+4g+3} (the key
      // order the S^T accumulator hands to this lane group)
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

  if (tok) {
    const float inv = 1.0f / l_run;
    float* yr = y + ((int64_t)b * T + t) * ((int64_t)H * HD) + h * HD;
#pragma unroll
    for (int i = 0; i < ND; ++i)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = 32 * i + 8 * r4 + 4 * g;
        float4 v;
        v.x = o[i][4 * r4 + 0] * inv;
        v.y = o[i][4 * r4 + 1] * inv;
        v.z = o[i][4 * r4 + 2] * inv;
        v.w = o[i][4 * r4 + 3] * inv;
        *(float4*)(yr + d) = v;
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
                      int64_t kv_plane, float* y) {
  static bool lds_set = false;
  if (!lds_set) {
    (void)hipFuncSetAttribute((const void*)k_attn_mfma<128>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    (void)hipFuncSetAttribute((const void*)k_attn_mfma<64>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    lds_set = true;
  }
  const int nvalid = pos0 + T;
  dim3 grid((T + NW * QW - 1) / (NW * QW), B * d.H);
  if (d.hd == 128) {
    const size_t lds = 2 * (KT * (128 + 8) + 128 * (KT + 8)) * sizeof(uint16_t);
    hipLaunchKernelGGL(k_attn_mfma<128>, grid, dim3(NW * 64), lds, s, qs, ks, vt, d.H, d.KH, T,
                       npos, nvalid, pos0, q_plane, kv_plane, y);
  } else {
    const size_t lds = 2 * (KT * (64 + 8) + 64 * (KT + 8)) * sizeof(uint16_t);
    hipLaunchKernelGGL(k_attn_mfma<64>, grid, dim3(NW * 64), lds, s, qs, ks, vt, d.H, d.KH, T,
                       npos, nvalid, pos0, q_plane, kv_plane, y);
  }
}

void launch_split_cache(hipStream_t s, const Dims& d, const float* kc, const float* vc, int B,
                        int maxT, int n, int npos, int64_t kv_plane, uint16_t* ks, uint16_t* vt) {
  if (n <= 0) return;
  hipLaunchKernelGGL(k_split_cache, dim3(n, B), dim3(256), 0, s, kc, vc, d.KH, d.hd, maxT, n, npos,
                     kv_plane, ks, vt);
}

}  // namespace fgpt
