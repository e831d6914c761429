// kern_epi.h -- the fused QKV epilogue shared by the GEMV and the MFMA GEMM.
//
// A rotation pair (stored rows r, r+1 of the pair-interleaved QKV matrix:
// head dims j and j+hd/2) arrives for token row m. q and k are rotated
// (src/lib/fortran_rope.f90:45-46: y1 = x1 c + x2 s, y2 = -x1 s + x2 c);
// k and the un-rotated v are appended to the cache at the row's position
// (src/lib/fortran_kv.f90:112-116): fp32, or bf16 (RNE) when a.kv16, in
// which case the split planes carry the rounded value (lo plane zero), so a
// chunk's attention sees what later steps read from the cache. When the split pointers are set
// (chunk attention follows), q, k and v are also written as operand planes
// (bf16 hi/lo, or one fp16 plane for a single-term pass) in the layouts the
// MFMA attention kernel reads:
//   qs [B][H][T][hd], ks [B][KH][npos][hd], vt [B][KH][hd][npos]
// (hi plane first, lo plane `*_plane` elements later).
#pragma once
#include "fgpt_internal.h"
#include "kern_common.h"

namespace fgpt {

// v = hi + lo in bf16: hi at p, lo at p + plane.
__device__ __forceinline__ void split_bf16(float v, uint16_t* p, int64_t plane) {
  const uint16_t h = f32_to_bf16_rne(v);
  p[0] = h;
  p[plane] = f32_to_bf16_rne(v - bf16_to_f32(h));
}

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// A store that bypasses cache allocation (NT) or an ordinary one. Outputs
// that only a later kernel reads, and that are too large to stay in L2 for
// it, are written streaming.
template <bool NT, typename V>
__device__ __forceinline__ void store_v(V* p, V v) {
  if constexpr (NT)
    __builtin_nontemporal_store(v, p);
  else
    *p = v;
}

// The same for two adjacent values as one 32-bit store per plane (p even).
template <bool NT = false>
__device__ __forceinline__ void split_bf16x2(float v0, float v1, uint16_t* p, int64_t plane) {
  const uint16_t h0 = f32_to_bf16_rne(v0), h1 = f32_to_bf16_rne(v1);
  const uint16_t l0 = f32_to_bf16_rne(v0 - bf16_to_f32(h0));
  const uint16_t l1 = f32_to_bf16_rne(v1 - bf16_to_f32(h1));
  store_v<NT>(reinterpret_cast<uint32_t*>(p), (uint32_t)h0 | ((uint32_t)h1 << 16));
  store_v<NT>(reinterpret_cast<uint32_t*>(p + plane), (uint32_t)l0 | ((uint32_t)l1 << 16));
}

// The same for four adjacent values as one 64-bit store per plane (p a
// multiple of 4 elements).
template <bool NT = false>
__device__ __forceinline__ void split_bf16x4(const float (&v)[4], uint16_t* p, int64_t plane) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint16_t hb = f32_to_bf16_rne(v[i]);
    h[i] = hb;
    l[i] = f32_to_bf16_rne(v[i] - bf16_to_f32(hb));
  }
  store_v<NT>(reinterpret_cast<u32x2_t*>(p), u32x2_t{h[0] | (h[1] << 16), h[2] | (h[3] << 16)});
  store_v<NT>(reinterpret_cast<u32x2_t*>(p + plane), u32x2_t{l[0] | (l[1] << 16), l[2] | (l[3] << 16)});
}

// Cache element stores: fp32, or bf16 (RNE) for a bf16 cache.
__device__ __forceinline__ void kv_put(const GemvArgs& a, float* c, int64_t i, float v) {
  if (a.kv16)
    reinterpret_cast<uint16_t*>(c)[i] = f32_to_bf16_rne(v);
  else
    c[i] = v;
}
__device__ __forceinline__ void kv_put4(const GemvArgs& a, float* c, int64_t i, float v0, float v1,
                                        float v2, float v3) {
  if (a.kv16) {
    const uint32_t lo = (uint32_t)f32_to_bf16_rne(v0) | ((uint32_t)f32_to_bf16_rne(v1) << 16);
    const uint32_t hi = (uint32_t)f32_to_bf16_rne(v2) | ((uint32_t)f32_to_bf16_rne(v3) << 16);
    *reinterpret_cast<u32x2_t*>(reinterpret_cast<uint16_t*>(c) + i) = u32x2_t{lo, hi};
  } else {
    *reinterpret_cast<float4*>(c + i) = make_float4(v0, v1, v2, v3);
  }
}
// The value a bf16 cache holds for v (v itself for an fp32 cache).
__device__ __forceinline__ float kv_val(const GemvArgs& a, float v) {
  return a.kv16 ? bf16_to_f32(f32_to_bf16_rne(v)) : v;
}

// Operand planes of the MFMA kernels: a value goes in as bf16 hi at p and
// bf16 lo at p + plane (the split format, ~16 significant bits), or, for a
// single-term fp16 pass (P16), as one fp16 at p.
template <bool P16>
__device__ __forceinline__ void put1(float v, uint16_t* p, int64_t plane) {
  if constexpr (P16)
    p[0] = f32_to_f16_rne(v);
  else
    split_bf16(v, p, plane);
}
template <bool P16, bool NT = false>
__device__ __forceinline__ void put2(float v0, float v1, uint16_t* p, int64_t plane) {
  if constexpr (P16)
    store_v<NT>(reinterpret_cast<uint32_t*>(p),
                (uint32_t)f32_to_f16_rne(v0) | ((uint32_t)f32_to_f16_rne(v1) << 16));
  else
    split_bf16x2<NT>(v0, v1, p, plane);
}
template <bool P16, bool NT = false>
__device__ __forceinline__ void put4(const float (&v)[4], uint16_t* p, int64_t plane) {
  if constexpr (P16)
    store_v<NT>(reinterpret_cast<u32x2_t*>(p),
                u32x2_t{(uint32_t)f32_to_f16_rne(v[0]) | ((uint32_t)f32_to_f16_rne(v[1]) << 16),
                        (uint32_t)f32_to_f16_rne(v[2]) | ((uint32_t)f32_to_f16_rne(v[3]) << 16)});
  else
    split_bf16x4<NT>(v, p, plane);
}

// The single-term fp16 pass stores its activations as fp16, whose largest
// finite value is 65504: an fp32 value of magnitude 65520 or more (or one
// that is not finite) would become inf. Such a value raises the pass's
// overflow flag, which the host turns into an error instead of returning
// inf / NaN logits.
template <bool P16>
__device__ __forceinline__ void f16_guard(const GemvArgs& a, float v) {
  if constexpr (P16) {
    if (!(fabsf(v) < 65520.f) && a.ovf) *a.ovf = 1u;
  }
}

// RoPE coefficients of stored column pair r for token row m (q and k
// columns; v columns take none).
__device__ __forceinline__ void qkv_pair_coeffs(const GemvArgs& a, int m, int pos0, int r,
                                                float& cs, float& sn) {
  const int hd = a.hd, qd = a.H * hd, kd = a.KH * hd;
  if (r < qd + kd) {
    const int base = r < qd ? r : r - qd;
    const int64_t at = (int64_t)(pos0 + m % a.T) * (hd / 2) + ((base % hd) >> 1);
    cs = a.cosb[at];
    sn = a.sinb[at];
  }
}

// qkv_pair_epilogue with the pair's RoPE coefficients already loaded.
template <bool P16 = false>
__device__ __forceinline__ void qkv_pair_store(const GemvArgs& a, int m, int pos0, int r,
                                               float x1, float x2, float cs, float sn) {
  const int hd = a.hd, qd = a.H * hd, kd = a.KH * hd;
  const int b = m / a.T, t = m % a.T, pos = pos0 + t;
  if (r < qd + kd) {
    const bool isq = r < qd;
    const int base = isq ? r : r - qd;
    const int head = base / hd, j = (base % hd) >> 1;
    const float y1 = x1 * cs + x2 * sn;
    const float y2 = x1 * (-sn) + x2 * cs;
    f16_guard<P16>(a, y1);
    f16_guard<P16>(a, y2);
    if (isq) {
      if (a.qs) {
        uint16_t* p = a.qs + (((int64_t)b * a.H + head) * a.T + t) * hd;
        put1<P16>(y1, p + j, a.q_plane);
        put1<P16>(y2, p + j + hd / 2, a.q_plane);
      } else {
        float* q = a.y + (int64_t)m * qd + head * hd;
        q[j] = y1;
        q[j + hd / 2] = y2;
      }
    } else {
      if (a.kc) {
        const int64_t k = ((int64_t)b * a.maxT + pos) * kd + head * hd;
        kv_put(a, a.kc, k + j, y1);
        kv_put(a, a.kc, k + j + hd / 2, y2);
      }
      if (a.ks) {
        uint16_t* p = a.ks + (((int64_t)b * a.KH + head) * a.npos + pos) * hd;
        put1<P16>(kv_val(a, y1), p + j, a.kv_plane);
        put1<P16>(kv_val(a, y2), p + j + hd / 2, a.kv_plane);
      }
    }
  } else {
    const int base = r - qd - kd;
    const int head = base / hd, j = (base % hd) >> 1;
    f16_guard<P16>(a, x1);
    f16_guard<P16>(a, x2);
    if (a.vc) {
      const int64_t v = ((int64_t)b * a.maxT + pos) * kd + head * hd;
      kv_put(a, a.vc, v + j, x1);
      kv_put(a, a.vc, v + j + hd / 2, x2);
    }
    if (a.vt) {
      uint16_t* p = a.vt + ((int64_t)b * a.KH + head) * hd * a.npos + pos;
      put1<P16>(kv_val(a, x1), p + (int64_t)j * a.npos, a.kv_plane);
      put1<P16>(kv_val(a, x2), p + (int64_t)(j + hd / 2) * a.npos, a.kv_plane);
    }
  }
}

// Four rotation pairs at stored columns r8 .. r8+7 (r8 % 8 == 0, so one
// head and dims j .. j+3 with j % 4 == 0) of token row m, x the eight
// values, cs/sn the four pairs' RoPE coefficients: the arithmetic of
// qkv_pair_store, with each plane's four dims written by one wide store.
template <bool NT = false, bool P16 = false>
__device__ __forceinline__ void qkv_quad_store(const GemvArgs& a, int m, int pos0, int r8,
                                               const float (&x)[8], const float4& cs,
                                               const float4& sn) {
  const int hd = a.hd, qd = a.H * hd, kd = a.KH * hd;
  const int b = m / a.T, t = m % a.T, pos = pos0 + t;
  const float c[4] = {cs.x, cs.y, cs.z, cs.w}, s[4] = {sn.x, sn.y, sn.z, sn.w};
  float y1[4], y2[4];
  if (r8 < qd + kd) {
    const bool isq = r8 < qd;
    const int base = isq ? r8 : r8 - qd;
    const int head = base / hd, j = (base % hd) >> 1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x1 = x[2 * i], x2 = x[2 * i + 1];
      y1[i] = x1 * c[i] + x2 * s[i];
      y2[i] = x1 * (-s[i]) + x2 * c[i];
      f16_guard<P16>(a, y1[i]);
      f16_guard<P16>(a, y2[i]);
    }
    if (isq) {
      if (a.qs) {
        uint16_t* p = a.qs + (((int64_t)b * a.H + head) * a.T + t) * hd;
        put4<P16, NT>(y1, p + j, a.q_plane);
        put4<P16, NT>(y2, p + j + hd / 2, a.q_plane);
      } else {
        float* q = a.y + (int64_t)m * qd + head * hd;
        *reinterpret_cast<float4*>(q + j) = make_float4(y1[0], y1[1], y1[2], y1[3]);
        *reinterpret_cast<float4*>(q + j + hd / 2) = make_float4(y2[0], y2[1], y2[2], y2[3]);
      }
    } else {
      if (a.kc) {
        const int64_t k = ((int64_t)b * a.maxT + pos) * kd + head * hd;
        kv_put4(a, a.kc, k + j, y1[0], y1[1], y1[2], y1[3]);
        kv_put4(a, a.kc, k + j + hd / 2, y2[0], y2[1], y2[2], y2[3]);
      }
      if (a.ks) {
        uint16_t* p = a.ks + (((int64_t)b * a.KH + head) * a.npos + pos) * hd;
        if (a.kv16) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            y1[i] = kv_val(a, y1[i]);
            y2[i] = kv_val(a, y2[i]);
          }
        }
        put4<P16, NT>(y1, p + j, a.kv_plane);
        put4<P16, NT>(y2, p + j + hd / 2, a.kv_plane);
      }
    }
  } else {
    const int base = r8 - qd - kd;
    const int head = base / hd, j = (base % hd) >> 1;
#pragma unroll
    for (int i = 0; i < 8; ++i) f16_guard<P16>(a, x[i]);
    if (a.vc) {
      const int64_t v = ((int64_t)b * a.maxT + pos) * kd + head * hd;
      kv_put4(a, a.vc, v + j, x[0], x[2], x[4], x[6]);
      kv_put4(a, a.vc, v + j + hd / 2, x[1], x[3], x[5], x[7]);
    }
    if (a.vt) {  // (tiles holding v columns normally take the row-fast path)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint16_t* p = a.vt + ((int64_t)b * a.KH + head) * hd * a.npos + pos;
        put1<P16>(kv_val(a, x[2 * i]), p + (int64_t)(j + i) * a.npos, a.kv_plane);
        put1<P16>(kv_val(a, x[2 * i + 1]), p + (int64_t)(j + i + hd / 2) * a.npos, a.kv_plane);
      }
    }
  }
}

template <bool P16 = false>
__device__ __forceinline__ void qkv_pair_epilogue(const GemvArgs& a, int m, int pos0, int r,
                                                  float x1, float x2) {
  float cs = 0.f, sn = 0.f;
  qkv_pair_coeffs(a, m, pos0, r, cs, sn);
  qkv_pair_store<P16>(a, m, pos0, r, x1, x2, cs, sn);
}

// One element of a rotation pair, for producers that hold one column per
// lane: stored column r of the pair-interleaved QKV matrix (r even: head
// dim j, r odd: dim j + hd/2, j = (r % hd) / 2), `own` its value and `other`
// the value of the pair's other column. Same arithmetic and destinations as
// qkv_pair_epilogue.
template <bool P16 = false>
__device__ __forceinline__ void qkv_elem_epilogue(const GemvArgs& a, int m, int pos0, int r,
                                                  float own, float other) {
  const int hd = a.hd, qd = a.H * hd, kd = a.KH * hd;
  const int b = m / a.T, t = m % a.T, pos = pos0 + t;
  const bool odd = r & 1;
  if (r < qd + kd) {
    const bool isq = r < qd;
    const int base = isq ? r : r - qd;
    const int head = base / hd, j = (base % hd) >> 1, dim = odd ? j + hd / 2 : j;
    const float cs = a.cosb[(int64_t)pos * (hd / 2) + j];
    const float sn = a.sinb[(int64_t)pos * (hd / 2) + j];
    const float x1 = odd ? other : own, x2 = odd ? own : other;
    const float yv = odd ? x1 * (-sn) + x2 * cs : x1 * cs + x2 * sn;
    f16_guard<P16>(a, yv);
    if (isq) {
      if (a.qs)
        put1<P16>(yv, a.qs + (((int64_t)b * a.H + head) * a.T + t) * hd + dim, a.q_plane);
      else
        a.y[(int64_t)m * qd + head * hd + dim] = yv;
    } else {
      if (a.kc) kv_put(a, a.kc, ((int64_t)b * a.maxT + pos) * kd + head * hd + dim, yv);
      if (a.ks)
        put1<P16>(kv_val(a, yv), a.ks + (((int64_t)b * a.KH + head) * a.npos + pos) * hd + dim,
                   a.kv_plane);
    }
  } else {
    const int base = r - qd - kd;
    const int head = base / hd, j = (base % hd) >> 1, dim = odd ? j + hd / 2 : j;
    f16_guard<P16>(a, own);
    if (a.vc) kv_put(a, a.vc, ((int64_t)b * a.maxT + pos) * kd + head * hd + dim, own);
    if (a.vt)
      put1<P16>(kv_val(a, own), a.vt + (((int64_t)b * a.KH + head) * hd + dim) * a.npos + pos,
                 a.kv_plane);
  }
}

}  // namespace fgpt
