// kern_fused.h -- device helpers shared by the persistent decode loops
// (kern_fused.hip: one KV head per query head; kern_fused_gqa.hip: grouped
// KV heads): the exchange slots between workgroups, their bounded waits,
// and the LDS dot products and wave sums the GEMV phases use.
#pragma once
#include <float.h>

#include "fgpt_internal.h"
#include "kern_common.h"

namespace fgpt {
namespace {

constexpr int FUSED_HD = 128;            // head dim this kernel is built for
constexpr int FUSED_THREADS = 320;       // 4 compute waves + 1 loader wave
constexpr long FUSED_MAX_SPIN = 1l << 20;  // polls before a hand-over is given up
// copies of the lm_head argmax candidates, each read by 256 / FUSED_LMC
// workgroups (the lm_head pseudo-layer: one copy read by all 256 5.4 us,
// 8 copies 4.6, 16 4.9, 64 5.3: more copies cost more write-through stores)
constexpr int FUSED_LMC = 8;
// sleeps (s_sleep units) before the first read and between reads of a
// hand-over across XCDs in kern_fused_gqa.hip (see slots_wait); depth-20
// GQA decode at 2047-2302 positions, ms a token: XPRE 8 0.382, 16 0.349,
// 24 0.390 (XGAP 4); XGAP 0 0.3477, 1 0.3475, 2 0.3484, 4 0.3502, 10 0.3585
// (XPRE 16, means of runs on one box); at XGAP 1, XPRE 12 0.357, 16 0.346,
// 20 0.356
constexpr int XPRE = 16, XGAP = 1;

__device__ __forceinline__ uint64_t slot_pack(float v, uint32_t ep) {
  return ((uint64_t)ep << 32) | (uint64_t)__float_as_uint(v);
}
__device__ __forceinline__ uint64_t slot_load(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// hand-over to workgroups of other XCDs: write-through to memory
__device__ __forceinline__ void slot_put_dev(uint64_t* p, float v, uint32_t ep) {
  __hip_atomic_store(p, slot_pack(v, ep), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// hand-over within the XCD: a plain store into the shared L2
__device__ __forceinline__ void slot_put_xcd(uint64_t* p, float v, uint32_t ep) {
  __hip_atomic_store(p, slot_pack(v, ep), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Wait until the n (<= NMAX) slots p[i * stride] carry epoch ep, then
// return their values in out. All loads go out at once; only slots still
// short of the epoch are read again. false: the bound was reached or the
// error flag was raised elsewhere (the flag is then raised here too).
// PRE, GAP: s_sleep units (64 clocks) before the first read and before each
// read again. Where the weights stream from HBM (kern_fused_gqa.hip), slots
// written through from other XCDs arrive later than a poll issued right
// after the reader's own publish, and polls that go out early slow the
// hand-over down (the depth-20 q/k/v hand-over: 3.0 us polling at once, 1.6
// us after a sleep of 16); where everything stays in the Infinity Cache
// (kern_fused.hip) polling at once is faster (the depth-12 loop with
// XPRE/XGAP on its hand-overs across XCDs: 0.1206 against 0.1147 ms a token,
// A/B on one box).
template <int NMAX, int PRE = 0, int GAP = 0>
__device__ bool slots_wait(const uint64_t* p, int64_t stride, int n, uint32_t ep, float* out,
                           uint32_t* err) {
  if (PRE > 0) __builtin_amdgcn_s_sleep(PRE);
  uint64_t v[NMAX];
#pragma unroll
  for (int i = 0; i < NMAX; ++i) v[i] = i < n ? slot_load(p + i * stride) : slot_pack(0.f, ep);
  for (long spin = 0;; ++spin) {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < NMAX; ++i) ok = ok && (uint32_t)(v[i] >> 32) == ep;
    if (ok) break;
    if (spin >= FUSED_MAX_SPIN ||
        ((spin & 255) == 255 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))) {
      __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
    if (GAP > 0) __builtin_amdgcn_s_sleep(GAP);
#pragma unroll
    for (int i = 0; i < NMAX; ++i)
      if (i < n && (uint32_t)(v[i] >> 32) != ep) v[i] = slot_load(p + i * stride);
  }
#pragma unroll
  for (int i = 0; i < NMAX; ++i)
    if (i < n) out[i] = __uint_as_float((uint32_t)v[i]);
  return true;
}

// Gather n slots (lane-strided over the 256 compute threads) into dst.
template <int NMAX, int PRE = 0, int GAP = 0>
__device__ bool gather_slots(const uint64_t* p, int n, uint32_t ep, float* dst, int tid,
                             uint32_t* err) {
  float v[NMAX];
  const int cnt = tid < n ? (n - tid + 255) / 256 : 0;
  if (!slots_wait<NMAX, PRE, GAP>(p + tid, 256, cnt, ep, v, err)) return false;
#pragma unroll
  for (int i = 0; i < NMAX; ++i)
    if (i < cnt) dst[tid + 256 * i] = v[i];
  return true;
}

// The lane's part of the dot products of NR bf16 rows (LDS, at byte
// offsets roff from w) with fp32 x (LDS) over K (a multiple of 128): the
// lane takes elements [CE k, CE k + CE) for k = lane, lane+64, ... (CE = 4
// when K is a multiple of 256, else 2, so every lane has the same count).
// Every load of the lane's chunks is issued before any arithmetic.
template <int NR, int K>
__device__ __forceinline__ void dot_rows(const uint8_t* w, const int (&roff)[NR], const float* x,
                                         int lane, float (&acc)[NR]) {
  static_assert(K % 128 == 0, "K a multiple of 128");
  constexpr int CE = K % 256 == 0 ? 4 : 2;
  constexpr int IT = K / (64 * CE);
  if constexpr (CE == 4) {
    float4 xv[IT];
    uint2 wv[IT][NR];
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      xv[i] = *(const float4*)(x + 4 * (lane + 64 * i));
#pragma unroll
      for (int r = 0; r < NR; ++r) wv[i][r] = *(const uint2*)(w + roff[r] + 8 * (lane + 64 * i));
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      float t = 0.f;
#pragma unroll
      for (int i = 0; i < IT; ++i)
        t += xv[i].x * __uint_as_float(wv[i][r].x << 16) +
             xv[i].y * __uint_as_float(wv[i][r].x & 0xFFFF0000u) +
             xv[i].z * __uint_as_float(wv[i][r].y << 16) +
             xv[i].w * __uint_as_float(wv[i][r].y & 0xFFFF0000u);
      acc[r] = t;
    }
  } else {
    float2 xv[IT];
    uint32_t wv[IT][NR];
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      xv[i] = *(const float2*)(x + 2 * (lane + 64 * i));
#pragma unroll
      for (int r = 0; r < NR; ++r) wv[i][r] = *(const uint32_t*)(w + roff[r] + 4 * (lane + 64 * i));
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      float t = 0.f;
#pragma unroll
      for (int i = 0; i < IT; ++i)
        t += xv[i].x * __uint_as_float(wv[i][r] << 16) +
             xv[i].y * __uint_as_float(wv[i][r] & 0xFFFF0000u);
      acc[r] = t;
    }
  }
}

// sum(x^2) over the wave, x (LDS) of K elements in dot_rows' lane split
template <int K>
__device__ __forceinline__ float sumsq(const float* x, int lane) {
  constexpr int IT = K / 256;
  float4 xv[IT];
#pragma unroll
  for (int i = 0; i < IT; ++i) xv[i] = *(const float4*)(x + 4 * (lane + 64 * i));
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < IT; ++i)
    ss += xv[i].x * xv[i].x + xv[i].y * xv[i].y + xv[i].z * xv[i].z + xv[i].w * xv[i].w;
  return wave_sum(ss);
}

__device__ __forceinline__ void amax_take(float& v, int& i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

constexpr int64_t round1k(int64_t x) { return (x + 1023) / 1024 * 1024; }

// Sums over the wave of RP (4 or 8) per-lane values at once: v[r] of every
// lane lands in this wave's LDS scratch (RP x 64 floats), each group of
// LPO = 64/RP lanes adds RP consecutive partials of one value, then a DPP
// butterfly over the group (quad permutes, then the half-row and row
// mirrors, which pair the same lanes as strides 4 and 8 once the smaller
// groups are uniform). The sum of v[r] is left in lanes [r*LPO, (r+1)*LPO).
template <int RP>
__device__ __forceinline__ float multi_sum(const float (&v)[RP], float* scr, int lane) {
  constexpr int LPO = 64 / RP;
  static_assert(RP == 4 || RP == 8, "groups of 16 or 8 lanes");
#pragma unroll
  for (int r = 0; r < RP; ++r) scr[r * 64 + lane] = v[r];
  const float* p = scr + (lane / LPO) * 64 + (lane % LPO) * RP;
  const float4 a = *(const float4*)p;
  float t = (a.x + a.y) + (a.z + a.w);
  if (RP == 8) {
    const float4 b = *(const float4*)(p + 4);
    t += (b.x + b.y) + (b.z + b.w);
  }
  t += dpp_f<0xB1>(t);
  t += dpp_f<0x4E>(t);
  t += dpp_f<0x141>(t);
  if (LPO == 16) t += dpp_f<0x140>(t);
  return t;
}

__device__ __forceinline__ float lane_value(float v, int src) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), src));
}

}  // namespace
}  // namespace fgpt
