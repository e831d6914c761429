// kern_sample.hip -- token sampling on the device: sample_next of
// src/lib/sample.f90:153-233 for one row of logits, by one 1024-thread
// workgroup with the row in LDS. In the reference's order: presence /
// frequency penalties over the whole history or over the last pwin ids
// (:33-51, :77-104), the repetition penalty (:56-71), the no-repeat n-gram
// ban (:109-130), the byte-level mask (:141-151), then either the first-max
// argmax (temp <= 0, no random draw) or a draw from softmax(logits / temp)
// restricted to the smallest prefix of ids, in descending probability,
// whose mass reaches topp, with the xorshift64* generator (:15-28).
//
// Differences of arithmetic order from the reference (which sums, sorts and
// scans sequentially): the softmax sum and the cumulative sums are tree and
// block scans; the descending sort is a bitonic network with ties in id
// order (the reference's quicksort leaves ties in an order of its own);
// expf is the device's. They move the drawn id only when the draw lands
// within rounding of a cumulative boundary, or inside a run of equal
// probabilities.
#include <cfloat>

#include "fgpt_internal.h"
#include "kern_common.h"

namespace fgpt {
namespace {

constexpr int ST = 1024;  // threads of a sampling workgroup
constexpr int NW = ST / 64;

// xorshift64* of rand_u01: the state advances, the top 24 bits of
// state * 2685821657736338717 give u in [0, 1)
__device__ float rand_u01(int64_t* st) {
  uint64_t x = (uint64_t)*st;
  if (x == 0) x = 2685821657736338717ull;
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  *st = (int64_t)x;
  const uint64_t y = x * 2685821657736338717ull;
  return (float)((y >> 40) & 0xFFFFFFull) / 16777216.0f;
}

__device__ __forceinline__ void amax_pick(float& v, int& i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

// first index of the maximum of w[0:V) (the reference's strict > scan)
__device__ int block_argmax(const float* w, int V, float* rv, int* ri) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = tid; i < V; i += ST)
    if (w[i] > bv) {
      bv = w[i];
      bi = i;
    }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) amax_pick(bv, bi, __shfl_xor(bv, o, 64), __shfl_xor(bi, o, 64));
  __syncthreads();
  if (lane == 0) {
    rv[wv] = bv;
    ri[wv] = bi;
  }
  __syncthreads();
  bv = rv[0];
  bi = ri[0];
  for (int k = 1; k < NW; ++k) amax_pick(bv, bi, rv[k], ri[k]);
  __syncthreads();
  return bi == 0x7fffffff ? 0 : bi;
}

__device__ float block_max(const float* w, int V, float* red) {
  float m = -INFINITY;
  for (int i = threadIdx.x; i < V; i += ST) m = fmaxf(m, w[i]);
  m = wave_max(m);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  m = red[0];
  for (int k = 1; k < NW; ++k) m = fmaxf(m, red[k]);
  __syncthreads();
  return m;
}

__device__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = 0.f;
  for (int k = 0; k < NW; ++k) t += red[k];
  __syncthreads();
  return t;
}

__device__ int block_min(int v, int* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  for (int k = 0; k < NW; ++k) v = min(v, red[k]);
  __syncthreads();
  return v;
}

// per-id counts of gen[lo:hi) into cnt[0:V) (ids outside [0, V) ignored)
__device__ void count_ids(const int32_t* gen, int lo, int hi, int V, int* cnt) {
  for (int i = threadIdx.x; i < V; i += ST) cnt[i] = 0;
  __syncthreads();
  for (int j = lo + threadIdx.x; j < hi; j += ST) {
    const int g = gen[j];
    if (g >= 0 && g < V) atomicAdd(&cnt[g], 1);
  }
  __syncthreads();
}

// Sort keys: the probability's bits (p >= 0, so they order as p does) above,
// 0x7fffffff - id below: descending key order is descending probability
// with ties in ascending id; key 0 (padding past V) sorts last.
__device__ __forceinline__ uint64_t prob_key(float p, int id) {
  return ((uint64_t)__float_as_uint(p) << 32) | (uint32_t)(0x7fffffff - id);
}

// v of lane (lane ^ D), D a power of two below 64: DPP within quads, a
// swizzle within 32-lane halves, a permute across them
template <int D>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v) {
  if constexpr (D == 1)
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);
  else if constexpr (D == 2)
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);
  else if constexpr (D < 32)
    return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, (D << 10) | 0x1F);
  else
    return (uint32_t)__shfl_xor((int)v, 32, 64);
}

// Bitonic network, descending, over np2 = EPT * ST keys; thread t holds
// elements EPT t .. EPT t + EPT - 1 in registers. A compare-exchange
// (k, j) of elements i and i ^ j orders them descending when i & k == 0,
// ascending otherwise. Partners j < EPT apart are in the same thread, up to
// 64 EPT apart in the same wavefront (lane ^ j / EPT); farther ones meet
// through LDS (kb, element e of thread t at e * ST + t).
template <int EPT, int J>
__device__ __forceinline__ void cx_regs(uint64_t (&key)[EPT], int k) {
  if constexpr (J < EPT) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      if (e & J) continue;
      const uint64_t a = key[e], b = key[e | J];
      const bool sw = ((EPT * tid + e) & k) == 0 ? a < b : a > b;
      key[e] = sw ? b : a;
      key[e | J] = sw ? a : b;
    }
  }
}

template <int EPT, int D>
__device__ __forceinline__ void cx_lanes(uint64_t (&key)[EPT], int k) {
  const int tid = threadIdx.x;
  const bool lower = (tid & D) == 0;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const uint32_t lo = lane_xor<D>((uint32_t)key[e]);
    const uint32_t hi = lane_xor<D>((uint32_t)(key[e] >> 32));
    const uint64_t other = ((uint64_t)hi << 32) | lo;
    const bool keep_max = lower == (((EPT * tid + e) & k) == 0);
    key[e] = (key[e] > other) == keep_max ? key[e] : other;
  }
}

template <int EPT>
__device__ __forceinline__ void cx_lds(uint64_t (&key)[EPT], uint64_t* kb, int k, int j) {
  const int tid = threadIdx.x, dt = j / EPT;  // partner thread tid ^ dt
#pragma unroll
  for (int e = 0; e < EPT; ++e) kb[e * ST + tid] = key[e];
  __syncthreads();
  uint64_t other[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) other[e] = kb[e * ST + (tid ^ dt)];
  __syncthreads();
  const bool lower = (tid & dt) == 0;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const bool keep_max = lower == (((EPT * tid + e) & k) == 0);
    key[e] = (key[e] > other[e]) == keep_max ? key[e] : other[e];
  }
}

template <int EPT>
__device__ void bitonic_desc(uint64_t (&key)[EPT], uint64_t* kb) {
  constexpr int NP2 = EPT * ST;
#pragma unroll
  for (int k = 2; k <= NP2; k <<= 1)
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j >= 64 * EPT) {
        cx_lds<EPT>(key, kb, k, j);
      } else if (j >= EPT) {
        switch (j / EPT) {
          case 1: cx_lanes<EPT, 1>(key, k); break;
          case 2: cx_lanes<EPT, 2>(key, k); break;
          case 4: cx_lanes<EPT, 4>(key, k); break;
          case 8: cx_lanes<EPT, 8>(key, k); break;
          case 16: cx_lanes<EPT, 16>(key, k); break;
          default: cx_lanes<EPT, 32>(key, k); break;
        }
      } else {
        switch (j) {
          case 1: cx_regs<EPT, 1>(key, k); break;
          case 2: cx_regs<EPT, 2>(key, k); break;
          default: cx_regs<EPT, 4>(key, k); break;
        }
      }
    }
}

// pr[0:V) / s sorted descending (ties by id) into pr (probabilities) and ox
// (ids), np2 = EPT * ST entries, the tail past V padding; pr and the aux
// array after it serve as the LDS exchange buffer meanwhile
template <int EPT>
__device__ void sort_probs(float* pr, int* ox, int V, float s) {
  const int tid = threadIdx.x;
  uint64_t key[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const int i = EPT * tid + e;
    key[e] = i < V ? prob_key(pr[i] / s, i) : 0ull;
  }
  __syncthreads();
  bitonic_desc<EPT>(key, reinterpret_cast<uint64_t*>(pr));
  __syncthreads();
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const int i = EPT * tid + e;
    pr[i] = __uint_as_float((uint32_t)(key[e] >> 32));
    ox[i] = 0x7fffffff - (int)(uint32_t)key[e];
  }
  __syncthreads();
}

// The whole of sample_next for one row. LDS: pr, aux (floats) and ox (ints),
// np2 entries each (np2 = V rounded up to a power of two). Every thread of
// the workgroup calls it; the id is valid in every thread.
__device__ int sample_row(const float* __restrict__ logits, int V, int np2,
                          const int32_t* __restrict__ gen, int ngen, const SampleCfg& c,
                          int64_t* state, float* pr, float* aux, int* ox) {
#pragma clang fp contract(off)
  __shared__ float rv[NW];
  __shared__ int ri[NW];
  __shared__ float bcast;
  const int tid = threadIdx.x;
  int* cnt = (int*)aux;
  for (int i = tid; i < V; i += ST) pr[i] = logits[i];
  __syncthreads();
  // presence + frequency: once per distinct id, l - pres - freq * count
  if (c.pwin > 0) {
    if (ngen > 0) {
      const int lo = ngen - c.pwin > 0 ? ngen - c.pwin : 0;
      if (c.pres != 0.f || c.freq != 0.f) {
        count_ids(gen, lo, ngen, V, cnt);
        for (int i = tid; i < V; i += ST)
          if (cnt[i] > 0) pr[i] = (pr[i] - c.pres) - c.freq * (float)cnt[i];
        __syncthreads();
      }
      if (c.plen != 0.f && ngen < c.pwin && tid == 0)
        pr[0] = pr[0] - (c.plen * (float)(c.pwin - ngen)) / (float)c.pwin;
      __syncthreads();
    }
  } else if ((c.pres != 0.f || c.freq != 0.f) && ngen > 0) {
    count_ids(gen, 0, ngen, V, cnt);
    for (int i = tid; i < V; i += ST)
      if (cnt[i] > 0) pr[i] = (pr[i] - c.pres) - c.freq * (float)cnt[i];
    __syncthreads();
  }
  // repetition penalty over the whole history: l / theta
  if (c.rep > 1.f && ngen > 0) {
    count_ids(gen, 0, ngen, V, cnt);
    for (int i = tid; i < V; i += ST)
      if (cnt[i] > 0) pr[i] = pr[i] / c.rep;
    __syncthreads();
  }
  // no-repeat n-gram: ids that would complete an n-gram seen in history
  const int nn = c.nblock;
  if (nn >= 2 && ngen >= nn) {
    for (int s = tid; s <= ngen - nn; s += ST) {
      int k = 0;
      while (k < nn - 1 && gen[s + k] == gen[ngen - nn + 1 + k]) ++k;
      if (k == nn - 1) {
        const int t = gen[s + nn - 1];
        if (t >= 0 && t < V) pr[t] = -FLT_MAX;
      }
    }
    __syncthreads();
  }
  if (c.byte_space) {
    for (int i = tid; i < V; i += ST)
      if (!(i < 128 || (i >= 256 && i < 512))) pr[i] = -FLT_MAX;
    __syncthreads();
  }
  if (c.temp <= 0.f) return block_argmax(pr, V, rv, ri);

  // temperature softmax
  const float t = c.temp < 1.0e-6f ? 1.0e-6f : c.temp;
  const float m = block_max(pr, V, rv);
  float part = 0.f;
  for (int i = tid; i < V; i += ST) {
    const float e = expf((pr[i] - m) / t);
    pr[i] = e;
    part += e;
  }
  const float s = block_sum(part, rv);
  // descending probability, ties by id: a bitonic network with the keys in
  // registers (the row normalised on the way in)
  switch (np2 / ST) {
    case 1: sort_probs<1>(pr, ox, V, s); break;
    case 2: sort_probs<2>(pr, ox, V, s); break;
    case 4: sort_probs<4>(pr, ox, V, s); break;
    default: sort_probs<8>(pr, ox, V, s); break;
  }
  // inclusive cumulative sums of the sorted probabilities: each thread owns
  // np2/ST consecutive entries, then an in-order scan of the thread totals
  const int per = np2 / ST > 0 ? np2 / ST : 1;
  const int b0 = tid * per;
  float run = 0.f;
  for (int q = 0; q < per; ++q)
    if (b0 + q < np2) {
      run += b0 + q < V ? pr[b0 + q] : 0.f;
      aux[b0 + q] = run;
    }
  __shared__ float tot[ST];
  __shared__ float wtot[NW];
  tot[tid] = run;
  __syncthreads();
  if (tid < NW) {
    float a = 0.f;
    for (int q = 0; q < 64; ++q) {
      a += tot[tid * 64 + q];
      tot[tid * 64 + q] = a;
    }
    wtot[tid] = a;
  }
  __syncthreads();
  if (tid == 0) {
    float a = 0.f;
    for (int q = 0; q < NW; ++q) {
      const float w = wtot[q];
      wtot[q] = a;
      a += w;
    }
  }
  __syncthreads();
  const float off = wtot[tid >> 6] + ((tid & 63) ? tot[tid - 1] : 0.f);
  for (int q = 0; q < per; ++q)
    if (b0 + q < np2) aux[b0 + q] += off;
  __syncthreads();
  // the nucleus: the first prefix whose mass reaches topp (all of V at >= 1)
  int cut = V;
  if (c.topp < 1.f) {
    int first = 0x7fffffff;
    for (int i = tid; i < V; i += ST)
      if (aux[i] >= c.topp && i < first) first = i;
    first = block_min(first, ri);
    cut = first < V ? first + 1 : V;
  }
  if (tid == 0) bcast = rand_u01(state) * aux[cut - 1];
  __syncthreads();
  const float u = bcast;
  int hit = 0x7fffffff;
  for (int i = tid; i < cut; i += ST)
    if (aux[i] >= u && i < hit) hit = i;
  hit = block_min(hit, ri);
  return ox[hit < cut ? hit : cut - 1];
}

}  // namespace

int sample_np2(int V) {
  int n = 1;
  while (n < V) n <<= 1;
  return n < ST ? ST : n;
}

int64_t sample_lds_bytes(int V) { return (int64_t)sample_np2(V) * 12; }

// One row: the id to out[0], the state advanced in place.
__global__ __launch_bounds__(ST) void k_sample_one(const float* __restrict__ logits, int V,
                                                   int np2, const int32_t* __restrict__ gen,
                                                   int ngen, SampleCfg c, int64_t* state,
                                                   int32_t* out) {
  extern __shared__ float lds[];
  __shared__ int64_t st;
  if (threadIdx.x == 0) st = *state;
  __syncthreads();
  const int id = sample_row(logits, V, np2, gen, ngen, c, &st, lds, lds + np2,
                            (int*)(lds + 2 * np2));
  if (threadIdx.x == 0) {
    out[0] = id;
    *state = st;
  }
}

// One step of the device sampling loop: the id for position pp from the
// logits of the pass just run, history = ids[n_known:pp].
__global__ __launch_bounds__(ST) void k_sample_step(SampleDev* __restrict__ sd,
                                                    const float* __restrict__ logits, int V,
                                                    int np2, int32_t* __restrict__ ids) {
  extern __shared__ float lds[];
  __shared__ int64_t st;
  const int pp = sd->pp;
  if (pp >= sd->n_total) return;
  if (threadIdx.x == 0) st = sd->rng;
  __syncthreads();
  const int id = sample_row(logits, V, np2, ids + sd->n_known, pp - sd->n_known, sd->cfg, &st,
                            lds, lds + np2, (int*)(lds + 2 * np2));
  if (threadIdx.x == 0) {
    ids[pp] = id;
    sd->inp[0] = id;
    sd->rng = st;
    sd->pp = pp + 1;
    sd->len = pp;
  }
}

static void raise_lds(const void* k, int64_t bytes) {
  if (bytes > 64 * 1024)
    (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

void launch_sample_one(hipStream_t s, const float* logits, int V, const int32_t* gen, int ngen,
                       const SampleCfg& c, int64_t* state, int32_t* out) {
  const int np2 = sample_np2(V);
  const int64_t lds = sample_lds_bytes(V);
  raise_lds((const void*)k_sample_one, lds);
  FG_LAUNCH(k_sample_one, dim3(1), dim3(ST), (unsigned)lds, s, logits, V, np2, gen, ngen,
                     c, state, out);
}

void launch_sample_step(hipStream_t s, SampleDev* sd, const float* logits, int V, int32_t* ids) {
  const int np2 = sample_np2(V);
  const int64_t lds = sample_lds_bytes(V);
  raise_lds((const void*)k_sample_step, lds);
  FG_LAUNCH(k_sample_step, dim3(1), dim3(ST), (unsigned)lds, s, sd, logits, V, np2, ids);
}

}  // namespace fgpt
