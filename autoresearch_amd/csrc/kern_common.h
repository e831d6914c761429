// kern_common.h -- device helpers shared by the gfx950 kernels.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fgpt {

// FG_LAUNCH: a kernel launch that carries the open timed region's events
// (LaunchEvents, fgpt_internal.h) in its dispatch packet when there is one.
#define FG_LAUNCH(kernel, grid, block, shmem, stream, ...)                                    \
  do {                                                                                        \
    ::fgpt::LaunchEvents& fg_ev_ = ::fgpt::launch_events();                                   \
    if (fg_ev_.stop) {                                                                        \
      hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)(shmem), stream,                   \
                            fg_ev_.n == 0 ? fg_ev_.start : nullptr, fg_ev_.stop, 0u,          \
                            __VA_ARGS__);                                                     \
      ++fg_ev_.n;                                                                             \
    } else {                                                                                  \
      hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);                    \
    }                                                                                         \
  } while (0)

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

// fp32 -> bf16 bits, round to nearest even: gfx950's v_cvt_pk_bf16_f32
// (one instruction for two values where the compiler pairs them; the same
// bits as adding 0x7fff + the kept lsb and truncating, for finite inputs).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// fp16 bits of v, round to nearest even (v_cvt_f16_f32).
__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Unpack 8 bf16 held in a uint4 (little-endian pairs) to floats.
__device__ __forceinline__ void unpack8(const uint4 v, float* f) {
  f[0] = __uint_as_float(v.x << 16);
  f[1] = __uint_as_float(v.x & 0xFFFF0000u);
  f[2] = __uint_as_float(v.y << 16);
  f[3] = __uint_as_float(v.y & 0xFFFF0000u);
  f[4] = __uint_as_float(v.z << 16);
  f[5] = __uint_as_float(v.z & 0xFFFF0000u);
  f[6] = __uint_as_float(v.w << 16);
  f[7] = __uint_as_float(v.w & 0xFFFF0000u);
}

// Workgroup barrier for LDS traffic only: waits for this wave's LDS
// operations (lgkmcnt) but, unlike __syncthreads(), not for its outstanding
// global loads, so prefetches issued before it stay in flight.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// 16 bytes per lane, memory -> LDS at m0 + 16*lane (the wavefront's 1 KB
// block starting at LDS byte offset `lds`, which must be wave-uniform).
// Issued from asm so that the compiler, which cannot tell which buffer a
// DMA fills, does not drain every load in flight before each LDS read; the
// kernels order them with stage_sync().
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds)
               : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_off(const void* p) {
  return (uint32_t)(size_t)(const __attribute__((address_space(3))) void*)p;
}

// Stage hand-over for DMA-filled LDS buffers: this wavefront's loads older
// than the newest N have landed, and its own LDS reads have returned
// (lgkmcnt(0): the compiler may sink the MFMAs that use them below this
// point, and a buffer is refilled by another wavefront right after the
// barrier); then the workgroup barrier.
template <int N>
__device__ __forceinline__ void stage_sync() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// v from the lane that a DPP pattern names (all lanes are valid sources).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum across the 64 lanes of a wavefront (result valid in every lane): the
// butterfly over lane strides 1, 2, 4, 8, 16, 32. Strides 1 and 2 are quad
// permutes; once quads (then groups of 8) hold equal values, the half-row
// and row mirrors pair the same values that strides 4 and 8 would; once
// rows of 16 are uniform, strides 16 and 32 are (row0 + row1) + (row2 +
// row3) from four lane reads. All VALU/DPP: no LDS-crossbar permutes.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  v += dpp_f<0x140>(v);  // row_mirror
  const int iv = __builtin_bit_cast(int, v);
  const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0));
  const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16));
  const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32));
  const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48));
  return (a + b) + (c + d);
}

// Sum across each half-wavefront (lanes 0-31 and 32-63 separately), in
// wave_sum's pattern: rows of 16 lanes by DPP, then (row0 + row1) and
// (row2 + row3).
__device__ __forceinline__ float half_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  const int iv = __builtin_bit_cast(int, v);
  const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0));
  const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16));
  const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32));
  const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48));
  return (threadIdx.x & 32) ? c + d : a + b;
}

// Maximum across each half-wavefront, in half_sum's pattern.
__device__ __forceinline__ float half_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  const int iv = __builtin_bit_cast(int, v);
  const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0));
  const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16));
  const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32));
  const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48));
  return (threadIdx.x & 32) ? fmaxf(c, d) : fmaxf(a, b);
}

// Maximum across the 64 lanes, in wave_sum's pattern.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  const int iv = __builtin_bit_cast(int, v);
  const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0));
  const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16));
  const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32));
  const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

}  // namespace fgpt
