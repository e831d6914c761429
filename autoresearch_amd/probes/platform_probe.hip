// platform_probe.hip -- measurements of the MI355X platform the engine's
// design rests on (no engine code; standalone, one GPU):
//
//   clock    shader clock (s_memtime against the 100 MHz s_memrealtime) of
//            one wavefront and of the whole chip under a dependent
//            v_mfma_f32_32x32x16_f16 loop, and the MFMA rate reached
//   launch   back-to-back cost of an empty kernel, and of a kernel that
//            writes N MB followed by one that reads them back
//   streams  one grid of busy workgroups, two on one stream, two on two
//            streams (does a second HIP stream overlap kernels?)
//
//   platform_probe [clock|launch|streams]...   (no argument: all three)
//
// Every loop has a fixed trip count; every kernel touches only its own
// buffers.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>

#define CK(x)                                                                    \
  do {                                                                           \
    hipError_t e_ = (x);                                                         \
    if (e_ != hipSuccess) {                                                      \
      fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
      exit(1);                                                                   \
    }                                                                            \
  } while (0)

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// iters steps of either 4 dependent fp16 MFMAs or one dependent fp32 FMA;
// block 0's first lane reports the elapsed shader and constant-clock ticks
__global__ void k_clock(long long* out, int iters, int mfma) {
  const long long c0 = clock64(), w0 = wall_clock64();
  f32x16_t acc = {};
  f16x8_t a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = (_Float16)(threadIdx.x * 0.001f);
    b[i] = (_Float16)0.5f;
  }
  float x = threadIdx.x;
  for (int i = 0; i < iters; ++i) {
    if (mfma) {
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
    } else {
      x = x * 1.0001f + 0.5f;
    }
  }
  const long long c1 = clock64(), w1 = wall_clock64();
  float s = x;
  for (int r = 0; r < 16; ++r) s += acc[r];
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    out[0] = c1 - c0;
    out[1] = w1 - w0;
    out[2] = (long long)s;  // keeps the loop's result live
  }
}

__global__ void k_empty(float* p) {
  if (p && threadIdx.x == 0 && blockIdx.x == 0) p[0] = 1.f;
}

__global__ void k_write(float4* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    p[i] = make_float4(i, i, i, i);
}

__global__ void k_read(const float4* p, int n, float* out) {
  float s = 0.f;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    s += p[i].x;
  if (s == 12345.f) out[0] = s;  // never true for the values k_write stores
}

// iters dependent FMAs per thread, then one LDS round trip
__global__ void k_busy(float* out, int iters) {
  extern __shared__ float sm[];
  float x = threadIdx.x;
  for (int i = 0; i < iters; ++i) x = x * 1.0001f + 0.5f;
  sm[threadIdx.x] = x;
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = sm[5];
}

static hipEvent_t e0, e1;

static float elapsed_ms() {
  float ms = 0.f;
  CK(hipEventSynchronize(e1));
  CK(hipEventElapsedTime(&ms, e0, e1));
  return ms;
}

static void probe_clock() {
  long long* d = nullptr;
  CK(hipMalloc(&d, 64));
  struct Case {
    int blocks, threads, iters, mfma;
    const char* name;
  } cs[] = {{1, 64, 2000000, 0, "1 wavefront, fp32 FMA chain"},
            {1, 64, 200000, 1, "1 wavefront, MFMA chain"},
            {1024, 256, 200000, 1, "4 wavefronts per SIMD, MFMA"},
            {2048, 512, 100000, 1, "16 wavefronts per SIMD, MFMA"}};
  for (const Case& c : cs) {
    for (int rep = 0; rep < 2; ++rep) {
      CK(hipEventRecord(e0, 0));
      hipLaunchKernelGGL(k_clock, dim3(c.blocks), dim3(c.threads), 0, 0, d, c.iters, c.mfma);
      CK(hipGetLastError());
      CK(hipEventRecord(e1, 0));
      const float ms = elapsed_ms();
      long long h[3];
      CK(hipMemcpy(h, d, sizeof h, hipMemcpyDeviceToHost));
      const double ghz = (double)h[0] / ((double)h[1] / 100e6) / 1e9;
      printf("clock   %-30s rep %d: %8.3f ms, shader clock %.3f GHz", c.name, rep, ms, ghz);
      if (c.mfma) {
        const double flop = 4.0 * c.iters * 32768.0 * (c.threads / 64) * c.blocks;
        printf(", %.0f TFLOP/s", flop / (ms * 1e-3) / 1e12);
      }
      printf("\n");
    }
  }
  CK(hipFree(d));
}

template <class F>
static float per_launch_us(F f, int n) {
  for (int i = 0; i < 10; ++i) f();
  CK(hipDeviceSynchronize());
  CK(hipEventRecord(e0, 0));
  for (int i = 0; i < n; ++i) f();
  CK(hipEventRecord(e1, 0));
  return elapsed_ms() * 1000.f / n;
}

static void probe_launch() {
  float4* d = nullptr;
  float* o = nullptr;
  CK(hipMalloc(&d, 64 << 20));
  CK(hipMalloc(&o, 64));
  printf("launch  empty kernel, 1 workgroup:          %.2f us each\n",
         per_launch_us([&] { hipLaunchKernelGGL(k_empty, dim3(1), dim3(64), 0, 0, (float*)nullptr); }, 1000));
  printf("launch  empty kernel, 256 x 512 threads:    %.2f us each\n",
         per_launch_us([&] { hipLaunchKernelGGL(k_empty, dim3(256), dim3(512), 0, 0, (float*)nullptr); }, 1000));
  printf("launch  empty kernel, 2048 x 256 threads:   %.2f us each\n",
         per_launch_us([&] { hipLaunchKernelGGL(k_empty, dim3(2048), dim3(256), 0, 0, (float*)nullptr); }, 1000));
  for (int mb : {1, 4, 16, 32}) {
    const int n = mb * (1 << 20) / 16;
    const float w = per_launch_us([&] { hipLaunchKernelGGL(k_write, dim3(1024), dim3(256), 0, 0, d, n); }, 500);
    const float wr = per_launch_us([&] {
      hipLaunchKernelGGL(k_write, dim3(1024), dim3(256), 0, 0, d, n);
      hipLaunchKernelGGL(k_read, dim3(1024), dim3(256), 0, 0, (const float4*)d, n, o);
    }, 500);
    printf("launch  write %2d MB: %.2f us; write then read back: %.2f us\n", mb, w, wr);
  }
  CK(hipGetLastError());
  CK(hipFree(d));
  CK(hipFree(o));
}

static void probe_streams() {
  float* d = nullptr;
  CK(hipMalloc(&d, 1 << 20));
  hipStream_t s[2];
  CK(hipStreamCreateWithFlags(&s[0], hipStreamNonBlocking));
  CK(hipStreamCreateWithFlags(&s[1], hipStreamNonBlocking));
  CK(hipFuncSetAttribute((const void*)k_busy, hipFuncAttributeMaxDynamicSharedMemorySize,
                         96 * 1024));
  for (int lds : {0, 65536}) {
    for (int blocks : {64, 128, 256}) {
      const int it = 200000;
      auto run = [&](int mode) {  // 0: one grid, 1: two on one stream, 2: one on each stream
        CK(hipDeviceSynchronize());
        CK(hipEventRecord(e0, 0));
        CK(hipStreamWaitEvent(s[0], e0, 0));
        CK(hipStreamWaitEvent(s[1], e0, 0));
        hipLaunchKernelGGL(k_busy, dim3(blocks), dim3(512), lds, s[0], d, it);
        if (mode == 1) hipLaunchKernelGGL(k_busy, dim3(blocks), dim3(512), lds, s[0], d, it);
        if (mode == 2) hipLaunchKernelGGL(k_busy, dim3(blocks), dim3(512), lds, s[1], d, it);
        CK(hipGetLastError());
        CK(hipDeviceSynchronize());
        CK(hipEventRecord(e1, 0));
        return elapsed_ms();
      };
      run(0);
      const float one = run(0), serial = run(1), two = run(2);
      printf("streams %3d workgroups of 512 threads, %5d B LDS: one grid %.3f ms, two on one "
             "stream %.3f ms, one on each of two streams %.3f ms\n",
             blocks, lds, one, serial, two);
    }
  }
  CK(hipStreamDestroy(s[0]));
  CK(hipStreamDestroy(s[1]));
  CK(hipFree(d));
}

int main(int argc, char** argv) {
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));
  bool any = false;
  for (int i = 1; i < argc; ++i) {
    any = true;
    if (!strcmp(argv[i], "clock")) probe_clock();
    else if (!strcmp(argv[i], "launch")) probe_launch();
    else if (!strcmp(argv[i], "streams")) probe_streams();
    else {
      fprintf(stderr, "usage: %s [clock|launch|streams]...\n", argv[0]);
      return 2;
    }
  }
  if (!any) {
    probe_clock();
    probe_launch();
    probe_streams();
  }
  return 0;
}
