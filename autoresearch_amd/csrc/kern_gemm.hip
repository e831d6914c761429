// kern_gemm.hip -- bf16 MFMA GEMM for prefill and batched decode (gfx950).
//
// C[M][N] = epi( s_m * (A[M][K] . W[N][K]^T) ), the y = x W^T of
// linear3d_sgemm (src/lib/fortran_blas.f90:39-57) with rmsnorm0's row scale
// s_m = 1/sqrt(mean(A_m^2) + eps) (src/lib/fortran_rmsnorm.f90:40-60) applied
// to the output rows when `norm` is set (rmsnorm is a per-row scale, so
// norm(x) W^T = s * (x W^T)).
//
// Precision: W is bf16 and exact (the weights are bf16-representable). A is
// an fp32 activation carried as two bf16 terms, A = hi + lo with
// hi = bf16(A), lo = bf16(A - hi), written in that form once by the kernel
// that produced it; both terms go through v_mfma_f32_32x32x16_bf16 with
// fp32 accumulation, so each product carries ~16 mantissa bits of A instead
// of 8. A single bf16 term moves depth-12 logits by ~3e-3 of max|logit|,
// more than the 2e-3 parity bound; the split keeps it ~5e-6. The row norm
// comes from per-row sums of squares of the fp32 values, also written by
// the producer (one partial per producer N tile, summed here in order).
//
// Pipeline: NST stages of BK-wide K slices (BK = 32, 64 or 128) in LDS,
// filled by global_load_lds_dwordx4 (memory -> LDS without registers),
// NST-1 slices in flight while the MFMAs consume the oldest. Each LDS row
// holds its 16-byte chunks XOR-swizzled by row so the MFMA operand reads
// (32 rows x one chunk per half-wavefront) do not collide in banks.
// Tiling: BM x BN per block of NWM x NWN 64-wide wavefronts, each owning
// (BM/NWM) x (BN/NWN) as 32x32 MFMA blocks, times KG groups of such
// wavefronts that split each slice's K steps between them. The epilogue is
// staged through LDS 64 rows at a time so each thread owns a column pair
// (coalesced stores; a QKV rotation pair in one thread). The host picks the
// tile per shape (launch_tile) so that one round of tiles covers the CUs.
#include "fgpt_internal.h"
#include "kern_common.h"
#include "kern_epi.h"

namespace fgpt {
// Epilogue outputs written streaming (no cache allocation): the ReLU^2 planes
// and the residual (fp32 and planes) are read only by later kernels, from
// other XCDs' L2 mostly, and are too large to stay cached for them (25 MB
// for fc at T=2048); measured ~2.5 us faster per fc and ~0.7 us per residual
// GEMM. QKV's scattered q/k/v stores gained nothing.
constexpr bool NT_RELU2 = true, NT_RESID = true, NT_QKV = false;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// One 32x32x16 MFMA step: bf16 operands, or (P16) fp16 ones.
template <bool P16>
__device__ __forceinline__ f32x16_t mma16(const bf16x8_t& a, const bf16x8_t& b, const f32x16_t& c) {
  if constexpr (P16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

namespace {

// 16-byte chunk slot of logical chunk c in row r of a stage whose rows hold
// BK bf16 (BK/8 chunks). gfx950's LDS has 64 banks (256 bytes a cycle), and
// a 16-byte read is served 16 lanes at a time: the 16 rows an MFMA operand
// read touches at one logical chunk must land on 16 different 16-byte bank
// groups. 128 / BK rows fill 256 bytes, so the XOR pattern changes every
// 128 / BK rows (every 4 rows of 64 bytes, every 2 rows of 128 bytes).
template <int BK>
__device__ __forceinline__ int swz(int r, int c) {
  constexpr int S = BK == 32 ? 2 : BK == 64 ? 1 : 0;
  static_assert(BK == 32 || BK == 64 || BK == 128, "stage row width");
  return c ^ ((r >> S) & (BK / 8 - 1));
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// One 64-row pass of the QKV epilogue from the staged tile (fp32 [64][SSTR],
// rows m0 + 64 q ..): q/k/v columns in items of four rotation pairs of one
// row (one wide store per plane and four dims); for tiles holding v columns
// that go to the transposed layout, items of one pair over four consecutive
// rows (positions), so v^T gets one wide store per dim. Rows that do not
// form an aligned run of four positions of one sequence take the per-pair
// path. Every item's RoPE coefficients are loaded before any item stores.
template <int BN, int NT, bool P16>
__device__ __forceinline__ void qkv_tile_pass(const GemvArgs& a, const float* stage,
                                              const float* sinv, int m0, int n0, int q,
                                              bool rows_fast, int pos0) {
  constexpr int SSTR = BN + 4, NI = 8 * BN / NT;  // items per thread (64 * BN / 8 in all)
  static_assert(NI * NT == 8 * BN, "epilogue items / block size mismatch");
  const int tid = threadIdx.x, M = a.M, hd = a.hd, qdk = (a.H + a.KH) * hd;
  if (!rows_fast) {
    float4 c4[NI], s4[NI];
#pragma unroll
    for (int k = 0; k < NI; ++k) {
      const int e = tid + k * NT, srow = e / (BN / 8), pc = 8 * (e % (BN / 8));
      const int m = m0 + q * 64 + srow, n = n0 + pc;
      c4[k] = s4[k] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (m < M && n < qdk) {
        const int base = n < a.H * hd ? n : n - a.H * hd;
        const int64_t at = (int64_t)(pos0 + m % a.T) * (hd / 2) + ((base % hd) >> 1);
        c4[k] = *reinterpret_cast<const float4*>(a.cosb + at);
        s4[k] = *reinterpret_cast<const float4*>(a.sinb + at);
      }
    }
#pragma unroll
    for (int k = 0; k < NI; ++k) {
      const int e = tid + k * NT, srow = e / (BN / 8), pc = 8 * (e % (BN / 8));
      const int ml = q * 64 + srow, m = m0 + ml;
      if (m >= M) continue;
      const float4 lo = *reinterpret_cast<const float4*>(stage + srow * SSTR + pc);
      const float4 hi = *reinterpret_cast<const float4*>(stage + srow * SSTR + pc + 4);
      const float sc = a.norm ? sinv[ml] : 1.f;
      const float x[8] = {lo.x * sc, lo.y * sc, lo.z * sc, lo.w * sc,
                          hi.x * sc, hi.y * sc, hi.z * sc, hi.w * sc};
      qkv_quad_store<NT_QKV, P16>(a, m, pos0, n0 + pc, x, c4[k], s4[k]);
    }
    return;
  }
#pragma unroll
  for (int k = 0; k < NI; ++k) {
    const int e = tid + k * NT, g = e % 16, pc = 2 * (e / 16);
    const int r0 = 4 * g, n = n0 + pc, mb = m0 + q * 64 + r0;
    float x1[4], x2[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float sc = a.norm ? sinv[q * 64 + r0 + i] : 1.f;
      x1[i] = stage[(r0 + i) * SSTR + pc] * sc;
      x2[i] = stage[(r0 + i) * SSTR + pc + 1] * sc;
    }
    const int t0 = mb % a.T, pos = pos0 + t0;
    const bool run4 = n >= qdk && a.vt && mb + 3 < M && t0 + 3 < a.T && (pos & 3) == 0;
    if (run4) {
      const int base = n - qdk, head = base / hd, j = (base % hd) >> 1, b = mb / a.T;
      uint16_t* p = a.vt + ((int64_t)b * a.KH + head) * hd * a.npos + pos;
      if (a.kv16) {  // the planes carry what the bf16 cache holds
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x1[i] = kv_val(a, x1[i]);
          x2[i] = kv_val(a, x2[i]);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f16_guard<P16>(a, x1[i]);
        f16_guard<P16>(a, x2[i]);
      }
      put4<P16, NT_QKV>(x1, p + (int64_t)j * a.npos, a.kv_plane);
      put4<P16, NT_QKV>(x2, p + (int64_t)(j + hd / 2) * a.npos, a.kv_plane);
      if (a.vc) {
        const int kd = a.KH * hd;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t v = ((int64_t)b * a.maxT + pos + i) * kd + head * hd;
          kv_put(a, a.vc, v + j, x1[i]);
          kv_put(a, a.vc, v + j + hd / 2, x2[i]);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (mb + i < M) qkv_pair_epilogue<P16>(a, mb + i, pos0, n, x1[i], x2[i]);
    }
  }
}

// KG > 1 splits each stage's 16-deep K steps over KG groups of NWM x NWN
// wavefronts (group g takes steps g, g + KG, ..): a tile too small to give
// every SIMD two wavefronts of its own still keeps them all busy. The
// groups' partial sums meet in the LDS staging buffer in a fixed order
// (KG - 1 first, 0 last), so the result does not depend on timing.
template <int EPI, int BM, int BN, int NWM, int NWN, int BK, int NST, int KG = 1, bool P16 = false>
__global__ __launch_bounds__(64 * NWM * NWN * KG) void k_gemm(GemvArgs a,
                                                             const int32_t* __restrict__ d_pos) {
  constexpr int NWT = NWM * NWN, NW = NWT * KG, NT = 64 * NW;
  constexpr int WM = BM / (32 * NWM), WN = BN / (32 * NWN);  // 32x32 blocks per wave
  // a stage: A hi rows, A lo rows, W rows of RB bytes each, loaded 1 KB
  // (1024 / RB rows) per wavefront instruction
  constexpr int RB = 2 * BK, CPR = BK / 8, RPG = 1024 / RB;
  constexpr int AP = P16 ? 1 : 2;  // operand planes of A (hi and lo, or one fp16)
  constexpr int ROWS = AP * BM + BN;
  constexpr int GROUPS = ROWS / RPG;         // 1 KB load groups per stage
  // groups per wavefront per stage; when NW does not divide GROUPS, the
  // spare slots repeat the last group (the same bytes to the same place)
  constexpr int GPW = (GROUPS + NW - 1) / NW;
  static_assert(ROWS % RPG == 0 && WM >= 1 && WN >= 1, "tile / wave grid mismatch");
  static_assert(KG == 1 || (BM == 64 && (BK / 16) % KG == 0), "K groups: one 64-row pass");
  constexpr int STAGE_BYTES = ROWS * RB;
  constexpr int SSTR = BN + 4;  // epilogue staging row stride (floats)
  // NST stages of STAGE_BYTES; after the K loop the same memory (sized for
  // the larger of the two) stages the epilogue (the DMA is issued from asm, so the compiler never waits on it
  // for an LDS read: the stage_sync() calls order them)
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  float* stage = reinterpret_cast<float*>(smem);
  __shared__ float sinv[BM];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int kg = wid / NWT, wm = (wid % NWT) / NWN, wn = wid % NWN;
  // Blocks go to the 8 XCDs round-robin by linear id. Remap so that XCD x
  // runs a contiguous run of tiles in row-major order: tiles sharing an A
  // row-block (and the weight panel sweep) stay in one XCD's L2.
  const int nbn = gridDim.x, ntile = gridDim.x * gridDim.y;
  int lin = blockIdx.x + nbn * blockIdx.y;
  if ((ntile & 7) == 0) lin = (lin & 7) * (ntile >> 3) + (lin >> 3);
  const int m0 = (lin / nbn) * BM, n0 = (lin % nbn) * BN;
  const int M = a.M, K = a.K;
  // split-K (a.part set): this block sums K range [kz*klen, kz*klen + klen)
  const int kz = blockIdx.z, klen = K / (int)gridDim.z, kbeg = kz * klen;

  // This lane's source rows for each of its load groups (fixed for the whole
  // K loop): group g covers stage rows RPG*g .. RPG*g+RPG-1; lane -> row
  // RPG*g + l/CPR, LDS slot l%CPR, which holds logical chunk swz(row, slot).
  const uint16_t* src[GPW];
#pragma unroll
  for (int q = 0; q < GPW; ++q) {
    const int g = min(wid + NW * q, GROUPS - 1);
    const int r = RPG * g + lane / CPR, slot = lane % CPR;
    const int c = swz<BK>(r, slot);
    if (r < AP * BM) {  // A hi (r < BM) or A lo
      const int ar = r < BM ? r : r - BM;
      const int row = min(m0 + ar, M - 1);  // rows past M are never stored
      src[q] = a.xs + (r < BM ? 0 : a.xs_plane) + (int64_t)row * K + kbeg + c * 8;
    } else {
      src[q] = a.w + (int64_t)(n0 + r - AP * BM) * K + kbeg + c * 8;
    }
  }

  // epilogue items (column pairs of a 64-row pass) per thread
  constexpr int EPT = 64 * (BN / 2) / NT;
  static_assert(EPT * NT == 64 * (BN / 2), "epilogue pass / block size mismatch");
  // RESID row sums of squares: within the wavefront when a row's BN / 2
  // column pairs are exactly one wavefront (BN = 128) or half of one
  // (BN = 64), else through LDS (sqs, a padded [64][BN / 2] after the
  // staged tile), each row summed in column order by one thread
  constexpr bool SQ_LDS = EPI == GV_RESID && BN != 64 && BN != 128;
  constexpr int SQS = BN / 2 + 1;
  // RESID: the residual tile is read now, so its latency hides behind the
  // K loop instead of stalling the epilogue
  float2 xres[EPI == GV_RESID ? (BM / 64) * EPT : 1];
  if (EPI == GV_RESID && !a.part) {
#pragma unroll
    for (int q = 0; q < BM / 64; ++q)
#pragma unroll
      for (int k = 0; k < EPT; ++k) {
        const int e = tid + k * NT, m = m0 + q * 64 + e / (BN / 2);
        xres[q * EPT + k] = m < M ? *reinterpret_cast<const float2*>(
                                        a.y + (int64_t)m * a.N + n0 + 2 * (e % (BN / 2)))
                                  : make_float2(0.f, 0.f);
      }
  }

  f32x16_t acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int nk = klen / BK;  // klen % BK == 0 (checked by the host)
  const int klast = klen - BK;
  uint32_t ldsq[GPW];  // LDS byte offset of each of this wavefront's groups
#pragma unroll
  for (int q = 0; q < GPW; ++q)
    ldsq[q] = __builtin_amdgcn_readfirstlane(lds_off(smem) + min(wid + NW * q, GROUPS - 1) * 1024);
  auto fill = [&](int stg, int k0) {
#pragma unroll
    for (int q = 0; q < GPW; ++q) dma16(src[q] + k0, ldsq[q] + stg * STAGE_BYTES);
  };
  auto consume = [&](int si) {
    const uint8_t* stg = smem + si * STAGE_BYTES;
#pragma unroll
    for (int k2 = 0; k2 < BK / 16 / KG; ++k2) {
      const int kk = k2 * KG + kg;         // this group's 16-deep step of the stage
      const int c = 2 * kk + (lane >> 5);  // logical chunk of this half-wave
      bf16x8_t ah[WM], al[WM], bw[WN];
#pragma unroll
      for (int i = 0; i < WM; ++i) {
        const int r = (wm * WM + i) * 32 + (lane & 31);
        ah[i] = *(const bf16x8_t*)(stg + r * RB + swz<BK>(r, c) * 16);
        if constexpr (!P16) al[i] = *(const bf16x8_t*)(stg + (BM + r) * RB + swz<BK>(BM + r, c) * 16);
      }
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        const int r = AP * BM + (wn * WN + j) * 32 + (lane & 31);
        bw[j] = *(const bf16x8_t*)(stg + r * RB + swz<BK>(r, c) * 16);
      }
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[i][j] = mma16<P16>(ah[i], bw[j], acc[i][j]);
      if constexpr (!P16) {
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
          for (int j = 0; j < WN; ++j) acc[i][j] = mma16<false>(al[i], bw[j], acc[i][j]);
      }
    }
  };
  // prologue: slices 0 .. NST-2 in flight; then each step waits for its
  // slice and refills the stage consumed one step earlier (NST-1 slices
  // ahead; loads past the end re-read the last slice so the outstanding
  // count is fixed)
#pragma unroll
  for (int si = 0; si < NST - 1; ++si) fill(si, min(si * BK, klast));
  for (int kt = 0; kt < nk; kt += NST) {
#pragma unroll
    for (int si = 0; si < NST; ++si) {
      if (kt + si < nk) {  // uniform; only the last group can be partial
        stage_sync<(NST - 2) * GPW>();
        fill((si + NST - 1) % NST, min((kt + si + NST - 1) * BK, klast));
        consume(si);
      }
    }
  }
  wait_vmcnt<0>();
  __syncthreads();

  // row scale from the producer's partial sums of squares
  if (a.norm && !a.part) {
    for (int r = tid; r < BM; r += NT) {
      float ssum = 0.f;
      if (m0 + r < M)
        for (int t = 0; t < a.ssq_n; ++t) ssum += a.ssq_in[(int64_t)(m0 + r) * a.ssq_n + t];
      sinv[r] = 1.0f / sqrtf(ssum / (float)K + a.eps);
    }
    __syncthreads();
  }

  // epilogue through LDS, 64 tile rows (two 32-row blocks) per pass
  const int pos0 = d_pos ? *d_pos : a.pos0;
  // Tiles holding v columns that go to the transposed bf16 layout
  // ([..][hd][npos]: positions contiguous) walk the staged tile row-fastest,
  // so a wavefront's stores cover 64 consecutive positions of one dim.
  const bool rows_fast = EPI == GV_QKV && a.vt && !a.part && n0 + BN > (a.H + a.KH) * a.hd;
  float* sqs = stage + KG * 64 * SSTR;
#pragma unroll
  for (int q = 0; q < BM / 64; ++q) {
    // each K group stages its partial tile in a region of its own, all at
    // once; one pass then adds the regions in a fixed order (KG - 1 first,
    // 0 last) into region 0
    {
      float* reg = stage + kg * 64 * SSTR;
#pragma unroll
      for (int i = 0; i < WM; ++i) {
        const int rb = wm * WM + i;  // 32-row block of the tile
        if (rb / 2 != q) continue;
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
          for (int rg = 0; rg < 16; ++rg) {
            const int r = 8 * (rg >> 2) + 4 * (lane >> 5) + (rg & 3);
            // (P16: the weights were stored scaled by 1 / wscale, a power of 2)
            reg[((rb & 1) * 32 + r) * SSTR + (wn * WN + j) * 32 + (lane & 31)] =
                P16 ? acc[i][j][rg] * a.wscale : acc[i][j][rg];
          }
      }
      __syncthreads();
      if constexpr (KG > 1) {
        constexpr int NQ4 = 64 * BN / 4;  // float4s of a pass
        for (int e = tid; e < NQ4; e += NT) {
          const int o = (e / (BN / 4)) * SSTR + 4 * (e % (BN / 4));
          float4 v = *reinterpret_cast<const float4*>(stage + (KG - 1) * 64 * SSTR + o);
#pragma unroll
          for (int g = KG - 2; g >= 0; --g) {
            const float4 w = *reinterpret_cast<const float4*>(stage + g * 64 * SSTR + o);
            v.x = v.x + w.x;
            v.y = v.y + w.y;
            v.z = v.z + w.z;
            v.w = v.w + w.w;
          }
          *reinterpret_cast<float4*>(stage + o) = v;
        }
        __syncthreads();
      }
    }
    // BN/2 consecutive e cover one row; with BN = 128 that is one
    // wavefront, with BN = 64 half of one (reductions stay in the wave)
    if constexpr (EPI == GV_QKV) {
      if (!a.part) {
        qkv_tile_pass<BN, NT, P16>(a, stage, sinv, m0, n0, q, rows_fast, pos0);
        __syncthreads();
        continue;
      }
    }
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const int e = tid + k * NT;
      const int srow = rows_fast ? e % 64 : e / (BN / 2);
      const int pc = rows_fast ? 2 * (e / 64) : 2 * (e % (BN / 2));
      const int ml = q * 64 + srow;
      const int m = m0 + ml, n = n0 + pc;
      const bool live = m < M;
      float v0 = stage[srow * SSTR + pc], v1 = stage[srow * SSTR + pc + 1];
      if (a.part) {  // raw partial; the reduce kernel applies norm and epilogue
        if (live)
          *reinterpret_cast<float2*>(a.part + ((int64_t)kz * M + m) * a.N + n) = make_float2(v0, v1);
        continue;
      }
      if (a.norm) {
        v0 *= sinv[ml];
        v1 *= sinv[ml];
      }
      if (EPI == GV_QKV) {
        if (live) qkv_pair_epilogue<P16>(a, m, pos0, n, v0, v1);
      } else if (EPI == GV_RESID) {
        float2 o = make_float2(0.f, 0.f);
        float* y = a.y + (int64_t)(live ? m : 0) * a.N + n;
        if (live) {
          o = xres[q * EPT + k];
          o.x += v0;
          o.y += v1;
          store_v<NT_RESID>(reinterpret_cast<f32x2_t*>(y), f32x2_t{o.x, o.y});
          f16_guard<P16>(a, o.x);
          f16_guard<P16>(a, o.y);
          put2<P16, NT_RESID>(o.x, o.y, a.ys + (int64_t)m * a.N + n, a.ys_plane);
        }
        // the row's sum of squares over this tile
        const float sq0 = o.x * o.x + o.y * o.y;
        if constexpr (SQ_LDS) {
          sqs[srow * SQS + pc / 2] = sq0;
        } else {
          const float sq = BN == 128 ? wave_sum(sq0) : half_sum(sq0);
          if (live && pc == 0) a.ssq_out[(int64_t)m * (a.N / BN) + n0 / BN] = sq;
        }
      } else if (EPI == GV_RELU2) {
        if (live) {
          const float t0 = v0 < 0.f ? 0.f : v0, t1 = v1 < 0.f ? 0.f : v1;
          f16_guard<P16>(a, t0 * t0);
          f16_guard<P16>(a, t1 * t1);
          put2<P16, NT_RELU2>(t0 * t0, t1 * t1, a.ys + (int64_t)m * a.N + n, a.ys_plane);
        }
      } else {
        if (live) *reinterpret_cast<float2*>(a.y + (int64_t)m * a.N + n) = make_float2(v0, v1);
      }
    }
    __syncthreads();
    if constexpr (SQ_LDS) {
      // P = NT / 64 adjacent threads per row, each summing BN / 2 / P of
      // its values in column order, then a fixed butterfly over the P
      constexpr int P = NT / 64, VPP = (BN / 2) / P;
      static_assert(P * VPP == BN / 2 && (P == 2 || P == 4 || P == 8), "row-sum split");
      const int row = tid / P, part = tid % P;
      float sum = 0.f;
#pragma unroll
      for (int v = 0; v < VPP; ++v) sum += sqs[row * SQS + part * VPP + v];
      sum += dpp_f<0xB1>(sum);                          // lane ^ 1
      if constexpr (P >= 4) sum += dpp_f<0x4E>(sum);    // lane ^ 2
      if constexpr (P == 8) sum += dpp_f<0x141>(sum);   // the other quad of eight
      if (!a.part && part == 0 && m0 + q * 64 + row < M)
        a.ssq_out[(int64_t)(m0 + q * 64 + row) * (a.N / BN) + n0 / BN] = sum;
      __syncthreads();
    }
  }
}

// ------------------------------------------------------------------ v2
// Wave tile (WM x 32) x (WN x 32), K slices of BK (32 or 64) per stage. The
// operand fragments of the next 16-deep step are read from LDS into a
// second register set while the MFMAs of the current one run (the last
// step of a slice runs after the next slice's barrier), so LDS latency hides
// behind MFMA work
// even at one wavefront per SIMD. The epilogue works straight from the
// accumulators: lane l of a 32x32 block holds column l % 32 of rows
// 8(r/4) + 4(l/32) + r%4, r = 0..15, so 32 lanes store 32 consecutive
// columns of one row.
template <int WM, int WN>
struct Frag {
  bf16x8_t h[WM], l[WM], w[WN];
};

template <int BM, int WM, int WN, bool P16, int BK = 32>
__device__ __forceinline__ void frag_load(Frag<WM, WN>& f, const uint8_t* stg, int kk, int wm,
                                          int wn, int lane) {
  constexpr int AP = P16 ? 1 : 2;
  const int c = 2 * kk + (lane >> 5);  // logical chunk of this half-wave
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    const int r = (wm * WM + i) * 32 + (lane & 31);
    f.h[i] = *(const bf16x8_t*)(stg + r * (2 * BK) + swz<BK>(r, c) * 16);
    if constexpr (!P16) f.l[i] = *(const bf16x8_t*)(stg + (BM + r) * (2 * BK) + swz<BK>(BM + r, c) * 16);
  }
#pragma unroll
  for (int j = 0; j < WN; ++j) {
    const int r = AP * BM + (wn * WN + j) * 32 + (lane & 31);
    f.w[j] = *(const bf16x8_t*)(stg + r * (2 * BK) + swz<BK>(r, c) * 16);
  }
}

template <int WM, int WN, bool P16>
__device__ __forceinline__ void frag_mma(const Frag<WM, WN>& f, f32x16_t (&acc)[WM][WN]) {
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[i][j] = mma16<P16>(f.h[i], f.w[j], acc[i][j]);
  if constexpr (!P16) {
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WN; ++j) acc[i][j] = mma16<false>(f.l[i], f.w[j], acc[i][j]);
  }
}

template <int EPI, int NWM, int NWN, int WM, int WN, int NST, bool P16 = false, int BK = 32>
__global__ __launch_bounds__(64 * NWM * NWN) void k_gemm2(GemvArgs a,
                                                         const int32_t* __restrict__ d_pos) {
  constexpr int RB = 2 * BK, CPR = BK / 8, RPG = 1024 / RB;
  constexpr int BM = NWM * WM * 32, BN = NWN * WN * 32;
  constexpr int NW = NWM * NWN, NT = 64 * NW;
  constexpr int AP = P16 ? 1 : 2;
  constexpr int ROWS = AP * BM + BN, GROUPS = ROWS / RPG, GPW = GROUPS / NW;
  static_assert(GROUPS % NW == 0, "tile / wave grid mismatch");
  constexpr int STAGE_BYTES = ROWS * RB;
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  __shared__ float sinv[BM];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid / NWN, wn = wid % NWN;
  // XCD x runs a contiguous run of tiles in row-major order (see k_gemm)
  const int nbn = gridDim.x, ntile = gridDim.x * gridDim.y;
  int lin = blockIdx.x + nbn * blockIdx.y;
  if ((ntile & 7) == 0) lin = (lin & 7) * (ntile >> 3) + (lin >> 3);
  const int m0 = (lin / nbn) * BM, n0 = (lin % nbn) * BN;
  const int M = a.M, K = a.K;

  const uint16_t* src[GPW];
#pragma unroll
  for (int q = 0; q < GPW; ++q) {
    const int g = wid + NW * q;
    const int r = RPG * g + lane / CPR, slot = lane % CPR;
    const int c = swz<BK>(r, slot);
    if (r < AP * BM) {
      const int ar = r < BM ? r : r - BM;
      const int row = min(m0 + ar, M - 1);  // rows past M are never stored
      src[q] = a.xs + (r < BM ? 0 : a.xs_plane) + (int64_t)row * K + c * 8;
    } else {
      src[q] = a.w + (int64_t)(n0 + r - AP * BM) * K + c * 8;
    }
  }

  f32x16_t acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int nk = K / BK, klast = K - BK;
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_off(smem) + wid * 1024);
  auto fill = [&](int stg, int k0) {
#pragma unroll
    for (int q = 0; q < GPW; ++q) dma16(src[q] + k0, lds0 + stg * STAGE_BYTES + NW * q * 1024);
  };
#pragma unroll
  for (int si = 0; si < NST - 1; ++si) fill(si, min(si * BK, klast));
  Frag<WM, WN> f0, f1;
  for (int kt = 0; kt < nk; kt += NST) {
#pragma unroll
    for (int si = 0; si < NST; ++si) {
      if (kt + si < nk) {
        stage_sync<(NST - 2) * GPW>();
        fill((si + NST - 1) % NST, min((kt + si + NST - 1) * BK, klast));
        const uint8_t* stg = smem + si * STAGE_BYTES;
        frag_load<BM, WM, WN, P16, BK>(f0, stg, 0, wm, wn, lane);
        if (kt + si > 0) frag_mma<WM, WN, P16>(f1, acc);  // last k-step of the previous slice
        frag_load<BM, WM, WN, P16, BK>(f1, stg, 1, wm, wn, lane);
        frag_mma<WM, WN, P16>(f0, acc);
#pragma unroll
        for (int kk = 2; kk < BK / 16; kk += 2) {
          frag_load<BM, WM, WN, P16, BK>(f0, stg, kk, wm, wn, lane);
          frag_mma<WM, WN, P16>(f1, acc);
          frag_load<BM, WM, WN, P16, BK>(f1, stg, kk + 1, wm, wn, lane);
          frag_mma<WM, WN, P16>(f0, acc);
        }
      }
    }
  }
  frag_mma<WM, WN, P16>(f1, acc);
  wait_vmcnt<0>();

  if (a.norm) {
    for (int r = tid; r < BM; r += NT) {
      float ssum = 0.f;
      if (m0 + r < M)
        for (int t = 0; t < a.ssq_n; ++t) ssum += a.ssq_in[(int64_t)(m0 + r) * a.ssq_n + t];
      sinv[r] = 1.0f / sqrtf(ssum / (float)K + a.eps);
    }
    __syncthreads();
  }

  const int pos0 = d_pos ? *d_pos : a.pos0;
  const int half = lane >> 5, cl = lane & 31;
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    const int rb = (wm * WM + i) * 32 + 4 * half;  // tile row of r = 0
    float ssq[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) ssq[r] = 0.f;
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int cb = n0 + (wn * WN + j) * 32, n = cb + cl;
      float v[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int rl = rb + 8 * (r >> 2) + (r & 3);
        const float u = P16 ? acc[i][j][r] * a.wscale : acc[i][j][r];
        v[r] = a.norm ? u * sinv[rl] : u;
      }
      if (EPI == GV_QKV) {
        const bool vblock = cb >= (a.H + a.KH) * a.hd;  // a 32-column block never straddles
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const int m = m0 + rb + 8 * rq;  // rows m .. m+3
          const int t = m % a.T;
          const int pos = pos0 + t;
          if (vblock && a.vt && !a.vc && m + 3 < M && t + 3 < a.T && (pos & 3) == 0) {
            // four consecutive positions of one dim: one 8-byte store per plane
            const int base = n - (a.H + a.KH) * a.hd;
            const int head = base / a.hd, j2 = (base % a.hd) >> 1;
            const int dim = (n & 1) ? j2 + a.hd / 2 : j2;
            const int b = m / a.T;
            uint16_t* p = a.vt + (((int64_t)b * a.KH + head) * a.hd + dim) * a.npos + pos;
            const float w4[4] = {v[4 * rq], v[4 * rq + 1], v[4 * rq + 2], v[4 * rq + 3]};
#pragma unroll
            for (int e = 0; e < 4; ++e) f16_guard<P16>(a, w4[e]);
            put4<P16>(w4, p, a.kv_plane);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float own = v[4 * rq + e];
              const float other = __shfl_xor(own, 1, 64);
              if (m + e < M) qkv_elem_epilogue<P16>(a, m + e, pos0, n, own, other);
            }
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + rb + 8 * (r >> 2) + (r & 3);
          if (m >= M) continue;
          const int64_t o = (int64_t)m * a.N + n;
          if (EPI == GV_RESID) {
            const float x = a.y[o] + v[r];
            a.y[o] = x;
            f16_guard<P16>(a, x);
            put1<P16>(x, a.ys + o, a.ys_plane);
            ssq[r] += x * x;
          } else if (EPI == GV_RELU2) {
            const float t = v[r] < 0.f ? 0.f : v[r];
            f16_guard<P16>(a, t * t);
            put1<P16>(t * t, a.ys + o, a.ys_plane);
          } else {
            __builtin_nontemporal_store(v[r], a.y + o);  // logits: read once, later
          }
        }
      }
    }
    if constexpr (EPI == GV_STORE) {
      // the cross-entropy's log-sum-exp, per row and NLL_GROUP_COLS-column
      // group (GB adjacent 32-column blocks of this wavefront): the group
      // maximum over the lane's GB values and the half-wavefront's 32 lanes,
      // then the sum of exp(v - max) (the hardware exp2 of (v - max) log2 e:
      // its relative error, a few ulp, is far below the tolerance of the
      // nll); the values are the logits just stored, bit for bit. Only
      // tilings whose wavefront row holds whole groups generate it; the
      // launcher picks one of those when nll_part is set.
      constexpr int GB = NLL_GROUP_COLS / 32;
      if constexpr (WN % GB == 0) {
        if (a.nll_part) {
          const int ng = a.N / NLL_GROUP_COLS;
#pragma unroll
          for (int q = 0; q < WN / GB; ++q) {
            const int grp = (n0 + (wn * WN + GB * q) * 32) / NLL_GROUP_COLS;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int rl = rb + 8 * (r >> 2) + (r & 3);
              float v[GB];
#pragma unroll
              for (int g = 0; g < GB; ++g) {
                const float u = P16 ? acc[i][GB * q + g][r] * a.wscale : acc[i][GB * q + g][r];
                v[g] = a.norm ? u * sinv[rl] : u;
              }
              float mx = v[0];
#pragma unroll
              for (int g = 1; g < GB; ++g) mx = fmaxf(mx, v[g]);
              mx = half_max(mx);
              float e = 0.f;
#pragma unroll
              for (int g = 0; g < GB; ++g) e += __expf(v[g] - mx);
              const float sm = half_sum(e);
              const int m = m0 + rl;
              if (cl == 0 && m < M)
                *reinterpret_cast<float2*>(a.nll_part + ((int64_t)m * ng + grp) * 2) =
                    make_float2(mx, sm);
            }
          }
        }
      }
    }
    if (EPI == GV_RESID) {
      // per-row partial over this wavefront's WN*32 columns
      const int nparts = a.N / (WN * 32), part = (n0 + wn * WN * 32) / (WN * 32);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float sq = ssq[r];
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) sq += __shfl_xor(sq, off, 64);
        const int m = m0 + rb + 8 * (r >> 2) + (r & 3);
        if (cl == 0 && m < M) a.ssq_out[(int64_t)m * nparts + part] = sq;
      }
    }
  }
}

template <int EPI, int NWM, int NWN, int WM, int WN, int NST, bool P16, int BK = 32>
void launch_cfg2(hipStream_t s, const GemvArgs& a, const int32_t* d_pos) {
  constexpr int BM = NWM * WM * 32, BN = NWN * WN * 32;
  constexpr size_t lds = (size_t)NST * ((P16 ? 1 : 2) * BM + BN) * 2 * BK;
  static_assert(lds + BM * sizeof(float) <= 160 * 1024, "tile exceeds the LDS");
  static std::atomic<uint64_t> attr{0};
  raise_lds_once((const void*)k_gemm2<EPI, NWM, NWN, WM, WN, NST, P16, BK>, lds, &attr);
  const dim3 g(a.N / BN, (unsigned)((a.M + BM - 1) / BM));
  FG_LAUNCH((k_gemm2<EPI, NWM, NWN, WM, WN, NST, P16, BK>), g, dim3(64 * NWM * NWN), lds, s, a,
                     d_pos);
}

template <int EPI, int BM, int BN, int NWM, int NWN, int BK, int NST, int KG, bool P16>
void launch_cfg(hipStream_t s, const GemvArgs& a, const int32_t* d_pos) {
  constexpr bool sq_lds = EPI == GV_RESID && BN != 64 && BN != 128;
  constexpr size_t pipe = (size_t)NST * ((P16 ? 1 : 2) * BM + BN) * 2 * BK;
  constexpr size_t epi =
      (size_t)KG * 64 * (BN + 4) * 4 + (sq_lds ? (size_t)64 * (BN / 2 + 1) * 4 : 0);
  constexpr size_t lds = pipe > epi ? pipe : epi;
  // gfx950: 160 KB of LDS per workgroup, the row scales (BM floats) included
  static_assert(lds + BM * sizeof(float) <= 160 * 1024, "tile exceeds the LDS");
  static std::atomic<uint64_t> attr{0};
  raise_lds_once((const void*)k_gemm<EPI, BM, BN, NWM, NWN, BK, NST, KG, P16>, lds, &attr);
  const dim3 g(a.N / BN, (unsigned)((a.M + BM - 1) / BM));
  FG_LAUNCH((k_gemm<EPI, BM, BN, NWM, NWN, BK, NST, KG, P16>), g, dim3(64 * NWM * NWN * KG),
                     lds, s, a, d_pos);
}

// 128 wide while that still leaves half the CUs a block (the wider tile
// reads the A panel half as often), else 64 wide
int tile_n(int64_t M, int N) {
  const int64_t mt64 = (M + 63) / 64;
  return (N % 128 == 0 && mt64 * (N / 128) >= 128) ? 128 : 64;
}

// The residual GEMMs (proj, proj2) at prefill sizes, where 64x128 tiles
// leave CUs idle and 64x96 tiles give more than half of them one each
// (M = 2048, N = 768: 256 tiles): 64x96 tiles with K split over 4
// wavefront groups, two wavefronts per SIMD (measured 2-4 us a launch
// faster than 64x128 tiles at one wavefront per SIMD).
bool resid_k4(int64_t M, int N, int K) {
  const int64_t mt64 = (M + 63) / 64, ncu = cu_count(), t96 = mt64 * (N / 96);
  return K % 64 == 0 && N % 96 == 0 && mt64 * (N / 128) < ncu && t96 <= ncu && 2 * t96 > ncu;
}

// The residual GEMMs where 64x128 tiles spill into a second round over the
// CUs and 64x160 tiles fill one (the depth-20 model's d_model 1280 at 2047
// rows: 320 tiles of 64x128, 256 of 64x160): K split over 2 wavefront
// groups of two (the staged tiles of four groups would not fit the LDS).
bool resid_160(int64_t M, int N, int K) {
  const int64_t mt64 = (M + 63) / 64, ncu = cu_count(), t160 = mt64 * (N / 160);
  return K % 64 == 0 && N % 160 == 0 && mt64 * (N / 128) > ncu && t160 <= ncu &&
         2 * t160 > ncu;
}

// Small M (batched decode, short chunks): too few output tiles to fill the
// chip, so K is split over blockIdx.z as well: 64x64 tiles, enough splits
// for ~256 blocks, each split a whole number of 32-wide slices.
constexpr int64_t SPLITK_MAX_M = 128;

int splitk_count(int64_t M, int N, int K) {
  if (M > SPLITK_MAX_M || N % 64 != 0) return 1;
  const int nb = (int)((M + 63) / 64) * (N / 64), nsl = K / 32;
  int sp = (256 + nb - 1) / nb;
  if (sp > nsl) sp = nsl;
  while (sp > 1 && nsl % sp != 0) --sp;
  return sp;
}

// Sum of the K-split partials in split order, then the row norm and the
// epilogue. Block = (row, 512 columns), a thread a column pair; the splits'
// loads go out eight at a time. RESID leaves one sum-of-squares partial per
// row and 512-column group.
constexpr int RED_COLS = 512;

template <int EPI>
__global__ __launch_bounds__(256) void k_splitk_reduce(GemvArgs a, int splits,
                                                       const int32_t* __restrict__ d_pos) {
  __shared__ float red[4];
  const int m = blockIdx.x, tid = threadIdx.x, N = a.N;
  const int n = blockIdx.y * RED_COLS + 2 * tid;
  float inv = 1.f;
  if (a.norm) {
    float ssum = 0.f;
    for (int t = 0; t < a.ssq_n; ++t) ssum += a.ssq_in[(int64_t)m * a.ssq_n + t];
    inv = 1.0f / sqrtf(ssum / (float)a.K + a.eps);
  }
  const int pos0 = d_pos ? *d_pos : a.pos0;
  float sq = 0.f;
  if (n < N) {
    float v0 = 0.f, v1 = 0.f;
    const float* P = a.part + (int64_t)m * N + n;
    const int64_t stride = (int64_t)a.M * N;
    for (int s0 = 0; s0 < splits; s0 += 8) {
      float2 p[8];
#pragma unroll
      for (int k = 0; k < 8; ++k)
        p[k] = s0 + k < splits ? *reinterpret_cast<const float2*>(P + (s0 + k) * stride)
                               : make_float2(0.f, 0.f);
#pragma unroll
      for (int k = 0; k < 8; ++k) {  // split order (a zero adds nothing)
        v0 += p[k].x;
        v1 += p[k].y;
      }
    }
    v0 *= inv;
    v1 *= inv;
    const int64_t o = (int64_t)m * N + n;
    if (EPI == GV_QKV) {
      qkv_pair_epilogue(a, m, pos0, n, v0, v1);
    } else if (EPI == GV_RESID) {
      float2 x = *reinterpret_cast<const float2*>(a.y + o);
      x.x += v0;
      x.y += v1;
      *reinterpret_cast<float2*>(a.y + o) = x;
      if (a.ys) split_bf16x2(x.x, x.y, a.ys + o, a.ys_plane);
      sq = x.x * x.x + x.y * x.y;
    } else if (EPI == GV_RELU2) {
      const float t0 = v0 < 0.f ? 0.f : v0, t1 = v1 < 0.f ? 0.f : v1;
      split_bf16x2(t0 * t0, t1 * t1, a.ys + o, a.ys_plane);
    } else {
      *reinterpret_cast<float2*>(a.y + o) = make_float2(v0, v1);
    }
  }
  if (EPI == GV_RESID && a.ssq_out) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off, 64);
    if ((tid & 63) == 0) red[tid >> 6] = sq;
    __syncthreads();
    if (tid == 0)
      a.ssq_out[(int64_t)m * gridDim.y + blockIdx.y] = red[0] + red[1] + red[2] + red[3];
  }
}

// The K-split partial sums of a small-M GEMM into a.part (64x64 tiles,
// blockIdx.z the split).
template <int EPI>
void launch_splitk_parts(hipStream_t s, const GemvArgs& a, int sp, const int32_t* d_pos) {
  constexpr size_t lds = (size_t)4 * (2 * 64 + 64) * 64;
  const dim3 g(a.N / 64, (unsigned)((a.M + 63) / 64), (unsigned)sp);
  FG_LAUNCH((k_gemm<EPI, 64, 64, 2, 2, 32, 4>), g, dim3(256), lds, s, a, d_pos);
}

// Tile choice. The LDS-staged epilogue (k_gemm) serves QKV and RESID,
// whose outputs are scattered or need per-row reductions; the register
// epilogue (k_gemm2) serves the plain stores of RELU2 and lm_head, with
// 128x256 tiles (wave 64x128) when there are >= 1.5 blocks per CU.

// The single-term fp16 kernels (a.f16) serve passes of more than
// SPLITK_MAX_M rows only, so they never split K.
template <int EPI, bool P16>
void launch_tile_p(hipStream_t s, const GemvArgs& a, const int32_t* d_pos) {
  if constexpr (P16 && (EPI == GV_RELU2 || EPI == GV_STORE)) {
    // single-term fc and lm_head over more than 4096 rows: 256x256 tiles (8
    // wavefronts of 128x64; one fp16 A plane leaves room for them), 4 % of
    // the GEMM time faster than 128x256 over 8 x 2048 rows in the layer stack;
    // two 64-wide K slices (128 KB) rather than three 32-wide ones, half the
    // barriers per K: 0.8 % of the 8 x 2048 eval forward (identical bits; at
    // 2048 rows the 128x256 tiles are 1.5 % slower with them)
    if (a.M > 4096 && a.N % 256 == 0) {
      GemvArgs b = a;
      b.part = nullptr;
      launch_cfg2<EPI, 2, 4, 4, 2, 2, P16, 64>(s, b, d_pos);
      return;
    }
  }
  if constexpr (EPI == GV_STORE) {
    // lm_head with the cross-entropy's partials: a register-epilogue tiling
    // (the only one that writes them; gemm_store_nll guarantees the shape)
    if (a.nll_part) {
      GemvArgs b = a;
      b.part = nullptr;
      launch_cfg2<EPI, 2, 2, 2, 4, 2, P16>(s, b, d_pos);
      return;
    }
  }
  const int sp = a.part && !P16 ? splitk_count(a.M, a.N, a.K) : 1;
  if (sp > 1) {
    launch_splitk_parts<EPI>(s, a, sp, d_pos);
    const dim3 rg((unsigned)a.M, (unsigned)((a.N + RED_COLS - 1) / RED_COLS));
    FG_LAUNCH((k_splitk_reduce<EPI>), rg, dim3(256), 0, s, a, sp, d_pos);
    return;
  }
  GemvArgs b = a;
  b.part = nullptr;  // the kernels below write the epilogue themselves
  const int64_t mt128 = (a.M + 127) / 128;
  // fc at prefill sizes: where 128x128 tiles spill into a second, mostly
  // empty round over the CUs, 128x192 tiles fit in one (QKV stays on
  // 128x128: its epilogue costs more per column in the wider tile)
  if constexpr (EPI == GV_RELU2) {
    const int64_t ncu = cu_count();
    if (a.N % 192 == 0 && a.K % 64 == 0 && mt128 * (a.N / 128) > ncu &&
        mt128 * (a.N / 192) <= ncu) {
      launch_cfg<EPI, 128, 192, 4, 2, 64, 2, 1, P16>(s, b, d_pos);
      return;
    }
  }
  if (a.N % 256 == 0 && ((EPI == GV_STORE && mt128 * (a.N / 256) >= 384) ||
                         (EPI == GV_RELU2 && mt128 * (a.N / 256) >= 768))) {
    launch_cfg2<EPI, 2, 2, 2, 4, 2, P16>(s, b, d_pos);
    return;
  }
  const bool big = a.N % 128 == 0 && mt128 * (a.N / 128) >= 256;
  if (big && (EPI == GV_RELU2 || EPI == GV_STORE)) {
    launch_cfg2<EPI, 4, 2, 1, 2, 3, P16>(s, b, d_pos);
    return;
  }
  if constexpr (EPI == GV_RESID) {
    if (resid_k4(a.M, a.N, a.K)) {
      launch_cfg<EPI, 64, 96, 2, 1, 64, 3, 4, P16>(s, b, d_pos);
      return;
    }
    if (resid_160(a.M, a.N, a.K)) {
      launch_cfg<EPI, 64, 160, 2, 1, 64, 3, 2, P16>(s, b, d_pos);
      return;
    }
  }
  const int bn = tile_n(a.M, a.N);
  if constexpr (EPI == GV_QKV) {
    // 128x128 tiles where they fit in one round and 64x128 ones would need
    // two (the depth-20 model at 2047 rows: 224 tiles against 448)
    const int64_t ncu = cu_count(), t128 = mt128 * (a.N / 128);
    if (bn == 128 && !big && t128 <= ncu && 2 * t128 > ncu) {
      launch_cfg<EPI, 128, 128, 4, 2, 32, 3, 1, P16>(s, b, d_pos);
      return;
    }
  }
  if (P16 && bn == 128 && big && EPI != GV_STORE && a.M > 1024 && a.K % 64 == 0)
    // single-term QKV and residual GEMMs that fill the chip with 128x128
    // tiles: 64-wide K slices, two stages (64 KB with one fp16 A plane):
    // 1-3 % of the GEMM time faster than 32-wide ones over 8 x 2048 rows,
    // and the depth-12 forward 0.9 % (1 x 2048) to 1.2 % (2 x 2048) faster
    launch_cfg<EPI, 128, 128, 4, 2, 64, 2, 1, P16>(s, b, d_pos);
  else if (bn == 128 && big)
    launch_cfg<EPI, 128, 128, 4, 2, 32, 3, 1, P16>(s, b, d_pos);  // 72 KB: two blocks per CU
  else if (bn == 128 && EPI == GV_RESID && a.K % 64 == 0)
    // the residual GEMMs (proj, proj2) inside the layer stack: 64-wide slices
    // (half the stage hand-overs) measured ~4 us a launch faster than 32-wide
    // ones at any depth
    launch_cfg<EPI, 64, 128, 2, 2, 64, 3, 1, P16>(s, b, d_pos);
  else if (bn == 128)
    launch_cfg<EPI, 64, 128, 2, 2, 32, 4, 1, P16>(s, b, d_pos);
  else
    launch_cfg<EPI, 64, 64, 2, 2, 32, 4, 1, P16>(s, b, d_pos);
}

template <int EPI>
void launch_tile(hipStream_t s, const GemvArgs& a, const int32_t* d_pos) {
  if (a.f16)
    launch_tile_p<EPI, true>(s, a, d_pos);
  else
    launch_tile_p<EPI, false>(s, a, d_pos);
}

}  // namespace

// Compute units of the current device (tile counts are weighed against it).
int cu_count() {
  static std::atomic<int> n[64];  // 0: not looked up yet (handles on several threads)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = n[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        v <= 0)
      v = 256;
    n[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

// lm_head writes the log-sum-exp partials over 1025 to 4096 rows. Measured
// against the separate pass over the logits on the depth-12 forward: 10-30
// us faster per pass at 2048 and 4096 rows, 10 us slower at 1024 (the pass
// over 128 MB of logits is short there); beyond 4096 rows the 256x256 tiles
// hold 64 rows a lane and the epilogue's reductions cost more than the pass.
bool gemm_store_nll(int64_t M, int N) { return M > 1024 && M <= 4096 && N % 256 == 0; }

// RESID on k_gemm: one sum-of-squares partial per row and N tile; split-K
// RESID (given split-K scratch): one per row and 512 columns.
int gemm_ssq_parts(int64_t M, int N, int K) {
  if (splitk_count(M, N, K) == 1 && resid_k4(M, N, K)) return N / 96;
  if (splitk_count(M, N, K) == 1 && resid_160(M, N, K)) return N / 160;
  return splitk_count(M, N, K) > 1 ? (N + RED_COLS - 1) / RED_COLS : N / tile_n(M, N);
}

int64_t gemm_splitk_floats(int64_t M, int N, int K) {
  const int sp = splitk_count(M, N, K);
  return sp > 1 ? (int64_t)sp * M * N : 0;
}

void launch_gemm_pos(hipStream_t s, GemvEpi epi, const GemvArgs& a, const int32_t* d_pos) {
  switch (epi) {
    case GV_QKV: launch_tile<GV_QKV>(s, a, d_pos); break;
    case GV_RESID: launch_tile<GV_RESID>(s, a, d_pos); break;
    case GV_RELU2: launch_tile<GV_RELU2>(s, a, d_pos); break;
    default: launch_tile<GV_STORE>(s, a, d_pos); break;
  }
}

int launch_gemm_partials(hipStream_t s, GemvEpi epi, const GemvArgs& a, const int32_t* d_pos) {
  const int sp = a.part && !a.f16 ? splitk_count(a.M, a.N, a.K) : 1;
  if (sp <= 1) return 0;
  switch (epi) {  // (the kernel writes raw partials whatever the epilogue)
    case GV_QKV: launch_splitk_parts<GV_QKV>(s, a, sp, d_pos); break;
    case GV_RESID: launch_splitk_parts<GV_RESID>(s, a, sp, d_pos); break;
    case GV_RELU2: launch_splitk_parts<GV_RELU2>(s, a, sp, d_pos); break;
    default: launch_splitk_parts<GV_STORE>(s, a, sp, d_pos); break;
  }
  return sp;
}

void launch_gemm(hipStream_t s, GemvEpi epi, const GemvArgs& a) {
  launch_gemm_pos(s, epi, a, nullptr);
}

}  // namespace fgpt
