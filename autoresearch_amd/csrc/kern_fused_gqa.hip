// kern_fused_gqa.hip -- the B=1 greedy decode loop (gpt_step fed back
// through its argmax, src/app/chat_text.f90:423-462 with
// src/lib/fortran_kv.f90:26-149 per step) as ONE persistent launch on
// gfx950, for models whose query heads share two KV heads (grouped-query
// attention: G = H / 2 query heads per KV head, src/lib/fortran_attn.f90:
// 317-362 with the head-to-KV-head map of :330-334).
//
// Why one launch: the depth-20 GQA model's weights (700 MB) stream from
// HBM every token, but each linear of a step is a few MB, and a kernel of
// its own pays its launch and a first load round trip (~4-5 us) for it: six
// launches a layer, most of a step. Here 256 workgroups, one per CU, run
// the whole loop, and each phase's weight slice streams into LDS a layer
// ahead (below), so the hand-overs between workgroups are what remains on
// the critical path.
//
// Work split (workgroup (g, c): the c-th of the 32 workgroups on XCD g; KV
// head k = g / 4, quarter q = g % 4, index in the group i = 32 q + c):
//   q/k/v rows of group k (its G query heads, then its k and v): rotation
//     pairs [i P / 128, (i + 1) P / 128) of the group's P = (G + 2) hd / 2
//   attention: positions i, i + 128, i + 256, ... of the group's G heads
//     (each cached K/V row is read once for the G heads)
//   the XCD's 32 partial results merged: G hd / 32 outputs per workgroup
//   the group's 4 quarter results merged (every workgroup of the group),
//     then c_proj over the group's G hd inputs for outputs
//     [i D / 128, (i + 1) D / 128)
//   c_fc rows [g dff/8 + c dff/256, ...) and c_proj2 over the XCD's dff/8
//     hidden units for outputs [c D/32, (c+1) D/32), as in kern_fused.hip
//   lm_head rows [b V/256, (b+1) V/256), b = g + 8 c
// The residual columns [c D/32, (c+1) D/32) are owned by workgroup (g, c)
// of every XCD: the two groups' c_proj partials and the 8 blocks' c_proj2
// partials are added to them in a fixed order.
//
// Hand-overs per layer (exchange slots as in kern_fused.hip: value | epoch,
// write-through across XCDs): q/k/v across the group's XCDs, workgroup
// partials within the XCD, XCD partials across the group, c_proj partials
// across, the residual within, the hidden block within, c_proj2 partials
// across, the residual within; the step ends with the lm_head argmax
// candidates of all 256 workgroups. Cache rows are written through
// (agent-scope stores), since the group's 4 XCDs read them.
//
// Weights: a layer's slice per workgroup (~133 KB at depth 20) does not fit
// in LDS twice, so each phase has its own LDS region, refilled for the next
// layer as soon as its phase is done: loader wave A fills the q/k/v and
// c_fc regions, loader wave B the c_proj and c_proj2 regions (two waves, so
// that each waits on its own in-order vector-memory counter for the batch
// the next phase needs). lm_head's rows go to the c_fc region and to the
// q/k/v + c_proj regions during the last layer; the next step's layer 0
// follows them. The q/k/v region doubles as the attention's staging area
// (between the q/k/v rows' use and their refill).
//
// Arithmetic per output element: rmsnorm0 (src/lib/fortran_rmsnorm.f90:
// 40-60) as a scale of the dot products, fp32 accumulation of bf16 weights
// times fp32 activations, rope_4d (src/lib/fortran_rope.f90:25-52) on the
// host's tables, attn_step's softmax (src/lib/fortran_attn.f90:317-362)
// merged from per-wave, per-workgroup and per-XCD partial results in a
// fixed order, relu2 (:697-710), residual adds (src/lib/fortran_kv.f90:
// 125-137), and the first-max argmax of src/lib/sample.f90:271-277.
#include <float.h>
#include <string.h>

#include <algorithm>

#include "kern_fused.h"

namespace fgpt {

namespace {

constexpr int GQA_THREADS = 384;  // 4 compute waves + 2 loader waves
// copies of the hand-overs every workgroup of a group reads (its q/k/v and
// the XCDs' partial attention results), one per XCD of the group: each
// copy's lines are then read by the 32 workgroups of one XCD, not by 128
constexpr int GQA_COPIES = 4;

constexpr int64_t max64(int64_t a, int64_t b) { return a > b ? a : b; }

// The work split's sizes for one model shape (head_dim 128, two KV heads,
// d_ff = 4 d_model); fused_layout_gqa computes the same values at run time.
template <int D_, int H_, int V_>
struct GqaShape {
  static constexpr int HD = 128, D = D_, H = H_, KH = 2, G = H_ / 2, V = V_, DFF = 4 * D_;
  static constexpr int NPR = (G + 2) * HD / 2;  // rotation pairs of a group's q/k/v rows
  static constexpr int QP = (NPR + 127) / 128;  // pairs per workgroup, at most
  static constexpr int GQ = G * HD;             // a group's query dims
  static constexpr int NPO = D / 128;           // c_proj outputs per workgroup of a group
  static constexpr int OPW = GQ / FUSED_NC;     // XCD-merge outputs per workgroup
  static constexpr int APS = GQ + 2 * G;        // slots of a partial: O, then (max, sum) per head
  static constexpr int C = D / FUSED_NC, FR = DFF / FUSED_NWG, HN = DFF / FUSED_NX;
  static constexpr int LR = V / FUSED_NWG;
  // staging in the q/k/v region: the waves' attention records, then the
  // XCD merge's inputs; the group merge's inputs reuse the records' bytes
  static constexpr int64_t R1 = 4LL * 4 * G * (HD + 4), R2 = 4LL * 32 * (OPW + 2 * G);
  static constexpr int64_t R3 = 4LL * 4 * APS;
  static constexpr int64_t AQ = round1k(2LL * QP * D * 2);
  static constexpr int64_t SQ = round1k(max64(AQ, R1 + R2));
  static constexpr int64_t SP = round1k((int64_t)NPO * GQ * 2);
  static constexpr int64_t SF = round1k((int64_t)FR * D * 2);
  static constexpr int64_t S2 = round1k((int64_t)C * HN * 2);
  static constexpr int64_t OFF_P = SQ, OFF_F = SQ + SP, OFF_2 = OFF_F + SF, WEND = OFF_2 + S2;
  // fused arena per workgroup: per layer the four regions' bytes (q/k/v
  // rows AQ, c_proj SP, c_fc SF, c_proj2 S2), then lm_head: NA rows padded
  // to SF, the other LR - NA rows
  static constexpr int NA = LR < (int)(SF / (D * 2)) ? LR : (int)(SF / (D * 2));
  static constexpr int64_t LMB_B = round1k((int64_t)(LR - NA) * D * 2);
  static constexpr int64_t SLICE = AQ + SP + SF + S2, LMB = SF + LMB_B;
  static constexpr int HY = HN > GQ ? HN : GQ;
  // cached positions per workgroup, at most: their K and V rows (1 KB a
  // position) are DMA'd into the c_proj2 region, idle from the layer's
  // start until c_proj2's rows refill it; AB a wave
  static constexpr int NPW = S2 / 1024 < 32 ? (int)(S2 / 1024) / 4 * 4 : 32, AB = NPW / 4;
  // LDS after the weight regions (floats): x, hidden / attention output,
  // q/k/v of the group, reduction scratch, red, ired, stop, place, rope
  static constexpr int64_t ACT = 4LL * (D + HY + (G + 2) * HD + 4 * 8 * 64 + 8 + 8 + 1 + 2 + HD);
  static constexpr int64_t LDS = WEND + ACT;
  // exchange slots
  static constexpr int64_t OFF_QL = 0;
  static constexpr int64_t OFF_AP = OFF_QL + 2LL * KH * GQA_COPIES * (G + 2) * HD;
  static constexpr int64_t OFF_XP = OFF_AP + 2LL * FUSED_NX * FUSED_NC * APS;
  static constexpr int64_t OFF_PP = OFF_XP + 2LL * KH * GQA_COPIES * 4 * APS;
  static constexpr int64_t OFF_XL = OFF_PP + 2LL * KH * D;
  static constexpr int64_t OFF_HL = OFF_XL + 2LL * FUSED_NX * D;
  static constexpr int64_t OFF_P2 = OFF_HL + 2LL * FUSED_NX * HN;
  static constexpr int64_t OFF_LM = OFF_P2 + 2LL * FUSED_NX * D;
  static constexpr int64_t SLOTS = OFF_LM + 2LL * FUSED_LMC * 2 * FUSED_NWG;
  // 1 KB DMA instructions per region (the loader waves' counter waits)
  static constexpr int NQ = (int)(AQ / 1024), NP = (int)(SP / 1024), NF = (int)(SF / 1024);
  static constexpr int N2 = (int)(S2 / 1024), NLB = (int)(LMB_B / 1024);
  static_assert(H_ % 2 == 0 && QP <= 4, "q/k/v pairs: one per compute wave");
  static_assert(D % 256 == 0 && GQ % 128 == 0 && GQ % FUSED_NC == 0 && C <= 64, "work split");
  static_assert(R3 <= R1, "the group merge's inputs must not overlap the XCD merge's");
  static_assert(LMB_B <= SQ + SP, "lm_head rows past the c_fc region fit the q/k/v + c_proj ones");
  static_assert(NQ <= 63 && NP <= 63 && NF <= 63 && N2 <= 63, "vmcnt immediates");
  static_assert(LDS <= 160 * 1024, "LDS");
  static_assert(AB >= 1 && HD == 128, "a cached position's K and V rows: 1 KB");
};
// The shapes built: the depth-20 GQA model's (d_model 1280, 10 heads over
// 2 KV heads, vocab 8192) and a small one the tests run.
typedef GqaShape<1280, 10, 8192> GqaD20;
typedef GqaShape<512, 4, 1024> GqaSmall;

// dma16 with the non-temporal hint: the weight stream, read once a token,
// should not displace the exchange slots and cache rows from the caches
__device__ __forceinline__ void dma16_nt(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(g), "s"(lds)
               : "memory", "m0");
}

// Sum (maximum) over the four 16-lane rows of the wave: every lane gets
// the sum of lanes l, l^16, l^32, l^48, by gfx950's lane-half and row swaps
// (v_permlane32_swap: lanes 32-63 of the first operand with lanes 0-31 of
// the second; v_permlane16_swap: odd rows of the first with even rows of
// the second), in the order (r0 + r2) + (r1 + r3).
__device__ __forceinline__ float rows4_sum(float v) {
  const uint32_t u = __float_as_uint(v);
  const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const float t = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const uint32_t w = __float_as_uint(t);
  const auto b = __builtin_amdgcn_permlane16_swap(w, w, false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ __forceinline__ float rows4_max(float v) {
  const uint32_t u = __float_as_uint(v);
  const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const float t = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const uint32_t w = __float_as_uint(t);
  const auto b = __builtin_amdgcn_permlane16_swap(w, w, false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

template <int N>
__device__ __forceinline__ void vm_wait() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Wait until the slots at p[off[i]] (i < n <= NMAX) carry epoch ep and
// return their values: slots_wait for slots at computed offsets.
template <int NMAX>
__device__ bool slots_wait_at(const uint64_t* p, const int (&off)[NMAX], int n, uint32_t ep,
                              float* out, uint32_t* err) {
  uint64_t v[NMAX];
#pragma unroll
  for (int i = 0; i < NMAX; ++i) v[i] = i < n ? slot_load(p + off[i]) : slot_pack(0.f, ep);
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
#pragma unroll
    for (int i = 0; i < NMAX; ++i)
      if (i < n && (uint32_t)(v[i] >> 32) != ep) v[i] = slot_load(p + off[i]);
  }
#pragma unroll
  for (int i = 0; i < NMAX; ++i)
    if (i < n) out[i] = __uint_as_float((uint32_t)v[i]);
  return true;
}

template <class Sh, bool TRACE>
__global__ __launch_bounds__(GQA_THREADS) void k_fused_gqa(FusedArgs a) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
  constexpr int HD = Sh::HD, D = Sh::D, G = Sh::G, KH = Sh::KH, V = Sh::V, KD = KH * HD;
  constexpr int GQ = Sh::GQ, APS = Sh::APS, OPW = Sh::OPW, NPO = Sh::NPO, NPR = Sh::NPR;
  constexpr int C = Sh::C, FR = Sh::FR, HN = Sh::HN, LR = Sh::LR, NA = Sh::NA;
  constexpr int AB = Sh::AB;
  constexpr int REC = HD + 4;          // floats per wave attention record: O, max, sum
  constexpr int XW = OPW + 2 * G;      // XCD-merge inputs per workgroup partial
  const int L = a.L;
  const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
  const bool comp = wv < 4, ldA = wv == 4, ldB = wv == 5;
  const float eps = a.eps;
  float* x_lds = (float*)(lds + Sh::WEND);
  float* hy = x_lds + D;               // the hidden block, or the group's attention output
  float* qkv_lds = hy + Sh::HY;        // q (G heads), k, v of the group
  float* scr0 = qkv_lds + (G + 2) * HD;  // reduction scratch, [4 waves][8][64]
  float* scr = scr0 + (comp ? wv : 0) * 8 * 64;
  float* red = scr0 + 4 * 8 * 64;      // [8]
  int* ired = (int*)(red + 8);         // [8]
  int* stop = ired + 8;
  int* place = stop + 1;
  float* rope = (float*)(place + 2);   // cos, sin of the step's position [2][HD/2]
  float* rec = (float*)lds;            // staging: [4 waves][G][REC]
  float* xg = (float*)(lds + Sh::R1);  // staging: [32][XW]
  float* gg = (float*)lds;             // staging: [4 quarters][APS]
  uint32_t* err = a.err;
  const int E = 8 * L + 8;  // epochs per step
  uint64_t* S = a.slots;
  const int64_t cu_bytes = (int64_t)L * Sh::SLICE + Sh::LMB;

  if (tid == 0) {
    uint32_t xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    const int gx = (int)(xcc & 7);
    const int cx = (int)atomicAdd(a.cnt + gx, 1u);
    *stop = 0;
    if (cx >= FUSED_NC) {
      __hip_atomic_store(err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *stop = 1;
    }
    place[0] = gx;
    place[1] = cx < FUSED_NC ? cx : 0;
  }
  lds_barrier();
  if (*stop) return;
  const int g = place[0], c = place[1], b = g + FUSED_NX * c;
  const int k = g >> 2, q = g & 3, gi = q * FUSED_NC + c;  // KV head, quarter, index in group
  const int plo = gi * NPR / 128, phi = (gi + 1) * NPR / 128;  // this workgroup's q/k/v pairs
  // optional phase timestamps (100 MHz device clock) of one step: stamp k
  // of layer l by thread 0 (14, 15: loader wave A's wait before the layer)
  auto mark = [&](int s, int l, int kk) {
    if (TRACE && s == a.trace_step &&
        tid == (kk == 14 || kk == 15 ? 256 : kk == 20 ? 320 : kk == 21 ? 64 : 0))
      a.trace[((int64_t)b * (L + 1) + l) * 32 + kk] = __builtin_amdgcn_s_memrealtime();
  };
  const uint8_t* arena = (const uint8_t*)a.arena + (int64_t)b * cu_bytes;

  // DMA of piece i of n of region R (0 q/k/v rows, 1 c_proj, 2 c_fc, 3
  // c_proj2) of layer l into its LDS region: its 1 KB chunks [i N / n,
  // (i + 1) N / n). Each region's refill is spread over several barriers of
  // the layer (see the schedule below) so that the weight stream, which at
  // this model size comes from HBM, does not arrive in bursts that the
  // hand-overs' polls queue behind. lm_head's rows: part 0 into the c_fc
  // region, part 1 into the q/k/v + c_proj regions.
  auto piece = [&](int l, int R, int i, int n) {
    constexpr int64_t soff[4] = {0, Sh::AQ, Sh::AQ + Sh::SP, Sh::AQ + Sh::SP + Sh::SF};
    constexpr int64_t doff[4] = {0, Sh::OFF_P, Sh::OFF_F, Sh::OFF_2};
    constexpr int nch[4] = {Sh::NQ, Sh::NP, Sh::NF, Sh::N2};
    const uint8_t* src = arena + (int64_t)l * Sh::SLICE + soff[R] + 16 * lane;
    const uint32_t dst = lds_off(lds + doff[R]);
    // (a rolled loop: unrolled, the chunks' addresses would each hold two
    // registers for the whole kernel)
#pragma unroll 1
    for (int ch = i * nch[R] / n; ch < (i + 1) * nch[R] / n; ++ch)
      dma16_nt(src + 1024 * ch, dst + 1024u * ch);
  };
  auto issue_lm = [&](int part) {
    const uint8_t* src = arena + (int64_t)L * Sh::SLICE + (part ? Sh::SF : 0) + 16 * lane;
    const uint32_t dst = lds_off(lds + (part ? 0 : Sh::OFF_F));
    const int n = part ? Sh::NLB : Sh::NF;
#pragma unroll 1
    for (int ch = 0; ch < n; ++ch) dma16_nt(src + 1024 * ch, dst + 1024u * ch);
  };
  // Loader schedule. Wave A (q/k/v rows, c_fc): Q(l+1) in two pieces at
  // B4b and B5 of layer l, F(l+1) in five at B6 of layer l and B0..B3 of
  // l+1. Wave B (cache rows, c_proj, c_proj2): layer l's cached K and V rows
  // of this workgroup's positions at B0 (into the c_proj2 region, waited
  // for before B1), 2(l) in five pieces at B2, B3, B4, B4b, B5, P(l+1) in
  // two at B5 and B6. At the last layer lm_head's part 1 (wave B, at B5)
  // and part 0 (wave A, at B6) take the place of the next layer's; the next
  // step's Q(0), P(0) follow the lm_head rows' use and F(0)'s first piece
  // the argmax exchange. The counter waits before the barriers that open a
  // region's phase leave the later pieces in flight.
  constexpr int NQP = 2, NPP = 2, NFP = 5, N2P = 5;  // pieces per region
  constexpr int WA_B0 = Sh::NF / NFP;                 // F's first piece
  constexpr int WA_B5 = Sh::NQ / NQP;                 // Q's first piece
  constexpr int WB_B6 = Sh::NP / NPP;                 // P's first piece
  auto next_step_rows = [&] {  // Q(0) and P(0) whole
    if (ldA)
      for (int i = 0; i < NQP; ++i) piece(0, 0, i, NQP);
    if (ldB)
      for (int i = 0; i < NPP; ++i) piece(0, 1, i, NPP);
  };

  // x = rmsnorm0(wte[id]) into x_lds (kern_fused.hip's order), x_own =
  // this workgroup's residual columns, and the RoPE row of position pos
  float x_own = 0.f;
  auto embed = [&](int id, int pos) {
    const bf16_t* row = a.wte + (int64_t)id * D;
    if (comp && tid < HD) rope[tid] = tid < HD / 2 ? a.cosb[(int64_t)pos * (HD / 2) + tid]
                                                   : a.sinb[(int64_t)pos * (HD / 2) + tid - HD / 2];
    if (comp) {
      float ss = 0.f;
      for (int kk = tid; kk < D; kk += 256) {
        const float v = bf16_to_f32(row[kk]);
        ss += v * v;
      }
      ss = wave_sum(ss);
      if (lane == 0) red[wv] = ss;
    }
    lds_barrier();
    if (comp) {
      const float t = red[0] + red[1] + red[2] + red[3];
      const float inv = 1.0f / sqrtf(t / (float)D + eps);
      for (int kk = tid; kk < D; kk += 256) x_lds[kk] = bf16_to_f32(row[kk]) * inv;
      if (wv == 0 && lane < C) x_own = bf16_to_f32(row[c * C + lane]) * inv;
    }
  };

  next_step_rows();
  if (ldA) piece(0, 2, 0, NFP);
  embed(*a.d_id0, a.len0);

  for (int s = 0; s < a.n_steps; ++s) {
    const int pos = a.len0 + s;
    for (int l = 0; l < L; ++l) {
      const int par = (s * L + l) & 1;
      const uint32_t ep = a.ep_base + (uint32_t)(s * E + l * 8);
      // (copy x of the group's q/k/v at QL + x (G+2) hd; of the XCD results at XP + x 4 APS)
      uint64_t* QL = S + Sh::OFF_QL + (int64_t)(par * KH + k) * GQA_COPIES * (G + 2) * HD;
      uint64_t* AP = S + Sh::OFF_AP + (int64_t)(par * FUSED_NX + g) * FUSED_NC * APS;
      uint64_t* XP = S + Sh::OFF_XP + (int64_t)(par * KH + k) * GQA_COPIES * 4 * APS;
      uint64_t* PP = S + Sh::OFF_PP + (int64_t)par * KH * D;
      uint64_t* XL = S + Sh::OFF_XL + (int64_t)(par * FUSED_NX + g) * D;
      uint64_t* HL = S + Sh::OFF_HL + (int64_t)(par * FUSED_NX + g) * HN;
      uint64_t* P2 = S + Sh::OFF_P2 + (int64_t)par * FUSED_NX * D;
      float* kc = a.kc + (int64_t)l * a.maxT * KD + k * HD;
      float* vc = a.vc + (int64_t)l * a.maxT * KD + k * HD;
      // B0: the q/k/v rows have landed (wave A: c_fc's batch may still fly)
      mark(s, l, 14);
      if (ldA) vm_wait<WA_B0>();
      mark(s, l, 15);
      lds_barrier();
      mark(s, l, 0);
      if (TRACE && s == a.trace_step && tid == 0)
        a.trace[((int64_t)b * (L + 1) + l) * 32 + 24] = __builtin_readcyclecounter();
      if (*stop) goto done;
      if (ldA) piece(l, 2, 1, NFP);
      if (ldB) {
        // the K and V rows of this workgroup's cached positions gi + 128 li
        // < pos, position li's 1 KB at 1 KB li of the c_proj2 region (lanes
        // 0-31 its K row, 32-63 its V row)
        const float* src = (lane < 32 ? kc : vc) + 4 * (lane & 31);
        const uint32_t dst = lds_off(lds + Sh::OFF_2);
#pragma unroll 1
        for (int li = 0; gi + 128 * li < pos; ++li)
          dma16(src + (int64_t)(gi + 128 * li) * KD, dst + 1024u * li);
      }
      if (comp) {
        // q/k/v pair plo + wave of the group: rows (2 w, 2 w + 1) of the
        // region, head dims j and j + hd/2 of part p / (hd/2)
        const int p = plo + wv;
        if (p < phi) {
          const int ro[2] = {2 * wv * D * 2, (2 * wv + 1) * D * 2};
          float acc[2];
          dot_rows<2, D>(lds, ro, x_lds, lane, acc);
          const float inv = 1.0f / sqrtf(sumsq<D>(x_lds, lane) / (float)D + eps);
          const float v0 = wave_sum(acc[0]) * inv, v1 = wave_sum(acc[1]) * inv;
          const int part = p / (HD / 2), j = p % (HD / 2);
          float y1 = v0, y2 = v1;
          if (part <= G) {  // q heads and k: rotated
            const float cs = rope[j], sn = rope[HD / 2 + j];
            y1 = v0 * cs + v1 * sn;
            y2 = v0 * (-sn) + v1 * cs;
          }
          if (lane < GQA_COPIES) {  // lane x writes copy x
            uint64_t* qx = QL + (int64_t)lane * (G + 2) * HD + part * HD + j;
            slot_put_dev(qx, y1, ep);
            slot_put_dev(qx + HD / 2, y2, ep);
          }
          if (lane == 0) {
            if (part >= G) {  // the cache row at pos, written through: read by the group's 4 XCDs
              float* cr = (part == G ? kc : vc) + (int64_t)pos * KD;
              __hip_atomic_store(cr + j, y1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              __hip_atomic_store(cr + j + HD / 2, y2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
          }
        }
        mark(s, l, 1);
        if (!gather_slots<((G + 2) * HD + 255) / 256, XPRE, XGAP>(QL + (int64_t)q * (G + 2) * HD, (G + 2) * HD, ep,
                                                       qkv_lds, tid, err))
          *stop = 1;
        mark(s, l, 19);
        mark(s, l, 21);
      }
      if (ldB) vm_wait<0>();  // the cache rows (and the c_proj rows before them)
      mark(s, l, 20);
      lds_barrier();  // B1
      mark(s, l, 2);
      if (*stop) goto done;
      if (ldA) piece(l, 2, 2, NFP);
      if (comp) {
        // the wave's scores for the G heads, one softmax over its slots.
        // 16 lanes a cached row (8 head dims each), 4 rows a wave: slot
        // (h, r) of wave w is position li = w + 4 (4 h + r), cached rows
        // from the c_proj2 region, the new position's k and v from the
        // hand-over. A score is a sum over the row's 16 lanes (DPP, no
        // lane reads); the rows' maxima, weight sums and weighted V sums
        // meet by lane swaps (rows4_max, rows4_sum).
        // Branch-free: every slot is read (in bounds: li clamped below NPW)
        // and weighed, those past pos masked.
        constexpr int NH = (AB + 3) / 4;
        const float scale = 1.0f / sqrtf((float)HD);
        const int r = lane >> 4, d0 = 8 * (lane & 15);
        float k8[NH][8], v8[NH][8];
        bool ok[NH];
#pragma unroll
        for (int h = 0; h < NH; ++h) {
          const int li = wv + 4 * (4 * h + r), pp = gi + 128 * li;
          ok[h] = pp <= pos;
          const float* rp = pp == pos ? qkv_lds + GQ
                                      : (const float*)(lds + Sh::OFF_2 + 1024 * min(li, Sh::NPW - 1));
          const float4 ka = *(const float4*)(rp + d0), kb = *(const float4*)(rp + d0 + 4);
          const float4 va = *(const float4*)(rp + HD + d0), vb = *(const float4*)(rp + HD + d0 + 4);
          const float kk[8] = {ka.x, ka.y, ka.z, ka.w, kb.x, kb.y, kb.z, kb.w};
          const float vv[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            k8[h][e] = ok[h] ? kk[e] : 0.f;
            v8[h][e] = ok[h] ? vv[e] : 0.f;
          }
        }
#pragma unroll
        for (int j = 0; j < G; ++j) {
          const float4 qa = *(const float4*)(qkv_lds + j * HD + d0);
          const float4 qb = *(const float4*)(qkv_lds + j * HD + d0 + 4);
          const float q8[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
          float sc[NH];
          float m = -FLT_MAX;  // (no position: max -FLT_MAX, sum 0, O 0)
#pragma unroll
          for (int h = 0; h < NH; ++h) {
            float t = q8[0] * k8[h][0];
#pragma unroll
            for (int e = 1; e < 8; ++e) t += q8[e] * k8[h][e];
            t += dpp_f<0xB1>(t);   // the row's 16 lanes: quad permutes, then
            t += dpp_f<0x4E>(t);   // the half-row and row mirrors
            t += dpp_f<0x141>(t);
            t += dpp_f<0x140>(t);
            sc[h] = ok[h] ? t * scale : -INFINITY;
            m = fmaxf(m, sc[h]);
          }
          m = rows4_max(m);
          float ls = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int h = 0; h < NH; ++h) {
            const float e = ok[h] ? __expf(sc[h] - m) : 0.f;
            ls += e;
#pragma unroll
            for (int x = 0; x < 8; ++x) o[x] += e * v8[h][x];
          }
          ls = rows4_sum(ls);
#pragma unroll
          for (int x = 0; x < 8; ++x) o[x] = rows4_sum(o[x]);
          float* rj = rec + (wv * G + j) * REC;
          if (lane < 16) {
            *(float4*)(rj + d0) = make_float4(o[0], o[1], o[2], o[3]);
            *(float4*)(rj + d0 + 4) = make_float4(o[4], o[5], o[6], o[7]);
          }
          if (lane == 0) {
            rj[HD] = m;
            rj[HD + 1] = ls;
          }
        }
      }
      lds_barrier();  // B2
      mark(s, l, 3);
      if (ldA) piece(l, 2, 3, NFP);
      if (ldB) piece(l, 3, 0, N2P);
      if (comp) {
        // this workgroup's partial: the 4 waves' records in wave order, to
        // the XCD: O (unnormalised) per query dim, then (max, sum) per head
        for (int idx = tid; idx < APS; idx += 256) {
          const int j = idx < GQ ? idx / HD : (idx - GQ) >> 1;
          float mx = rec[j * REC + HD];
#pragma unroll
          for (int w = 1; w < 4; ++w) mx = fmaxf(mx, rec[(w * G + j) * REC + HD]);
          float t = 0.f;
          if (idx < GQ || ((idx - GQ) & 1)) {
            const int e = idx < GQ ? idx % HD : HD + 1;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
              const float* rw = rec + (w * G + j) * REC;
              t += __expf(rw[HD] - mx) * rw[e];
            }
          } else {
            t = mx;
          }
          slot_put_xcd(AP + (int64_t)c * APS + idx, t, ep + 1);
        }
        mark(s, l, 4);
        // the XCD's 32 partials this workgroup merges: O at its OPW
        // outputs, and every head's (max, sum)
        constexpr int NXG = (32 * XW + 255) / 256;
        int off[NXG];
        int cnt = 0;
#pragma unroll
        for (int i = 0; i < NXG; ++i) {
          const int t = tid + 256 * i;
          off[i] = 0;
          if (t < 32 * XW) {
            const int w = t / XW, e = t % XW;
            off[i] = w * APS + (e < OPW ? c * OPW + e : GQ + (e - OPW));
            cnt = i + 1;
          }
        }
        float v[NXG];
        if (!slots_wait_at<NXG>(AP, off, cnt, ep + 1, v, err)) *stop = 1;
#pragma unroll
        for (int i = 0; i < NXG; ++i)
          if (i < cnt) xg[tid + 256 * i] = v[i];
      }
      lds_barrier();  // B3
      mark(s, l, 5);
      if (*stop) goto done;
      if (ldA) piece(l, 2, 4, NFP);
      if (ldB) piece(l, 3, 1, N2P);

      if (comp) {
        // the XCD's result for outputs [c OPW, (c+1) OPW) of the group's
        // query dims, and (max, sum) of the heads whose first dim is here:
        // item it on 8 lanes, each over partials k, k + 8, k + 16, k + 24,
        // the 8 lanes met by DPP (quad permutes, then the half-row mirror)
        const int it = tid >> 3, k8 = tid & 7;
        static_assert(OPW + G <= 32, "XCD-merge items on 8 lanes each");
        if (it < OPW + G) {
          const int o = c * OPW + (it < OPW ? it : 0);
          const int j = it < OPW ? o / HD : it - OPW;
          if (it < OPW || c == j * HD / OPW) {
            const int e = it < OPW ? it : OPW + 2 * j + 1;
            float mw[4], vw[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float* xw = xg + (k8 + 8 * i) * XW;
              mw[i] = xw[OPW + 2 * j];
              vw[i] = xw[e];
            }
            float mx = fmaxf(fmaxf(mw[0], mw[1]), fmaxf(mw[2], mw[3]));
            mx = fmaxf(mx, dpp_f<0xB1>(mx));
            mx = fmaxf(mx, dpp_f<0x4E>(mx));
            mx = fmaxf(mx, dpp_f<0x141>(mx));
            float t = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) t += __expf(mw[i] - mx) * vw[i];
            t += dpp_f<0xB1>(t);
            t += dpp_f<0x4E>(t);
            t += dpp_f<0x141>(t);
            if (k8 < GQA_COPIES) {  // lane x of the item writes copy x
              uint64_t* xp = XP + (int64_t)(k8 * 4 + q) * APS;
              if (it < OPW) {
                slot_put_dev(xp + o, t, ep + 2);
              } else {
                slot_put_dev(xp + GQ + 2 * j, mx, ep + 2);
                slot_put_dev(xp + GQ + 2 * j + 1, t, ep + 2);
              }
            }
          }
        }
        mark(s, l, 6);
        // the group's 4 quarter results
        if (!gather_slots<(4 * APS + 255) / 256, XPRE, XGAP>(XP + (int64_t)q * 4 * APS, 4 * APS, ep + 2, gg,
                                                  tid, err))
          *stop = 1;
      }
      lds_barrier();  // B4 (c_proj's rows landed before B1)
      mark(s, l, 7);
      if (*stop) goto done;
      if (ldB) piece(l, 3, 2, N2P);
      if (comp) {
        // the group's attention output: the 4 quarters in order
        for (int o = tid; o < GQ; o += 256) {
          const int j = o / HD;
          float mx = gg[GQ + 2 * j];
#pragma unroll
          for (int qq = 1; qq < 4; ++qq) mx = fmaxf(mx, gg[qq * APS + GQ + 2 * j]);
          float t = 0.f, ls = 0.f;
#pragma unroll
          for (int qq = 0; qq < 4; ++qq) {
            const float e = __expf(gg[qq * APS + GQ + 2 * j] - mx);
            t += e * gg[qq * APS + o];
            ls += e * gg[qq * APS + GQ + 2 * j + 1];
          }
          hy[o] = t / ls;
        }
      }
      lds_barrier();  // B4b
      mark(s, l, 8);
      if (ldA && l + 1 < L) piece(l + 1, 0, 0, NQP);
      if (ldB) piece(l, 3, 3, N2P);

      if (comp) {
        // c_proj over the group's query dims for outputs gi NPO + r: wave w
        // takes r = w, w + 4, ...
        constexpr int NRP = (NPO + 3) / 4;
        int ro[NRP];
#pragma unroll
        for (int i = 0; i < NRP; ++i) ro[i] = min(wv + 4 * i, NPO - 1) * GQ * 2;
        float acc[NRP];
        dot_rows<NRP, GQ>(lds + Sh::OFF_P, ro, hy, lane, acc);
#pragma unroll
        for (int i = 0; i < NRP; ++i) {
          const float t = wave_sum(acc[i]);
          const int r = wv + 4 * i;
          if (lane == 0 && r < NPO) slot_put_dev(PP + (int64_t)k * D + gi * NPO + r, t, ep + 3);
        }
        mark(s, l, 9);
      }
      // residual += the two groups' c_proj partials (groups in order)
      if (wv == 0 && lane < C) {
        float pv[2];
        if (!slots_wait<2, XPRE, XGAP>(PP + c * C + lane, D, KH, ep + 3, pv, err)) *stop = 1;
        const float t = pv[0] + pv[1];
        x_own = x_own + t;
        slot_put_xcd(XL + c * C + lane, x_own, ep + 4);
      }
      mark(s, l, 10);
      if (comp && !*stop && !gather_slots<(D + 255) / 256>(XL, D, ep + 4, x_lds, tid, err))
        *stop = 1;
      if (ldA) {  // c_fc's rows (the next q/k/v rows' first piece may still fly)
        if (l + 1 < L)
          vm_wait<WA_B5>();
        else
          vm_wait<0>();
      }
      lds_barrier();  // B5
      mark(s, l, 11);
      if (*stop) goto done;
      if (ldA && l + 1 < L) piece(l + 1, 0, 1, NQP);
      if (ldB) {
        piece(l, 3, 4, N2P);
        if (l + 1 < L)
          piece(l + 1, 1, 0, NPP);
        else
          issue_lm(1);
      }
      // h = relu2(rmsnorm0(x) c_fc^T) for this workgroup's fc rows: wave w
      // takes rows w, w+4, ... (four at a time)
      if (comp) {
        const float inv = 1.0f / sqrtf(sumsq<D>(x_lds, lane) / (float)D + eps);
        // wave w takes rows w, w + 4, ..., FR / 4 of them in one pass
        constexpr int NRF = FR / 4;
        static_assert(FR % 4 == 0 && NRF <= 8, "fc rows per wave");
        float acc[8];
        int ro[NRF];
#pragma unroll
        for (int i = 0; i < NRF; ++i) ro[i] = (wv + 4 * i) * D * 2;
        {
          float t[NRF];
          dot_rows<NRF, D>(lds + Sh::OFF_F, ro, x_lds, lane, t);
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[i] = i < NRF ? t[i] : 0.f;
        }
        float t = multi_sum<8>(acc, scr, lane) * inv;
        t = t < 0.f ? 0.f : t;
        const int r = wv + 4 * (lane >> 3);
        if ((lane & 7) == 0 && (lane >> 3) < NRF) slot_put_xcd(HL + c * FR + r, t * t, ep + 5);
        mark(s, l, 12);
        if (!gather_slots<(HN + 255) / 256>(HL, HN, ep + 5, hy, tid, err)) *stop = 1;
      }
      if (ldB) {  // c_proj2's rows (the next c_proj rows, or lm_head's, may still fly)
        if (l + 1 < L)
          vm_wait<WB_B6>();
        else
          vm_wait<Sh::NLB>();
      }
      lds_barrier();  // B6
      mark(s, l, 13);
      if (*stop) goto done;
      if (ldA) {
        if (l + 1 < L)
          piece(l + 1, 2, 0, NFP);
        else
          issue_lm(0);
      }
      if (ldB && l + 1 < L) piece(l + 1, 1, 1, NPP);
      // c_proj2 partial over this XCD's fc block: wave w takes outputs w,
      // w+4, ... (eight at a time)
      if (comp) {
        // wave w takes outputs w, w + 4, ..., C / 4 of them, their dot
        // products in one pass, summed eight at a time
        constexpr int NOC = C / 4;
        static_assert(C % 4 == 0 && NOC <= 16, "c_proj2 outputs per wave");
        float v[NOC];
        {
          int ro[NOC];
#pragma unroll
          for (int i = 0; i < NOC; ++i) ro[i] = (wv + 4 * i) * HN * 2;
          dot_rows<NOC, HN>(lds + Sh::OFF_2, ro, hy, lane, v);
        }
#pragma unroll
        for (int i0 = 0; i0 < NOC; i0 += 8) {
          float u[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) u[i] = i0 + i < NOC ? v[i0 + i] : 0.f;
          const float t = multi_sum<8>(u, scr, lane);
          const int i = i0 + (lane >> 3), j = wv + 4 * i;
          if ((lane & 7) == 0 && i < NOC) slot_put_dev(P2 + (int64_t)g * D + c * C + j, t, ep + 6);
        }
        mark(s, l, 16);
      }
      // residual += the 8 blocks' c_proj2 partials (blocks in order)
      if (wv == 0 && lane < C) {
        float pv[8];
        if (!slots_wait<8, XPRE, XGAP>(P2 + c * C + lane, D, FUSED_NX, ep + 6, pv, err)) *stop = 1;
        float t = pv[0];
#pragma unroll
        for (int kk = 1; kk < FUSED_NX; ++kk) t += pv[kk];
        x_own = x_own + t;
        slot_put_xcd(XL + c * C + lane, x_own, ep + 7);
      }
      mark(s, l, 17);
      if (comp && !*stop && !gather_slots<(D + 255) / 256>(XL, D, ep + 7, x_lds, tid, err))
        *stop = 1;
      mark(s, l, 18);
      if (TRACE && s == a.trace_step && tid == 0)
        a.trace[((int64_t)b * (L + 1) + l) * 32 + 25] = __builtin_readcyclecounter();
    }
    {
      // lm_head rows of this workgroup (wave w: rows w, w+4, ..., eight at
      // a time; rows below NA in the c_fc region, the others in the q/k/v
      // + c_proj regions) and their first-max argmax candidate
      const uint32_t ep = a.ep_base + (uint32_t)(s * E + 8 * L);
      uint64_t* LMC = S + Sh::OFF_LM + (int64_t)(s & 1) * FUSED_LMC * 2 * FUSED_NWG;
      if (ldA || ldB) vm_wait<0>();
      lds_barrier();  // lm_head's rows have landed
      mark(s, L, 0);
      if (*stop) goto done;
      if (comp) {
        const float inv = 1.0f / sqrtf(sumsq<D>(x_lds, lane) / (float)D + eps);
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        auto roff = [](int r) {
          return r < NA ? (int)Sh::OFF_F + r * D * 2 : (r - NA) * D * 2;
        };
        for (int r0 = wv; r0 < LR; r0 += 32) {
          float acc[8];
          int ro[2][4];
#pragma unroll
          for (int i = 0; i < 8; ++i) ro[i >> 2][i & 3] = roff(min(r0 + 4 * i, LR - 1));  // (rows past LR: ignored)
          {
            float t[4];
            dot_rows<4, D>(lds, ro[0], x_lds, lane, t);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = t[i];
            dot_rows<4, D>(lds, ro[1], x_lds, lane, t);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[4 + i] = t[i];
          }
          const float v = multi_sum<8>(acc, scr, lane) * inv;
          const int r = r0 + 4 * (lane >> 3), id = b * LR + r;
          if ((lane & 7) == 0 && r < LR && a.logits_out) a.logits_out[(int64_t)s * V + id] = v;
#pragma unroll
          for (int qq = 0; qq < 8; ++qq)
            if (r0 + 4 * qq < LR) amax_take(bv, bi, lane_value(v, 8 * qq), b * LR + r0 + 4 * qq);
        }
        if (lane == 0) {
          red[wv] = bv;
          ired[wv] = bi;
        }
        mark(s, L, 1);
      }
      lds_barrier();
      if (s + 1 < a.n_steps) next_step_rows();  // (their regions are free now)
      // the first-max argmax over the 256 candidates, as kern_fused.hip
      if (wv == 0) {
        if (lane < FUSED_LMC) {
          float v = red[0];
          int i = ired[0];
          for (int w = 1; w < 4; ++w) amax_take(v, i, red[w], ired[w]);
          uint64_t* cp = LMC + (int64_t)lane * 2 * FUSED_NWG;
          slot_put_dev(cp + b, v, ep);
          slot_put_dev(cp + FUSED_NWG + b, __int_as_float(i), ep);
        }
        float cv[8];
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        if (slots_wait<8, XPRE, XGAP>(LMC + (int64_t)(b % FUSED_LMC) * 2 * FUSED_NWG + lane, 64, 8,
                                      ep, cv, err)) {
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) amax_take(bv, bi, cv[kk], __float_as_int(cv[4 + kk]));
        } else {
          *stop = 1;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
          const float v2 = __shfl_xor(bv, o, 64);
          const int i2 = __shfl_xor(bi, o, 64);
          amax_take(bv, bi, v2, i2);
        }
        if (lane == 0) {
          red[4] = bv;
          ired[4] = bi;
        }
      }
      mark(s, L, 2);
      lds_barrier();
      mark(s, L, 3);
      if (*stop) goto done;
      if (ldA && s + 1 < a.n_steps) piece(0, 2, 0, NFP);
      int id = ired[4];
      if (id == 0x7fffffff) id = 0;  // no finite candidate: position 1, as the scan starts there
      if (b == 0 && tid == 0) a.ids_out[s] = id;
      if (s + 1 < a.n_steps) embed(id, pos + 1);
    }
  }
done:
  if (ldA || ldB) vm_wait<0>();  // no LDS-DMA may outlive the workgroup
}

}  // namespace

FusedLayout fused_layout_gqa(const Dims& d, const char** why) {
  FusedLayout f;
  auto no = [&](const char* r) {
    if (why) *why = r;
    f.ok = false;
    return f;
  };
  if (d.hd != FUSED_HD) return no("head_dim is not 128");
  if (d.KH != 2 || d.H % 2 != 0) return no("grouped KV heads other than two");
  if (d.dff != 4 * d.D ||
      !((d.D == GqaD20::D && d.H == GqaD20::H && d.V == GqaD20::V) ||
        (d.D == GqaSmall::D && d.H == GqaSmall::H && d.V == GqaSmall::V)))
    return no("no persistent-decode build for these dims (d_model 1280 / 10 heads over 2 KV "
              "heads / vocab 8192, or 512 / 4 / 1024)");
  const bool big = d.D == GqaD20::D;
  f.kind = 1;
  f.max_len = 128 * (big ? GqaD20::NPW : GqaSmall::NPW);  // positions gi + 128 li, li < NPW
  f.C = d.D / FUSED_NC;
  f.FR = d.dff / FUSED_NWG;
  f.HN = d.dff / FUSED_NX;
  f.LR = d.V / FUSED_NWG;
  f.QR = 2 * (big ? GqaD20::QP : GqaSmall::QP);
  f.wq = 0;
  f.wp = big ? GqaD20::AQ : GqaSmall::AQ;
  f.wf = f.wp + (big ? GqaD20::SP : GqaSmall::SP);
  f.w2 = f.wf + (big ? GqaD20::SF : GqaSmall::SF);
  f.slice = big ? GqaD20::SLICE : GqaSmall::SLICE;
  f.lmb = big ? GqaD20::LMB : GqaSmall::LMB;
  f.wbuf = big ? GqaD20::WEND : GqaSmall::WEND;
  f.cu_bytes = (int64_t)d.L * f.slice + f.lmb;
  f.lds_bytes = big ? GqaD20::LDS : GqaSmall::LDS;
  f.off_ql = big ? GqaD20::OFF_QL : GqaSmall::OFF_QL;
  f.off_ap = big ? GqaD20::OFF_AP : GqaSmall::OFF_AP;
  f.off_xp = big ? GqaD20::OFF_XP : GqaSmall::OFF_XP;
  f.off_pp = big ? GqaD20::OFF_PP : GqaSmall::OFF_PP;
  f.off_xl = big ? GqaD20::OFF_XL : GqaSmall::OFF_XL;
  f.off_hl = big ? GqaD20::OFF_HL : GqaSmall::OFF_HL;
  f.off_p2 = big ? GqaD20::OFF_P2 : GqaSmall::OFF_P2;
  f.off_lm = big ? GqaD20::OFF_LM : GqaSmall::OFF_LM;
  f.slots = big ? GqaD20::SLOTS : GqaSmall::SLOTS;
  f.ok = true;
  return f;
}

namespace {

template <class Sh>
void pack_gqa(const Dims& d, const FusedLayout& f, const Weights& w, const bf16_t* hm, bf16_t* hf) {
  constexpr int D = Sh::D, HD = Sh::HD, G = Sh::G, GQ = Sh::GQ, NPR = Sh::NPR;
  const int qd = d.qd(), kd = d.kvd();
  memset(hf, 0, (size_t)FUSED_NWG * f.cu_bytes);
  for (int b = 0; b < FUSED_NWG; ++b) {
    const int g = b % FUSED_NX, c = b / FUSED_NX, k = g >> 2, gi = (g & 3) * FUSED_NC + c;
    const int plo = gi * NPR / 128, phi = (gi + 1) * NPR / 128;
    uint8_t* cu = (uint8_t*)hf + (int64_t)b * f.cu_bytes;
    for (int l = 0; l < d.L; ++l) {
      const bf16_t* base = hm + (size_t)l * w.layer_stride;
      uint8_t* sl = cu + (int64_t)l * Sh::SLICE;
      // q/k/v pairs: stored rows 2j, 2j+1 of the part (dims j, j + hd/2)
      for (int p = plo; p < phi; ++p) {
        const int part = p / (HD / 2), j = p % (HD / 2);
        const int64_t r0 = part < G ? (int64_t)(k * G + part) * HD
                                    : qd + (int64_t)(part - G) * kd + (int64_t)k * HD;
        for (int e = 0; e < 2; ++e)
          memcpy(sl + (int64_t)(2 * (p - plo) + e) * D * 2,
                 base + w.off_qkv + (r0 + 2 * j + e) * D, (size_t)D * 2);
      }
      // c_proj rows gi NPO + r, the group's query columns
      for (int r = 0; r < Sh::NPO; ++r)
        memcpy(sl + Sh::AQ + (int64_t)r * GQ * 2,
               base + w.off_proj + (int64_t)(gi * Sh::NPO + r) * qd + (int64_t)k * GQ,
               (size_t)GQ * 2);
      for (int r = 0; r < Sh::FR; ++r)
        memcpy(sl + Sh::AQ + Sh::SP + (int64_t)r * D * 2,
               base + w.off_fc + ((int64_t)g * Sh::HN + (int64_t)c * Sh::FR + r) * D, (size_t)D * 2);
      for (int j = 0; j < Sh::C; ++j)
        memcpy(sl + Sh::AQ + Sh::SP + Sh::SF + (int64_t)j * Sh::HN * 2,
               base + w.off_proj2 + (int64_t)(c * Sh::C + j) * d.dff + (int64_t)g * Sh::HN,
               (size_t)Sh::HN * 2);
    }
    const bf16_t* lm = hm + (size_t)w.layer_stride * d.L + (int64_t)b * Sh::LR * D;
    uint8_t* ls = cu + (int64_t)d.L * Sh::SLICE;
    memcpy(ls, lm, (size_t)Sh::NA * D * 2);
    if (Sh::LR > Sh::NA)
      memcpy(ls + Sh::SF, lm + (int64_t)Sh::NA * D, (size_t)(Sh::LR - Sh::NA) * D * 2);
  }
}

template <class Sh>
hipError_t launch_gqa(hipStream_t s, const FusedLayout& f, const FusedArgs& a) {
  if (f.slice != Sh::SLICE || f.lmb != Sh::LMB || f.lds_bytes != Sh::LDS ||
      f.off_lm != Sh::OFF_LM || f.off_xp != Sh::OFF_XP || f.slots != Sh::SLOTS)
    return hipErrorInvalidValue;  // (host and device layouts disagree)
  const void* kfn = a.trace ? (const void*)k_fused_gqa<Sh, true> : (const void*)k_fused_gqa<Sh, false>;
  hipError_t e = hipFuncSetAttribute(kfn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)f.lds_bytes);
  if (e != hipSuccess) return e;
  FusedArgs aa = a;
  void* args[] = {&aa};
  return hipLaunchCooperativeKernel(kfn, dim3(FUSED_NWG), dim3(GQA_THREADS), args,
                                    (unsigned)f.lds_bytes, s);
}

}  // namespace

void fused_pack_gqa(const Dims& d, const FusedLayout& f, const Weights& w, const bf16_t* hm,
                    bf16_t* hf) {
  if (d.D == GqaD20::D)
    pack_gqa<GqaD20>(d, f, w, hm, hf);
  else
    pack_gqa<GqaSmall>(d, f, w, hm, hf);
}

hipError_t launch_fused_gqa(hipStream_t s, const Dims& d, const FusedLayout& f,
                            const FusedArgs& a) {
  if (d.D == GqaD20::D && d.H == GqaD20::H && d.V == GqaD20::V) return launch_gqa<GqaD20>(s, f, a);
  if (d.D == GqaSmall::D && d.H == GqaSmall::H && d.V == GqaSmall::V)
    return launch_gqa<GqaSmall>(s, f, a);
  return hipErrorInvalidValue;
}

}  // namespace fgpt
