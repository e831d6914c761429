// kern_fused.hip -- the B=1 greedy decode loop (gpt_step fed back through
// its argmax, src/app/chat_text.f90:423-462 with src/lib/fortran_kv.f90:
// 26-149 per step) as ONE persistent launch on gfx950.
//
// Why one launch: at B=1 every linear of a step is a few MB of weights,
// which a kernel of its own cannot stream faster than its launch and its
// first load take (~3-5 us each, 62 launches a step). Here 256 workgroups,
// one per CU, run the whole loop; the weights of the next pseudo-layer (a
// layer, or lm_head) stream into LDS while the current one computes, so a
// hand-over of activations between workgroups is the only thing on the
// critical path.
//
// Work split (workgroup (g, c): the c-th of the 32 workgroups on XCD g):
//   q/k/v rows of head g (XCD g < H)   12 rows per workgroup (6 RoPE pairs)
//   attention of head g                 every workgroup of XCD g, recomputed
//   c_proj, head g's 128 columns        C = D/32 outputs per workgroup
//   c_fc rows [g*dff/8, (g+1)*dff/8)    dff/256 rows per workgroup
//   c_proj2 columns of that fc block    C outputs per workgroup
//   lm_head rows [b*V/256, (b+1)*V/256)
// The residual columns [c*C, (c+1)*C) are owned (identically, in registers)
// by workgroup (g, c) of every XCD: c_proj's per-head partials and
// c_proj2's per-block partials are added to them in a fixed order.
//
// Hand-overs ("exchange slots", 8 bytes: fp32 value | 32-bit epoch << 32).
// Within one XCD a plain store lands in that XCD's L2, where agent-scope
// (sc1) loads of the other workgroups see it; across XCDs the store is an
// agent-scope (sc1, write-through) store. A reader polls until the slot
// carries the epoch of the hand-over it waits for: every hand-over of a
// launch has its own epoch and the host advances the base across launches,
// so a stale slot is never taken. Every poll is bounded: past the bound the
// workgroup raises the error flag and all workgroups leave, so the grid
// always drains. Per layer: q/k/v within the XCD, (from FUSED_SPLIT_MIN
// positions on) the attention partials of the XCD's workgroups within,
// c_proj partials across, the updated residual within, the fc block
// within, c_proj2 partials across, the residual within; the step ends with
// the lm_head argmax candidates of all 256 workgroups, one hand-over
// across.
//
// Arithmetic per output element: rmsnorm0 (src/lib/fortran_rmsnorm.f90:
// 40-60) as a scale of the dot products, fp32 accumulation of bf16 weights
// times fp32 activations, rope_4d (src/lib/fortran_rope.f90:25-52) on the
// host's tables, attn_step's softmax (src/lib/fortran_attn.f90:317-362) as
// an online softmax over 8 position groups merged in group order, relu2
// (:697-710), residual adds (src/lib/fortran_kv.f90:125-137), and the
// first-max argmax of src/lib/sample.f90:271-277.
#include <float.h>
#include <string.h>

#include <algorithm>

#include "kern_fused.h"

namespace fgpt {

namespace {

// The work split's sizes for one model shape (head_dim 128, d_ff = 4
// d_model); fused_layout computes the same values at run time.
template <int D_, int H_, int V_>
struct FusedShape {
  static constexpr int HD = 128, D = D_, H = H_, V = V_, DFF = 4 * D_;
  static constexpr int QR = 3 * HD / FUSED_NC, C = D / FUSED_NC, FR = DFF / FUSED_NWG;
  static constexpr int HN = DFF / FUSED_NX, LR = V / FUSED_NWG;
  static constexpr int64_t WQ = 0, WP = round1k((int64_t)QR * D * 2);
  static constexpr int64_t WF = WP + round1k((int64_t)C * HD * 2);
  static constexpr int64_t W2 = WF + round1k((int64_t)FR * D * 2);
  static constexpr int64_t SLICE = W2 + round1k((int64_t)C * HN * 2);
  static constexpr int64_t LMB = round1k((int64_t)LR * D * 2);
  static constexpr int64_t WBUF = SLICE > LMB ? SLICE : LMB;
  static constexpr int64_t OFF_QL = 0, OFF_PP = 2 * FUSED_NX * 3 * HD;
  static constexpr int64_t OFF_XL = OFF_PP + 2 * FUSED_NX * D;
  static constexpr int64_t OFF_HL = OFF_XL + 2 * FUSED_NX * D;
  static constexpr int64_t OFF_P2 = OFF_HL + 2 * FUSED_NX * HN;
  static constexpr int64_t OFF_LM = OFF_P2 + 2 * FUSED_NX * D;
  // (the argmax candidates: two step parities x FUSED_LMC copies)
  static constexpr int64_t OFF_AP = OFF_LM + 2 * FUSED_LMC * 2 * FUSED_NWG;
  static constexpr int64_t SLOTS = OFF_AP + 2 * FUSED_NX * FUSED_SPLIT_WG * (HD + 2);
};
// The shapes the persistent decode is built for: depth-12's (d_model 768,
// 6 heads, vocab 8192) and a small one the tests run.
typedef FusedShape<768, 6, 8192> ShapeD12;
typedef FusedShape<256, 2, 1024> ShapeSmall;

template <class Sh, bool TRACE>
__global__ __launch_bounds__(FUSED_THREADS) void k_fused_decode(FusedArgs a) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
  constexpr int HD = Sh::HD;
  constexpr int QLN = 3 * HD;            // q, k, v of one head
  constexpr int NP = QLN / 64;           // rotation pairs per workgroup (6)
  constexpr int LPP = HD / 4;            // lanes per cached row in the attention
  constexpr int NG = 4 * (64 / LPP);     // position groups
  // positions per group, at most: below FUSED_SPLIT_MIN, or (split) of
  // this workgroup's every FUSED_SPLIT_WG-th position
  constexpr int PPG = std::max(FUSED_SPLIT_MIN / NG, FUSED_MAX_LEN / (FUSED_SPLIT_WG * NG));
  constexpr int AST = HD + 4;            // floats per group record: o, m, l
  constexpr int APS = HD + 2;            // slots per workgroup attention partial: o, m, l
  constexpr int AB = 8;                  // attention positions per batch
  static_assert(LPP == 32 && NP == 6, "the work split is laid out for head_dim 128");
  constexpr int D = Sh::D, H = Sh::H, V = Sh::V, KD = Sh::H * HD;
  constexpr int C = Sh::C, FR = Sh::FR, HN = Sh::HN, LR = Sh::LR, QR = Sh::QR;
  const int L = a.L;
  const int64_t cu_bytes = (int64_t)L * Sh::SLICE + Sh::LMB;
  const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
  const bool comp = wv < 4, loader = wv == 4;
  const float eps = a.eps;
  float* x_lds = (float*)(lds + 2 * Sh::WBUF);
  float* h_lds = x_lds + D;
  float* qkv_lds = h_lds + HN;
  float* att = qkv_lds + QLN;   // [NG][AST]
  float* scr0 = att + NG * AST;  // reduction scratch, [4 waves][8][64] (16-byte aligned)
  float* scr = scr0 + (comp ? wv : 0) * 8 * 64;  // this wave's
  float* red = scr0 + 4 * 8 * 64;  // [8]
  int* ired = (int*)(red + 8);  // [8]
  int* stop = ired + 8;         // nonzero: leave (a hand-over failed)
  int* place = stop + 1;        // this workgroup's XCD and its index there
  float* rope = (float*)(place + 2);  // cos, sin of the step's position [2][HD/2]
  // split attention: the XCD's workgroup partials [FUSED_SPLIT_WG][AST], at the
  // first 16-byte boundary past rope (an offset from lds, so LDS accesses)
  constexpr int64_t ROPE_END = 2 * Sh::WBUF + 4 * ((int64_t)D + HN + QLN + NG * AST + 4 * 8 * 64 +
                                                   8 + 8 + 1 + 2 + HD);
  float* apart = (float*)(lds + (ROPE_END + 15) / 16 * 16);
  uint32_t* err = a.err;
  const int E = 8 * L + 8;      // epochs per step
  const int total = a.n_steps * (L + 1);  // pseudo-layers of the launch
  uint64_t* S = a.slots;

  // Placement: the XCD this workgroup runs on (XCC_ID) and its index among
  // that XCD's workgroups, from a per-launch counter (one workgroup per CU,
  // 32 CUs per XCD). Which block index the dispatcher sends to which XCD
  // is not relied on: it varies from launch to launch.
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
  const bool head = g < H;
  // optional phase timestamps (100 MHz device clock) of one step
  auto mark = [&](int s, int l, int k) {
    if (TRACE && s == a.trace_step && tid == (k == 14 || k == 15 ? 256 : 0))
      a.trace[((int64_t)b * (L + 1) + l) * 32 + k] = __builtin_amdgcn_s_memrealtime();
  };
  // DMA of pseudo-layer G's weight slices into its LDS buffer (loader
  // wave), in three parts issued at three barriers of the pseudo-layer
  // before, so the stream into LDS is spread over the whole layer
  auto issue = [&](int G, int part) {
    const int l = G % (L + 1);
    const uint8_t* src = (const uint8_t*)a.arena + (int64_t)b * cu_bytes;
    uint8_t* dst = lds + (G & 1) * Sh::WBUF;
    int64_t off = 0, n;
    if (l < L) {
      off = head ? 0 : Sh::WF;  // workgroups of XCDs >= H hold no q/k/v or c_proj rows
      src += (int64_t)l * Sh::SLICE;
      n = Sh::SLICE - off;
    } else {
      src += (int64_t)L * Sh::SLICE;
      n = Sh::LMB;
    }
    const int64_t nch = n / 1024, k0 = part * nch / 3, k1 = (part + 1) * nch / 3;
    for (int64_t k = off + 1024 * k0; k < off + 1024 * k1; k += 1024)
      dma16(src + k + 16 * lane, lds_off(dst + k));
  };
  auto waitdma = [] { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); };

  // x = rmsnorm0(wte[id]) into x_lds (k_embed_norm's order: 256 strided
  // partial sums, then the four waves' sums in order), x_own = this
  // workgroup's residual columns, and the RoPE row of position pos
  float x_own = 0.f;
  auto embed = [&](int id, int pos) {
    const bf16_t* row = a.wte + (int64_t)id * D;
    if (comp && tid < HD) rope[tid] = tid < HD / 2 ? a.cosb[(int64_t)pos * (HD / 2) + tid]
                                                   : a.sinb[(int64_t)pos * (HD / 2) + tid - HD / 2];
    if (comp) {
      float ss = 0.f;
      for (int k = tid; k < D; k += 256) {
        const float v = bf16_to_f32(row[k]);
        ss += v * v;
      }
      ss = wave_sum(ss);
      if (lane == 0) red[wv] = ss;
    }
    lds_barrier();
    if (comp) {
      const float t = red[0] + red[1] + red[2] + red[3];
      const float inv = 1.0f / sqrtf(t / (float)D + eps);
      for (int k = tid; k < D; k += 256) x_lds[k] = bf16_to_f32(row[k]) * inv;
      if (wv == 0 && lane < C) x_own = bf16_to_f32(row[c * C + lane]) * inv;
    }
  };

  if (loader) {
    issue(0, 0);
    issue(0, 1);
    issue(0, 2);
  }
  embed(*a.d_id0, a.len0);

  for (int s = 0; s < a.n_steps; ++s) {
    const int pos = a.len0 + s;
    for (int l = 0; l <= L; ++l) {
      const int G = s * (L + 1) + l;
      const uint8_t* W = lds + (G & 1) * Sh::WBUF;  // (an LDS address: ds_read, not flat)
      // B0: this pseudo-layer's weights have landed; the next one's go out
      mark(s, l, 14);
      if (loader) waitdma();
      mark(s, l, 15);
      lds_barrier();
      mark(s, l, 0);
      if (TRACE && s == a.trace_step && tid == 0)
        a.trace[((int64_t)b * (L + 1) + l) * 32 + 24] = __builtin_readcyclecounter();
      if (*stop) goto done;
      if (loader && G + 1 < total) issue(G + 1, 0);
      if (l == L) break;  // lm_head below
      const int par = (s * L + l) & 1;
      const uint32_t ep = a.ep_base + (uint32_t)(s * E + l * 8);
      uint64_t* QL = S + Sh::OFF_QL + (int64_t)(par * 8 + g) * QLN;
      uint64_t* PP = S + Sh::OFF_PP + (int64_t)par * 8 * D;
      uint64_t* XL = S + Sh::OFF_XL + (int64_t)(par * 8 + g) * D;
      uint64_t* HL = S + Sh::OFF_HL + (int64_t)(par * 8 + g) * HN;
      uint64_t* P2 = S + Sh::OFF_P2 + (int64_t)par * 8 * D;
      float* kc = a.kc + (int64_t)l * a.maxT * KD + g * HD;
      float* vc = a.vc + (int64_t)l * a.maxT * KD + g * HD;
      if (head) {
        // q, k, v rows of head g: wave w takes RoPE pairs w and w+4 (of 6)
        if (comp) {
          const bool two = wv + 4 < NP;
          // rows 2w, 2w+1 and (when there is a second pair) 2w+8, 2w+9
          const int ro[4] = {2 * wv * D * 2, (2 * wv + 1) * D * 2, (two ? 2 * wv + 8 : 2 * wv) * D * 2,
                             (two ? 2 * wv + 9 : 2 * wv + 1) * D * 2};
          float acc[4];
          dot_rows<4, D>(W + Sh::WQ, ro, x_lds, lane, acc);
          const float inv = 1.0f / sqrtf(sumsq<D>(x_lds, lane) / (float)D + eps);
          const float r4 = multi_sum<4>(acc, scr, lane);
          const float rv[4] = {lane_value(r4, 0) * inv, lane_value(r4, 16) * inv,
                               lane_value(r4, 32) * inv, lane_value(r4, 48) * inv};
          if (lane < (two ? 2 : 1)) {
            const int pi = wv + 4 * lane;
            const float v0 = lane ? rv[2] : rv[0], v1 = lane ? rv[3] : rv[1];
            const int r0 = c * QR + 2 * pi, part = r0 / HD, j = (r0 % HD) >> 1;
            float y1 = v0, y2 = v1;
            if (part < 2) {
              const float cs = rope[j], sn = rope[HD / 2 + j];
              y1 = v0 * cs + v1 * sn;
              y2 = v0 * (-sn) + v1 * cs;
            }
            slot_put_xcd(QL + part * HD + j, y1, ep);
            slot_put_xcd(QL + part * HD + j + HD / 2, y2, ep);
            if (part > 0) {  // (head g's cache rows are written and read by XCD g only)
              float* cr = (part == 1 ? kc : vc) + (int64_t)pos * KD;
              cr[j] = y1;
              cr[j + HD / 2] = y2;
            }
          }
          mark(s, l, 1);
        }
        // attention of head g over positions 0..pos: group grp (half a
        // wave) takes positions grp, grp+NG, ... -- or, from FUSED_SPLIT_MIN
        // positions on, workgroup c < FUSED_SPLIT_WG takes only the
        // positions c, c + FUSED_SPLIT_WG, ... (group grp: c +
        // FUSED_SPLIT_WG (grp + NG i)), the others none, and the partial
        // results are merged after one more hand-over. The current
        // position's k and v come from the hand-over, earlier ones from the
        // cache. The first batch's cache rows are requested before the wait
        // for q/k/v.
        const bool split = pos >= FUSED_SPLIT_MIN;  // (uniform)
        const bool attend = !split || c < FUSED_SPLIT_WG;
        const int grp = wv * 2 + (lane >> 5), dl = lane & 31;
        const int pb = split ? c : 0, ps = split ? FUSED_SPLIT_WG : 1;
        auto posof = [&](int i) { return pb + ps * (grp + NG * i); };
        float4 kr[AB], vr[AB];
        if (comp) {
#pragma unroll
          for (int i = 0; i < AB; ++i) {
            const int p = posof(i);
            if (attend && p < pos) {
              kr[i] = *(const float4*)(kc + (int64_t)p * KD + 4 * dl);
              vr[i] = *(const float4*)(vc + (int64_t)p * KD + 4 * dl);
            }
          }
          if (!gather_slots<2>(QL, QLN, ep, qkv_lds, tid, err)) *stop = 1;
        }
        lds_barrier();  // B1
        mark(s, l, 2);
        if (*stop) goto done;
        if (comp && attend) {
          const float4 q4 = *(const float4*)(qkv_lds + 4 * dl);
          const float scale = 1.0f / sqrtf((float)HD);
          float m = -INFINITY, lsum = 0.f;
          float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 1
          for (int i0 = 0; i0 < PPG && posof(i0) <= pos; i0 += AB) {
#pragma unroll
            for (int i = 0; i < AB; ++i) {
              const int p = posof(i0 + i);
              if (p >= pos) {
                kr[i] = *(const float4*)(qkv_lds + HD + 4 * dl);
                vr[i] = *(const float4*)(qkv_lds + 2 * HD + 4 * dl);
              } else if (i0 > 0) {
                kr[i] = *(const float4*)(kc + (int64_t)p * KD + 4 * dl);
                vr[i] = *(const float4*)(vc + (int64_t)p * KD + 4 * dl);
              }
            }
            // the batch's scores (independent half-wave sums), then one
            // online-softmax update for the batch
            float sc[AB];
            float mb = -INFINITY;
#pragma unroll
            for (int i = 0; i < AB; ++i) {
              const float dp = q4.x * kr[i].x + q4.y * kr[i].y + q4.z * kr[i].z + q4.w * kr[i].w;
              sc[i] = posof(i0 + i) <= pos ? half_sum(dp) * scale : -INFINITY;
              mb = fmaxf(mb, sc[i]);
            }
            const float mn = fmaxf(m, mb), al = __expf(m - mn);
            lsum *= al;
            o.x *= al;
            o.y *= al;
            o.z *= al;
            o.w *= al;
#pragma unroll
            for (int i = 0; i < AB; ++i) {
              const float e = __expf(sc[i] - mn);
              lsum += e;
              o.x += e * vr[i].x;
              o.y += e * vr[i].y;
              o.z += e * vr[i].z;
              o.w += e * vr[i].w;
            }
            m = mn;
          }
          *(float4*)(att + grp * AST + 4 * dl) = o;
          if (dl == 0) {
            att[grp * AST + HD] = m;
            att[grp * AST + HD + 1] = lsum;
          }
        }
        lds_barrier();  // B2
        mark(s, l, 3);
        // the groups' records merged in group order: this lane's head dims
        // 2*lane, 2*lane+1 (o0, o1, unnormalised), the maximum and the sum
        float mx = -INFINITY, ls = 0.f, o0 = 0.f, o1 = 0.f;
        if (comp && attend) {
#pragma unroll
          for (int q = 0; q < NG; ++q) mx = fmaxf(mx, att[q * AST + HD]);
#pragma unroll
          for (int q = 0; q < NG; ++q) {
            const float w = __expf(att[q * AST + HD] - mx);
            ls += att[q * AST + HD + 1] * w;
            o0 += att[q * AST + 2 * lane] * w;
            o1 += att[q * AST + 2 * lane + 1] * w;
          }
        }
        if (split) {
          // this workgroup's partial to the XCD (wave 0), then every
          // workgroup merges the FUSED_SPLIT_WG partials in workgroup order
          uint64_t* AP = S + Sh::OFF_AP + (int64_t)(par * 8 + g) * FUSED_SPLIT_WG * APS;
          if (wv == 0 && attend) {
            slot_put_xcd(AP + (int64_t)c * APS + 2 * lane, o0, ep + 6);
            slot_put_xcd(AP + (int64_t)c * APS + 2 * lane + 1, o1, ep + 6);
            if (lane == 0) {
              slot_put_xcd(AP + (int64_t)c * APS + HD, mx, ep + 6);
              slot_put_xcd(AP + (int64_t)c * APS + HD + 1, ls, ep + 6);
            }
          }
          if (comp) {
            // slot j = w * APS + e of the FUSED_SPLIT_WG x APS lands at
            // apart[w * AST + e]
            constexpr int NJ = (FUSED_SPLIT_WG * APS + 255) / 256;
            float v[NJ];
            const int cnt = (FUSED_SPLIT_WG * APS - tid + 255) / 256;
            if (!slots_wait<NJ>(AP + tid, 256, cnt, ep + 6, v, err)) *stop = 1;
#pragma unroll
            for (int i = 0; i < NJ; ++i)
              if (i < cnt) {
                const int j = tid + 256 * i;
                apart[(j / APS) * AST + j % APS] = v[i];
              }
          }
          lds_barrier();  // B2s
          mark(s, l, 12);
          if (*stop) goto done;
          mx = -INFINITY;
          ls = o0 = o1 = 0.f;
          if (comp) {
#pragma unroll
            for (int w = 0; w < FUSED_SPLIT_WG; ++w) mx = fmaxf(mx, apart[w * AST + HD]);
#pragma unroll
            for (int w = 0; w < FUSED_SPLIT_WG; ++w) {
              const float e = __expf(apart[w * AST + HD] - mx);
              ls += apart[w * AST + HD + 1] * e;
              o0 += apart[w * AST + 2 * lane] * e;
              o1 += apart[w * AST + 2 * lane + 1] * e;
            }
          }
        }
        // c_proj partial of head g over this workgroup's C output columns:
        // wave w takes outputs w, w+4, ...
        if (comp) {
          const float il = 1.0f / ls;
          const float ao0 = o0 * il, ao1 = o1 * il;  // head dims 2*lane, 2*lane+1
          for (int j0 = wv; j0 < C; j0 += 32) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const int j = min(j0 + 4 * i, C - 1);
              const uint32_t wp = *(const uint32_t*)(W + Sh::WP + (int64_t)j * HD * 2 + 4 * lane);
              v[i] = ao0 * __uint_as_float(wp << 16) + ao1 * __uint_as_float(wp & 0xFFFF0000u);
            }
            const float t = multi_sum<8>(v, scr, lane);
            const int j = j0 + 4 * (lane >> 3);
            if ((lane & 7) == 0 && j < C) slot_put_dev(PP + (int64_t)g * D + c * C + j, t, ep + 1);
          }
          mark(s, l, 4);
        }
      }
      // residual += sum of the heads' c_proj partials (heads in order)
      if (wv == 0 && lane < C) {
        float pv[8];
        if (!slots_wait<8>(PP + c * C + lane, D, H, ep + 1, pv, err)) *stop = 1;
        float t = pv[0];
        for (int h = 1; h < H; ++h) t += pv[h];
        x_own = x_own + t;
        slot_put_xcd(XL + c * C + lane, x_own, ep + 2);
      }
      mark(s, l, 5);
      if (comp && !*stop && !gather_slots<8>(XL, D, ep + 2, x_lds, tid, err)) *stop = 1;
      lds_barrier();  // B3
      mark(s, l, 6);
      if (*stop) goto done;
      if (loader && G + 1 < total) issue(G + 1, 1);
      // h = relu2(rmsnorm0(x) c_fc^T) for this workgroup's fc rows: wave w
      // takes rows w, w+4, ... (four at a time)
      if (comp) {
        const float inv = 1.0f / sqrtf(sumsq<D>(x_lds, lane) / (float)D + eps);
        for (int r0 = wv; r0 < FR; r0 += 16) {
          float acc[4];
          int ro[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) ro[i] = min(r0 + 4 * i, FR - 1) * D * 2;  // (rows past FR: ignored)
          dot_rows<4, D>(W + Sh::WF, ro, x_lds, lane, acc);
          float t = multi_sum<4>(acc, scr, lane) * inv;
          t = t < 0.f ? 0.f : t;
          const int r = r0 + 4 * (lane >> 4);
          if ((lane & 15) == 0 && r < FR) slot_put_xcd(HL + c * FR + r, t * t, ep + 3);
        }
        mark(s, l, 7);
        if (!gather_slots<8>(HL, HN, ep + 3, h_lds, tid, err)) *stop = 1;
      }
      lds_barrier();  // B4
      mark(s, l, 8);
      if (*stop) goto done;
      if (loader && G + 1 < total) issue(G + 1, 2);
      // c_proj2 partial over this XCD's fc block: wave w takes outputs w,
      // w+4, ... (eight at a time)
      if (comp) {
        for (int j0 = wv; j0 < C; j0 += 32) {
          float v[8];
          int ro[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) ro[i] = min(j0 + 4 * i, C - 1) * HN * 2;  // (outputs past C: ignored)
          dot_rows<8, HN>(W + Sh::W2, ro, h_lds, lane, v);
          const float t = multi_sum<8>(v, scr, lane);
          const int j = j0 + 4 * (lane >> 3);
          if ((lane & 7) == 0 && j < C) slot_put_dev(P2 + (int64_t)g * D + c * C + j, t, ep + 4);
        }
        mark(s, l, 9);
      }
      // residual += sum of the 8 blocks' c_proj2 partials (blocks in order)
      if (wv == 0 && lane < C) {
        float pv[8];
        if (!slots_wait<8>(P2 + c * C + lane, D, FUSED_NX, ep + 4, pv, err)) *stop = 1;
        float t = pv[0];
#pragma unroll
        for (int k = 1; k < FUSED_NX; ++k) t += pv[k];
        x_own = x_own + t;
        slot_put_xcd(XL + c * C + lane, x_own, ep + 5);
      }
      mark(s, l, 10);
      if (comp && !*stop && !gather_slots<8>(XL, D, ep + 5, x_lds, tid, err)) *stop = 1;
      mark(s, l, 11);
      if (TRACE && s == a.trace_step && tid == 0)
        a.trace[((int64_t)b * (L + 1) + l) * 32 + 25] = __builtin_readcyclecounter();
    }
    {
      // lm_head rows of this workgroup (wave w: rows w, w+4, ..., eight at
      // a time) and their first-max argmax candidate
      const int G = s * (L + 1) + L;
      const uint8_t* W = lds + (G & 1) * Sh::WBUF;
      const uint32_t ep = a.ep_base + (uint32_t)(s * E + 8 * L);
      // argmax candidates of the 256 workgroups, [2][256][2] (value, index)
      uint64_t* LMC = S + Sh::OFF_LM + (int64_t)(s & 1) * FUSED_LMC * 2 * FUSED_NWG;
      if (comp) {
        const float inv = 1.0f / sqrtf(sumsq<D>(x_lds, lane) / (float)D + eps);
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        for (int r0 = wv; r0 < LR; r0 += 32) {
          float acc[8];
          int ro[2][4];
#pragma unroll
          for (int i = 0; i < 8; ++i) ro[i >> 2][i & 3] = min(r0 + 4 * i, LR - 1) * D * 2;  // (rows past LR: ignored)
          {
            float t[4];
            dot_rows<4, D>(W, ro[0], x_lds, lane, t);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = t[i];
            dot_rows<4, D>(W, ro[1], x_lds, lane, t);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[4 + i] = t[i];
          }
          const float v = multi_sum<8>(acc, scr, lane) * inv;
          const int r = r0 + 4 * (lane >> 3), id = b * LR + r;
          if ((lane & 7) == 0 && r < LR && a.logits_out) a.logits_out[(int64_t)s * V + id] = v;
          // rows in increasing order across the eight groups
#pragma unroll
          for (int q = 0; q < 8; ++q)
            if (r0 + 4 * q < LR) amax_take(bv, bi, lane_value(v, 8 * q), b * LR + r0 + 4 * q);
        }
        if (lane == 0) {
          red[wv] = bv;
          ired[wv] = bi;
        }
        mark(s, L, 1);
      }
      lds_barrier();  // B5
      if (loader && G + 1 < total) issue(G + 1, 1);
      // the first-max argmax over all 256 candidates in one hand-over
      // across XCDs: every workgroup publishes its candidate (value in
      // slot b, index in slot 256 + b) into FUSED_LMC copies (lane k of
      // wave 0 writes copy k), and reads all 256 from copy b % FUSED_LMC
      // (wave 0: four candidates a lane, values and indices in one wait),
      // so the 256 readers are spread over FUSED_LMC regions; every
      // workgroup reduces them alike
      if (wv == 0) {
        if (lane < FUSED_LMC) {
          float v = red[0];
          int i = ired[0];
          for (int w = 1; w < 4; ++w) amax_take(v, i, red[w], ired[w]);
          uint64_t* cp = LMC + (int64_t)lane * 2 * FUSED_NWG;
          slot_put_dev(cp + b, v, ep);
          slot_put_dev(cp + FUSED_NWG + b, __int_as_float(i), ep);
        }
        float cv[8];  // candidates lane + 64 k: values (k < 4), then their indices
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        if (slots_wait<8>(LMC + (int64_t)(b % FUSED_LMC) * 2 * FUSED_NWG + lane, 64, 8, ep, cv,
                          err)) {
#pragma unroll
          for (int k = 0; k < 4; ++k) amax_take(bv, bi, cv[k], __float_as_int(cv[4 + k]));
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
      lds_barrier();  // B6
      mark(s, L, 3);
      if (*stop) goto done;
      if (loader && G + 1 < total) issue(G + 1, 2);
      int id = ired[4];
      if (id == 0x7fffffff) id = 0;  // no finite candidate: position 1, as the scan starts there
      if (b == 0 && tid == 0) a.ids_out[s] = id;
      if (s + 1 < a.n_steps) embed(id, pos + 1);
    }
  }
done:
  if (loader) waitdma();  // no LDS-DMA may outlive the workgroup
}

}  // namespace

FusedLayout fused_layout(const Dims& d, const char** why) {
  FusedLayout f;
  auto no = [&](const char* r) {
    if (why) *why = r;
    f.ok = false;
    return f;
  };
  if (d.KH != d.H) return fused_layout_gqa(d, why);
  if (d.hd != FUSED_HD) return no("head_dim is not 128");
  if (d.H > FUSED_NX) return no("more heads than XCDs");
  if (d.D % FUSED_NC != 0 || d.D / FUSED_NC > 64) return no("d_model not a multiple of 32 up to 2048");
  if (d.dff % (FUSED_NWG * 2) != 0) return no("d_ff not a multiple of 512");
  if (d.V % FUSED_NWG != 0) return no("vocab not a multiple of 256");
  if (d.D > 8 * 256 || d.dff / FUSED_NX > 8 * 256) return no("d_model or d_ff too large");
  if (d.dff != 4 * d.D || !((d.D == ShapeD12::D && d.H == ShapeD12::H && d.V == ShapeD12::V) ||
                            (d.D == ShapeSmall::D && d.H == ShapeSmall::H && d.V == ShapeSmall::V)))
    return no("no persistent-decode build for these dims (d_model 768 / 6 heads / vocab 8192, "
              "or 256 / 2 / 1024)");
  auto r1k = [](int64_t x) { return (x + 1023) / 1024 * 1024; };
  f.QR = 3 * d.hd / FUSED_NC;
  f.C = d.D / FUSED_NC;
  f.FR = d.dff / FUSED_NWG;
  f.HN = d.dff / FUSED_NX;
  f.LR = d.V / FUSED_NWG;
  f.wq = 0;
  f.wp = r1k((int64_t)f.QR * d.D * 2);
  f.wf = f.wp + r1k((int64_t)f.C * d.hd * 2);
  f.w2 = f.wf + r1k((int64_t)f.FR * d.D * 2);
  f.slice = f.w2 + r1k((int64_t)f.C * f.HN * 2);
  f.lmb = r1k((int64_t)f.LR * d.D * 2);
  f.wbuf = std::max(f.slice, f.lmb);
  f.cu_bytes = (int64_t)d.L * f.slice + f.lmb;
  const int NG = 4 * (64 / (FUSED_HD / 4));
  // x, h, q/k/v, attention groups, reduction scratch, red, ired, stop,
  // place, rope (floats / ints)
  const int64_t act = 4 * ((int64_t)d.D + f.HN + 3 * FUSED_HD + NG * (FUSED_HD + 4) + 4 * 8 * 64 +
                           8 + 8 + 1 + 2 + FUSED_HD);
  // then the split attention's partials [FUSED_SPLIT_WG][hd + 4] on a
  // 16-byte boundary
  f.lds_bytes = (2 * f.wbuf + act + 15) / 16 * 16 + 4 * (int64_t)FUSED_SPLIT_WG * (FUSED_HD + 4);
  if (f.lds_bytes > 160 * 1024) return no("weight slices do not fit twice in LDS");
  f.off_ql = 0;
  f.off_pp = f.off_ql + 2 * FUSED_NX * 3 * (int64_t)d.hd;
  f.off_xl = f.off_pp + 2 * FUSED_NX * (int64_t)d.D;
  f.off_hl = f.off_xl + 2 * FUSED_NX * (int64_t)d.D;
  f.off_p2 = f.off_hl + 2 * FUSED_NX * (int64_t)f.HN;
  f.off_lm = f.off_p2 + 2 * FUSED_NX * (int64_t)d.D;
  f.off_ap = f.off_lm + 2 * FUSED_LMC * 2 * (int64_t)FUSED_NWG;
  f.slots = f.off_ap + 2 * FUSED_NX * FUSED_SPLIT_WG * (int64_t)(d.hd + 2);
  f.ok = true;
  return f;
}

void fused_pack(const Dims& d, const FusedLayout& f, const Weights& w, const bf16_t* hm,
                bf16_t* hf) {
  if (f.kind == 1) return fused_pack_gqa(d, f, w, hm, hf);
  const int D = d.D, hd = d.hd, H = d.H, qd = d.qd(), kd = d.kvd();
  memset(hf, 0, (size_t)FUSED_NWG * f.cu_bytes);
  for (int b = 0; b < FUSED_NWG; ++b) {
    const int g = b % FUSED_NX, c = b / FUSED_NX;
    uint8_t* cu = (uint8_t*)hf + (int64_t)b * f.cu_bytes;
    for (int l = 0; l < d.L; ++l) {
      const bf16_t* base = hm + (size_t)l * w.layer_stride;
      bf16_t* sl = (bf16_t*)(cu + (int64_t)l * f.slice);
      if (g < H) {
        // head g's rows in [q | k | v] order, each part pair-interleaved
        // as the main arena stores it
        for (int i = 0; i < f.QR; ++i) {
          const int r = c * f.QR + i, part = r / hd, s = r % hd;
          const int64_t src_row = part == 0 ? (int64_t)g * hd + s
                                            : qd + (int64_t)(part - 1) * kd + (int64_t)g * hd + s;
          memcpy(sl + f.wq / 2 + (int64_t)i * D, base + w.off_qkv + src_row * D, (size_t)D * 2);
        }
        // c_proj rows c*C .. c*C+C-1, head g's columns
        for (int j = 0; j < f.C; ++j)
          memcpy(sl + f.wp / 2 + (int64_t)j * hd,
                 base + w.off_proj + (int64_t)(c * f.C + j) * qd + (int64_t)g * hd, (size_t)hd * 2);
      }
      for (int r = 0; r < f.FR; ++r)
        memcpy(sl + f.wf / 2 + (int64_t)r * D,
               base + w.off_fc + ((int64_t)g * f.HN + (int64_t)c * f.FR + r) * D, (size_t)D * 2);
      for (int j = 0; j < f.C; ++j)
        memcpy(sl + f.w2 / 2 + (int64_t)j * f.HN,
               base + w.off_proj2 + (int64_t)(c * f.C + j) * d.dff + (int64_t)g * f.HN,
               (size_t)f.HN * 2);
    }
    const bf16_t* lm = hm + (size_t)w.layer_stride * d.L;
    memcpy(cu + (int64_t)d.L * f.slice, lm + (int64_t)b * f.LR * D, (size_t)f.LR * D * 2);
  }
}

uint32_t fused_epochs(const Dims& d, int n_steps) { return (uint32_t)n_steps * (8u * d.L + 8u); }

template <class Sh>
static hipError_t launch_shape(hipStream_t s, const FusedLayout& f, const FusedArgs& a) {
  if (f.slice != Sh::SLICE || f.lmb != Sh::LMB || f.wbuf != Sh::WBUF || f.wf != Sh::WF ||
      f.off_lm != Sh::OFF_LM || f.off_ap != Sh::OFF_AP || f.slots != Sh::SLOTS)
    return hipErrorInvalidValue;  // (host and device layouts disagree)
  const void* k = a.trace ? (const void*)k_fused_decode<Sh, true> : (const void*)k_fused_decode<Sh, false>;
  hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)f.lds_bytes);
  if (e != hipSuccess) return e;
  FusedArgs aa = a;
  void* args[] = {&aa};
  return hipLaunchCooperativeKernel(k, dim3(FUSED_NWG), dim3(FUSED_THREADS), args,
                                    (unsigned)f.lds_bytes, s);
}

hipError_t launch_fused_decode(hipStream_t s, const Dims& d, const FusedLayout& f,
                               const FusedArgs& a) {
  if (f.kind == 1) return launch_fused_gqa(s, d, f, a);
  if (d.D == ShapeD12::D && d.H == ShapeD12::H && d.V == ShapeD12::V)
    return launch_shape<ShapeD12>(s, f, a);
  if (d.D == ShapeSmall::D && d.H == ShapeSmall::H && d.V == ShapeSmall::V)
    return launch_shape<ShapeSmall>(s, f, a);
  return hipErrorInvalidValue;
}

}  // namespace fgpt
