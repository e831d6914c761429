// fgpt_engine.hip -- the C ABI of include/fgpt.h: model upload, workspace,
// RoPE tables, KV caches and the orchestration of the gfx950 kernels for
// gpt_forward / gpt_step / gpt_step_multi (14NGiestas/autoresearch
// src/lib/fortran_gpt.f90:54-199, src/lib/fortran_kv.f90:26-289).
#include <stdarg.h>
#include <stddef.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <atomic>
#include <condition_variable>
#include <map>
#include <mutex>
#include <string>
#include <system_error>
#include <thread>
#include <vector>

#include <unistd.h>

#include "../../include/fgpt.h"
#include "fgpt_internal.h"

using namespace fgpt;

// ------------------------------------------------------------------ errors
static thread_local int32_t g_err_code = FG_OK;
static thread_local char g_err_msg[512] = "";

static int32_t seterr(int32_t code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err_msg, sizeof g_err_msg, fmt, ap);
  va_end(ap);
  g_err_code = code;
  return code;
}

int32_t fgpt::set_error(int32_t code, const char* msg) { return seterr(code, "%s", msg); }

#define HIPCHK(x)                                                                   \
  do {                                                                              \
    hipError_t e_ = (x);                                                            \
    if (e_ != hipSuccess) return seterr(FG_EHIP, "%s: %s", #x, hipGetErrorString(e_)); \
  } while (0)

#define RCCHK(x)                   \
  do {                             \
    int32_t r_ = (x);              \
    if (r_ != FG_OK) return r_;    \
  } while (0)

extern "C" int32_t fg_version(void) { return 101; }

extern "C" int32_t fg_last_error(char* buf, int32_t len) {
  if (buf && len > 0) {
    strncpy(buf, g_err_msg, (size_t)len - 1);
    buf[len - 1] = '\0';
  }
  return g_err_code;
}

// ------------------------------------------------------------------ handles
struct fg_model {
  Dims d{};
  int device = 0;
  hipStream_t stream = nullptr;
  Weights w;
  float* d_cos = nullptr;
  float* d_sin = nullptr;
  int rope_cap = 0, rope_n = 0;
  Work ws;
  // bf16 hi/lo planes for the MFMA chunk attention: q [rows][qd], and
  // k / v^T for up to split_kv_elems elements per plane
  uint16_t* qs = nullptr;
  uint16_t* ks = nullptr;
  uint16_t* vt = nullptr;
  int64_t split_kv_elems = 0;
  // partial results of the chunk attention
  float* attn_part = nullptr;
  int64_t attn_floats = 0;
  // fg_sample's device copies (logits row, history, state, id), grown on use
  char* samp = nullptr;
  int64_t samp_bytes = 0;
  int64_t work_bytes = 0;
  int64_t gen = 0;      // bumped whenever a buffer a captured graph uses moves
  std::atomic<int> busy{0};
  // per-launch HIP-event timing (fg_timing): off unless asked for
  bool timing = false;
  struct TRec {
    int kind;
    hipEvent_t a, b;
    double flops, bytes;
  };
  std::vector<TRec> trecs;
  std::vector<hipEvent_t> evpool;
  // the persistent B=1 greedy decode (kern_fused.hip): its weight copy,
  // exchange slots, error flag and the next launch's first epoch
  FusedLayout fl;
  bf16_t* fused_w = nullptr;
  uint64_t* fused_slots = nullptr;
  uint32_t* fused_err = nullptr;
  uint32_t fused_ep = 1;
  bool fused_on = true;  // fg_set_option(FG_OPT_FUSED_DECODE)
  // FG_OPT_FORWARD_F16: the fp16 copy of the GEMM weights (the bf16 arena's
  // layout, each value times w16_scale, a power of 2; wte unused), made on
  // first use; w16_inv = 1 / w16_scale; wmax = max |w| of those weights
  bool fwd_f16 = false;
  uint16_t* w16 = nullptr;
  float w16_scale = 1.f, w16_inv = 1.f, wmax = 0.f;
  std::string fused_why = "not set up";
  // the single-term fp16 passes' overflow flag (device, one word): set by
  // an epilogue whose fp16 store would round to inf (FG_ERANGE)
  uint32_t* d_ovf = nullptr;
  // fg_forward_pos's per-item positive-score counts (device), grown on use
  uint32_t* d_pos = nullptr;
  int64_t pos_cap = 0;
  // two pinned staging buffers (and their events) for large copies to the
  // caller's host memory, made on first use (copy_out)
  void* pin[2] = {nullptr, nullptr};
  hipEvent_t pin_ev[2] = {nullptr, nullptr};
};

struct fg_kv {
  fg_model* m = nullptr;
  int B = 0, maxT = 0, len = 0;
  int filled = 0;  // positions this cache has computed (high-water mark of len)
  float* k = nullptr;  // [L][B][maxT][KH*hd], fp32 or (kv16) bf16 elements
  float* v = nullptr;
  bool kv16 = false;
  int32_t* d_len = nullptr;  // device copy of len for replayed steps; d_len[1] = len at
                             // the start of the current fg_decode_greedy call
  int32_t* d_ids = nullptr;  // [B] ids fed to the next step
  int32_t* d_out = nullptr;  // [cap_out] greedy ids
  int64_t cap_out = 0;
  float* d_lgs = nullptr;    // [cap_lgs] per-step logits of fg_decode_greedy
  float* d_part = nullptr;   // per-chunk partials of the single-query attention
  // its arrival counters, max(B, GEMV_MAX_ROWS) * H, zero between launches
  // (every row count this cache is stepped with: greedy, sampling, spec)
  uint32_t* d_dcnt = nullptr;
  int64_t cap_lgs = 0;
  // greedy speculative decoding (fg_decode_spec): the loop's device state
  // and its pinned host mirror, the sequence's ids [maxT], and the
  // single-query attention partials of up to GEMV_MAX_ROWS rows
  SpecDev* d_sst = nullptr;
  SpecDev* h_sst = nullptr;
  // the sampling loop's device state and pinned mirror (fg_decode_sample)
  SampleDev* d_smp = nullptr;
  SampleDev* h_smp = nullptr;
  int32_t* d_sids = nullptr;  // [maxT] the sequence's ids (speculative and sampling loops)
  float* d_spart = nullptr;
  // captured runs of greedy steps keyed by (steps, with_logits), and runs
  // of speculative rounds keyed by (rounds, 100 + rows per pass); valid for gen
  std::map<std::pair<int, int>, hipGraphExec_t> graphs;
  int64_t graphs_gen = -1;
};

namespace {

struct Guard {
  std::atomic<int>* f;
  bool ok;
  explicit Guard(fg_model* m) : f(&m->busy) {
    int z = 0;
    ok = f->compare_exchange_strong(z, 1);
  }
  ~Guard() {
    if (ok) f->store(0);
  }
};

#define GUARD(m)                                                                  \
  Guard guard_(m);                                                                \
  if (!guard_.ok) return seterr(FG_EBUSY, "handle in use by another thread");     \
  HIPCHK(hipSetDevice((m)->device))

hipEvent_t get_event(fg_model* m) {
  if (!m->evpool.empty()) {
    hipEvent_t e = m->evpool.back();
    m->evpool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  (void)hipEventCreate(&e);
  return e;
}

// Launch f on s; with timing on, bracket it with events and keep the
// algorithmic flops / bytes of the launch for fg_timing_read.
template <class F>
void timed(fg_model* m, hipStream_t s, int kind, double flops, double bytes, F&& f) {
  (void)s;
  if (!m->timing) {
    f();
    return;
  }
  hipEvent_t a = get_event(m), b = get_event(m);
  LaunchEvents& e = launch_events();
  e = LaunchEvents{a, b, 0};
  f();  // its kernels record a (the first) and b (each) in their dispatch
  const int n = e.n;
  e = LaunchEvents{};
  if (n > 0) {
    m->trecs.push_back({kind, a, b, flops, bytes});
  } else {
    m->evpool.push_back(a);
    m->evpool.push_back(b);
  }
}

// The same for a launch that cannot carry events (the cooperative launch):
// events recorded on the stream around it.
template <class F>
void timed_stream(fg_model* m, hipStream_t s, int kind, double flops, double bytes, F&& f) {
  if (!m->timing) {
    f();
    return;
  }
  hipEvent_t a = get_event(m), b = get_event(m);
  (void)hipEventRecord(a, s);
  f();
  (void)hipEventRecord(b, s);
  m->trecs.push_back({kind, a, b, flops, bytes});
}

int32_t check_device(int* dev_out) {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n < 1) return seterr(FG_ENODEV, "no HIP device visible");
  int dev = 0;
  HIPCHK(hipGetDevice(&dev));
  hipDeviceProp_t p;
  HIPCHK(hipGetDeviceProperties(&p, dev));
  if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
    return seterr(FG_ENODEV, "device %d is %s, this build targets gfx950", dev, p.gcnArchName);
  *dev_out = dev;
  return FG_OK;
}

// Initialisation and uploads are queued on the handle's own stream, never on
// the null stream. The handle's stream is non-blocking, so nothing orders
// null-stream work (plain hipMemset / hipMemcpy) against it, and a plain
// hipMemset of device memory may return before the fill has run: a clear
// queued there can land after the handle's first kernels have written the
// buffer. (A new fp32 KV cache is ~7 GB of clearing at the B=64 batched
// decode shape; the split key/value planes cleared behind it were zeroed
// again after the prompt's first QKV tiles had written them, and the
// sequences whose rows those tiles hold left the reference's greedy ids.)
// Every buffer the engine allocates starts zeroed through here, so no read
// of an unwritten element can depend on what the memory held before.
int32_t dev_zero(fg_model* m, void* p, size_t bytes) {
  if (p && bytes) HIPCHK(hipMemsetAsync(p, 0, bytes, m->stream));
  return FG_OK;
}

// Host -> device (or device -> device) copy on the handle's stream, complete
// on return (the source may be released afterwards).
int32_t dev_copy(fg_model* m, void* dst, const void* src, size_t bytes, hipMemcpyKind kind) {
  if (!bytes) return FG_OK;
  HIPCHK(hipMemcpyAsync(dst, src, bytes, kind, m->stream));
  HIPCHK(hipStreamSynchronize(m->stream));
  return FG_OK;
}

// Before a buffer the handle owns is freed or replaced: every stream may
// still have work reading it (the device-pointer entry points run on the
// caller's stream), so wait for the whole device.
int32_t quiesce(fg_model* m) {
  HIPCHK(hipStreamSynchronize(m->stream));
  HIPCHK(hipDeviceSynchronize());
  return FG_OK;
}

}  // namespace

int32_t fgpt::check_dims(const fg_dims* in, Dims* d) {
  if (!in) return seterr(FG_EARG, "dims is NULL");
  d->L = in->n_layer;
  d->D = in->d_model;
  d->H = in->n_head;
  d->KH = in->n_kv_head;
  d->hd = in->head_dim;
  d->V = in->vocab_size;
  d->dff = 4 * in->d_model;
  d->eps = in->eps;
  if (d->L < 1 || d->D < 1 || d->H < 1 || d->KH < 1 || d->V < 1)
    return seterr(FG_EDIMS, "dims must be positive");
  if (d->hd != 64 && d->hd != 128)
    return seterr(FG_EDIMS, "head_dim %d unsupported (64 or 128)", d->hd);
  if (d->H * d->hd != d->D)
    return seterr(FG_EDIMS, "n_head*head_dim (%d) must equal d_model (%d)", d->H * d->hd, d->D);
  if (d->H % d->KH != 0) return seterr(FG_EDIMS, "n_head %% n_kv_head != 0");
  if (d->D % 128 != 0) return seterr(FG_EDIMS, "d_model %d not a multiple of 128", d->D);
  if (d->V % 64 != 0) return seterr(FG_EDIMS, "vocab %d not a multiple of 64", d->V);
  if (!(d->eps > 0.f)) return seterr(FG_EDIMS, "eps must be > 0");
  return FG_OK;
}

namespace {

// fp32 -> bf16 bits, refusing values that are not exactly representable.
int32_t to_bf16_exact(const float* src, size_t n, bf16_t* dst, const char* name) {
  for (size_t i = 0; i < n; ++i) {
    uint32_t u;
    memcpy(&u, &src[i], 4);
    if ((u & 0xFFFFu) != 0)
      return seterr(FG_EWEIGHT, "%s[%zu] = %.9g is not bf16-representable", name, i, src[i]);
    dst[i] = (bf16_t)(u >> 16);
  }
  return FG_OK;
}

// The persistent decode serves B=1 greedy loops when the dims fit its work
// split and the device is the one it is laid out for: 256 CUs (8 XCDs of
// 32) and cooperative launches. When it does not, fg_decode_greedy keeps the
// captured per-kernel steps.
int32_t setup_fused(fg_model* m, const bf16_t* host_main) {
  const char* why = nullptr;
  m->fl = fused_layout(m->d, &why);
  if (!m->fl.ok) {
    m->fused_why = why;
    return FG_OK;
  }
  hipDeviceProp_t p;
  HIPCHK(hipGetDeviceProperties(&p, m->device));
  if (p.multiProcessorCount != FUSED_NWG || !p.cooperativeLaunch) {
    m->fused_why = "device is not a 256-CU part with cooperative launch";
    return FG_OK;
  }
  if (p.sharedMemPerBlock < (size_t)m->fl.lds_bytes && p.maxSharedMemoryPerMultiProcessor <
                                                            (size_t)m->fl.lds_bytes) {
    m->fused_why = "not enough LDS per workgroup";
    return FG_OK;
  }
  std::vector<bf16_t> hf((size_t)FUSED_NWG * m->fl.cu_bytes / 2);
  fused_pack(m->d, m->fl, m->w, host_main, hf.data());
  HIPCHK(hipMalloc((void**)&m->fused_w, hf.size() * 2));
  HIPCHK(hipMalloc((void**)&m->fused_slots, (size_t)m->fl.slots * 8));
  HIPCHK(hipMalloc((void**)&m->fused_err, 4 * (1 + FUSED_NX)));
  RCCHK(dev_zero(m, m->fused_slots, (size_t)m->fl.slots * 8));
  RCCHK(dev_zero(m, m->fused_err, 4 * (1 + FUSED_NX)));
  RCCHK(dev_copy(m, m->fused_w, hf.data(), hf.size() * 2, hipMemcpyHostToDevice));
  m->fused_ep = 1;
  m->fused_why = "";
  return FG_OK;
}

int32_t upload_weights(fg_model* m, const float* const st[8]) {
  const Dims& d = m->d;
  static const char* names[8] = {"wte", "c_q", "c_k", "c_v", "c_proj", "c_fc", "c_proj2", "lm_head"};
  for (int i = 0; i < 8; ++i)
    if (!st[i]) return seterr(FG_EARG, "weight buffer %s is NULL", names[i]);
  const size_t D = d.D, qd = d.qd(), kd = d.kvd(), dff = d.dff, V = d.V;
  Weights& w = m->w;
  w.off_qkv = 0;
  w.off_proj = (size_t)d.nqkv() * D;
  w.off_fc = w.off_proj + D * qd;
  w.off_proj2 = w.off_fc + dff * D;
  w.layer_stride = w.off_proj2 + D * dff;
  const size_t n_total = w.layer_stride * d.L + 2 * V * D;
  std::vector<bf16_t> h(n_total);
  for (int l = 0; l < d.L; ++l) {
    bf16_t* dst = h.data() + (size_t)l * w.layer_stride;
    // fused, pair-interleaved QKV rows
    const float* srcs[3] = {st[1] + (size_t)l * qd * D, st[2] + (size_t)l * kd * D,
                            st[3] + (size_t)l * kd * D};
    const int heads[3] = {d.H, d.KH, d.KH};
    size_t row = 0;
    for (int part = 0; part < 3; ++part) {
      for (int hh = 0; hh < heads[part]; ++hh) {
        for (int s = 0; s < d.hd; ++s) {
          const float* src = srcs[part] + ((size_t)hh * d.hd + pair_dim(s, d.hd)) * D;
          RCCHK(to_bf16_exact(src, D, dst + row * D, names[1 + part]));
          ++row;
        }
      }
    }
    RCCHK(to_bf16_exact(st[4] + (size_t)l * D * qd, D * qd, dst + w.off_proj, "c_proj"));
    RCCHK(to_bf16_exact(st[5] + (size_t)l * dff * D, dff * D, dst + w.off_fc, "c_fc"));
    RCCHK(to_bf16_exact(st[6] + (size_t)l * D * dff, D * dff, dst + w.off_proj2, "c_proj2"));
  }
  bf16_t* tail = h.data() + w.layer_stride * d.L;
  RCCHK(to_bf16_exact(st[7], V * D, tail, "lm_head"));
  RCCHK(to_bf16_exact(st[0], V * D, tail + V * D, "wte"));
  w.bytes = n_total * sizeof(bf16_t);
  float wmax = 0.f;  // over every GEMM weight (the layers and lm_head)
  for (size_t i = 0; i < w.layer_stride * d.L + V * D; ++i) {
    uint32_t u = (uint32_t)(h[i] & 0x7FFF) << 16;
    float f;
    memcpy(&f, &u, 4);
    wmax = std::max(wmax, f);
  }
  m->wmax = wmax;
  HIPCHK(hipMalloc((void**)&w.base, w.bytes));
  RCCHK(dev_copy(m, w.base, h.data(), w.bytes, hipMemcpyHostToDevice));
  HIPCHK(hipMalloc((void**)&m->d_ovf, 4));
  RCCHK(dev_zero(m, m->d_ovf, 4));
  HIPCHK(hipStreamSynchronize(m->stream));
  w.lm = w.base + w.layer_stride * d.L;
  w.wte = w.lm + V * D;
  return setup_fused(m, h.data());
}

void free_work(fg_model* m) {
  Work& ws = m->ws;
  void* ptrs[] = {ws.x, ws.q, ws.ao, ws.h, ws.logits, ws.ids, ws.tgt, ws.nll, ws.stat, ws.amax,
                  ws.xs, ws.aos, ws.hs, ws.ssq, ws.part, ws.nllp, m->qs};
  for (void* p : ptrs)
    if (p) (void)hipFree(p);
  ws = Work();
  m->qs = nullptr;
  m->work_bytes = 0;
}

// Host threads that copy out of pinned staging memory, shared by every
// handle of the process: a copy is split over the workers and the calling
// thread, one copy at a time (handles copying large outputs at once take
// turns). A forked child gets a pool object of its own, with new mutexes,
// condition variables and workers: what it inherited (locks possibly held by
// parent threads that do not exist in the child) is never touched again.
class CopyPool {
 public:
  static void copy(void* dst, const void* src, size_t n) {
    CopyPool* pool = instance();
    std::lock_guard<std::mutex> one(pool->job_mu_);
    pool->run_job(static_cast<char*>(dst), static_cast<const char*>(src), n);
  }

 private:
  explicit CopyPool(pid_t pid) : pid_(pid) {}
  // The pool of this process, made on first use and again after a fork.
  // Objects are never destroyed: detached workers wait on their members
  // until exit, and a parent's object is left as the fork found it.
  static CopyPool* instance() {
    static std::atomic<CopyPool*> cur{nullptr};
    const pid_t me = getpid();
    CopyPool* p = cur.load(std::memory_order_acquire);
    while (!p || p->pid_ != me) {
      CopyPool* fresh = new CopyPool(me);  // (no threads until its first job)
      if (cur.compare_exchange_strong(p, fresh, std::memory_order_acq_rel)) return fresh;
      delete fresh;  // another thread of this process made one first: p holds it now
    }
    return p;
  }

  static constexpr int kWorkers = 7;
  const pid_t pid_;
  std::mutex job_mu_, mu_;
  std::condition_variable go_, done_;
  char* dst_ = nullptr;
  const char* src_ = nullptr;
  size_t n_ = 0, step_ = 0;
  uint64_t gen_ = 0;
  int pending_ = 0, nw_ = 0;  // nw_: workers running (fewer if the system refused threads)
  bool started_ = false;

  void part(int i) {
    const size_t b = (size_t)i * step_;
    if (b < n_) memcpy(dst_ + b, src_ + b, std::min(step_, n_ - b));
  }
  void worker(int i, uint64_t seen) {
    for (;;) {
      {
        std::unique_lock<std::mutex> lk(mu_);
        go_.wait(lk, [&] { return gen_ != seen; });
        seen = gen_;
      }
      part(i);
      std::lock_guard<std::mutex> lk(mu_);
      if (--pending_ == 0) done_.notify_one();
    }
  }
  void run_job(char* dst, const char* src, size_t n) {
    if (!started_) {
      started_ = true;
      try {
        for (; nw_ < kWorkers; ++nw_) std::thread([this, i = nw_, g = gen_] { worker(i, g); }).detach();
      } catch (const std::system_error&) {
        // the calling thread copies what no worker takes
      }
    }
    {
      std::lock_guard<std::mutex> lk(mu_);
      dst_ = dst;
      src_ = src;
      n_ = n;
      step_ = (n + nw_) / (nw_ + 1);
      pending_ = nw_;
      ++gen_;
    }
    go_.notify_all();
    part(nw_);
    std::unique_lock<std::mutex> lk(mu_);
    done_.wait(lk, [&] { return pending_ == 0; });
  }
};

// bytes from device memory to the caller's host memory (pageable), queued
// after the work on stream s. Large copies go through two pinned staging
// buffers: chunk i lands by DMA while host threads copy chunk i-1 out
// (T=2048 logits, 67 MB: ~1.3 ms instead of ~3.7 ms straight to pageable
// memory). Returns with the copy complete.
int32_t copy_out(fg_model* m, void* dst, const void* src, size_t bytes, hipStream_t s) {
  constexpr size_t kChunk = (size_t)8 << 20;
  if (bytes < kChunk) {
    HIPCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s));
    HIPCHK(hipStreamSynchronize(s));
    return FG_OK;
  }
  for (int i = 0; i < 2; ++i) {
    if (!m->pin[i]) HIPCHK(hipHostMalloc(&m->pin[i], kChunk, hipHostMallocDefault));
    if (!m->pin_ev[i]) HIPCHK(hipEventCreateWithFlags(&m->pin_ev[i], hipEventDisableTiming));
  }
  const size_t nch = (bytes + kChunk - 1) / kChunk;
  auto len = [&](size_t i) { return std::min(kChunk, bytes - i * kChunk); };
  for (size_t i = 0; i <= nch; ++i) {
    if (i < nch) {
      HIPCHK(hipMemcpyAsync(m->pin[i & 1], static_cast<const char*>(src) + i * kChunk, len(i),
                            hipMemcpyDeviceToHost, s));
      HIPCHK(hipEventRecord(m->pin_ev[i & 1], s));
    }
    if (i >= 1) {
      const size_t j = i - 1;
      HIPCHK(hipEventSynchronize(m->pin_ev[j & 1]));
      CopyPool::copy(static_cast<char*>(dst) + j * kChunk, m->pin[j & 1], len(j));
    }
  }
  return FG_OK;
}

int32_t ensure_work(fg_model* m, int64_t rows) {
  if (rows <= m->ws.rows) return FG_OK;
  RCCHK(quiesce(m));
  free_work(m);
  const Dims& d = m->d;
  Work& ws = m->ws;
  int64_t total = 0;
  auto alloc = [&](void** p, int64_t bytes) -> int32_t {
    total += bytes;
    HIPCHK(hipMalloc(p, (size_t)bytes));
    return dev_zero(m, *p, (size_t)bytes);
  };
  RCCHK(alloc((void**)&ws.x, rows * d.D * 4));
  RCCHK(alloc((void**)&ws.q, rows * d.qd() * 4));
  RCCHK(alloc((void**)&ws.ao, rows * d.qd() * 4));
  RCCHK(alloc((void**)&ws.h, rows * d.dff * 4));
  RCCHK(alloc((void**)&ws.logits, rows * d.V * 4));
  RCCHK(alloc((void**)&ws.ids, rows * 4));
  RCCHK(alloc((void**)&ws.tgt, rows * 4));
  RCCHK(alloc((void**)&ws.nll, rows * 4));
  RCCHK(alloc((void**)&ws.stat, rows * 4));
  RCCHK(alloc((void**)&ws.amax, rows * 4));
  RCCHK(alloc((void**)&m->qs, rows * d.qd() * 2 * 2));
  RCCHK(alloc((void**)&ws.xs, rows * d.D * 2 * 2));
  RCCHK(alloc((void**)&ws.aos, rows * d.qd() * 2 * 2));
  RCCHK(alloc((void**)&ws.hs, rows * d.dff * 2 * 2));
  RCCHK(alloc((void**)&ws.ssq, rows * (d.D / 64) * 4));
  if (d.V % 256 == 0) RCCHK(alloc((void**)&ws.nllp, rows * (d.V / NLL_GROUP_COLS) * 2 * 4));
  // split-K partials of the small-M GEMMs: the largest any row count up to
  // `rows` needs over the five GEMM shapes
  int64_t part = 0;
  for (int64_t r = 1; r <= rows && r <= 128; ++r) {
    const int64_t shapes[5][2] = {{d.nqkv(), d.D}, {d.D, d.qd()}, {d.dff, d.D}, {d.D, d.dff},
                                  {d.V, d.D}};
    for (auto& sh : shapes)
      part = std::max(part, gemm_splitk_floats(r, (int)sh[0], (int)sh[1]));
  }
  if (part > 0) RCCHK(alloc((void**)&ws.part, part * 4));
  HIPCHK(hipStreamSynchronize(m->stream));  // the clears, before any caller stream's work
  ws.rows = rows;
  m->work_bytes = total;
  m->gen++;
  return FG_OK;
}

// hi/lo key and value planes for B sequences of npos (padded) positions.
int32_t ensure_split(fg_model* m, int64_t elems) {
  if (elems <= m->split_kv_elems) return FG_OK;
  RCCHK(quiesce(m));
  if (m->ks) HIPCHK(hipFree(m->ks));
  if (m->vt) HIPCHK(hipFree(m->vt));
  m->ks = m->vt = nullptr;
  m->split_kv_elems = 0;
  HIPCHK(hipMalloc((void**)&m->ks, (size_t)elems * 2 * 2));
  HIPCHK(hipMalloc((void**)&m->vt, (size_t)elems * 2 * 2));
  // the attention reads whole 64-key steps: padding positions must hold
  // finite values (zero here; later only values this engine wrote)
  RCCHK(dev_zero(m, m->ks, (size_t)elems * 2 * 2));
  RCCHK(dev_zero(m, m->vt, (size_t)elems * 2 * 2));
  HIPCHK(hipStreamSynchronize(m->stream));
  m->split_kv_elems = elems;
  m->gen++;
  return FG_OK;
}

// Scratch of the chunk attention for B x T queries after pos0 cached ones.
int32_t ensure_attn(fg_model* m, int B, int T, int pos0) {
  const int64_t floats = attn_scratch_floats(m->d, B, T, pos0);
  if (floats <= m->attn_floats) return FG_OK;
  RCCHK(quiesce(m));
  if (m->attn_part) HIPCHK(hipFree(m->attn_part));
  m->attn_part = nullptr;
  m->attn_floats = 0;
  HIPCHK(hipMalloc((void**)&m->attn_part, (size_t)floats * 4));
  RCCHK(dev_zero(m, m->attn_part, (size_t)floats * 4));
  HIPCHK(hipStreamSynchronize(m->stream));
  m->attn_floats = floats;
  m->gen++;
  return FG_OK;
}

int npos_pad(int n) { return (n + 63) / 64 * 64; }

// The fp32 GEMV serves up to four token rows (its rows sit in LDS); beyond
// that every linear of the pass runs on the MFMA GEMM with split operands.
bool use_gemm(const Dims& d, int64_t rows) {
  return rows > 4 || rows * (int64_t)d.dff * 4 > 65536;
}

// y = epi(x W^T) on the path chosen for the pass. Algorithmic traffic:
// weights once, activations in and out once (RESID reads the residual).
void linear(fg_model* m, hipStream_t s, GemvEpi epi, const GemvArgs& a, const int32_t* d_pos,
            bool gm) {
  const double M = a.M, N = a.N, K = a.K;
  const double flops = 2.0 * M * N * K;
  const double bytes = N * K * 2 + M * K * 4 + M * N * 4 * (epi == GV_RESID ? 2 : 1);
  if (gm)
    timed(m, s, FG_K_GEMM, flops, bytes, [&] { launch_gemm_pos(s, epi, a, d_pos); });
  else
    timed(m, s, FG_K_GEMV, flops, bytes, [&] { launch_gemv_pos(s, epi, a, d_pos); });
}

GemvArgs base_args(fg_model* m, const Work& ws) {
  GemvArgs a;
  memset(&a, 0, sizeof a);
  a.part = ws.part;
  a.eps = m->d.eps;
  a.cosb = m->d_cos;
  a.sinb = m->d_sin;
  a.H = m->d.H;
  a.KH = m->d.KH;
  a.hd = m->d.hd;
  return a;
}

struct PassOpts {
  int pos_host = -1;      // host value of the first position (timing model), -1: pos0
  bool embed = true;      // false: x already holds the embedded rows
  bool rows_single = false;  // every row as a single cached step (see layer_stack)
  const int32_t* d_rows = nullptr;  // rows_single: rows live, read on the device
  bool kv16 = false;      // the cache holds bf16 elements
  bool f16 = false;       // single-term fp16 MFMA pass where the MFMA path runs (> 128 rows)
  float* nll_part = nullptr;  // lm_head writes the cross-entropy's partials here (GEMM path)
  // (nullable) the chunk attention's positive-score counts, attn_items(...)
  // per layer, layer after layer
  uint32_t* pos_cnt = nullptr;
  // (nullable) the single-query attention's arrival counters
  // (attn_decode_counters(d, rows) of them, zero between launches)
  uint32_t* dec_cnt = nullptr;
};

// One pass over rows = B*T token rows: embedding of ids, the layer stack,
// lm_head into logits. Positions: pos0 (+ *d_pos if given) + row % T. K/V
// go to kc/vc with [L][B][maxT][KH*hd] layout (layer stride lstride floats),
// or only to the split planes when kc is null (gpt_forward). Attention: the
// single-query kernel for a cached step (T == 1, attn_step), else the causal
// chunk kernel (causal_attn / attn_chunk). With o.rows_single the T rows
// of a sequence are T consecutive single steps in one pass: fp32 GEMV and
// the single-query kernel per row, each row's arithmetic that of the step
// it stands for (a speculative verification pass).
void layer_stack(fg_model* m, hipStream_t s, const int32_t* ids, int B, int T, int pos0,
                 const int32_t* d_pos, float* kc, float* vc, int maxT, int64_t lstride,
                 float* dec_part, float* logits, const PassOpts& o = PassOpts(),
                 Work* ws_in = nullptr) {
  const Dims& d = m->d;
  Work& ws = ws_in ? *ws_in : m->ws;
  const int rows = B * T;
  const bool gm = !o.rows_single && use_gemm(d, rows);
  // the single-term fp16 pass: MFMA GEMMs of more than 128 rows (no split K)
  const bool f16 = o.f16 && gm && rows > 128 && m->w16;
  auto W = [&](const bf16_t* p) { return f16 ? m->w16 + (p - m->w.base) : p; };
  const int pos_host = o.pos_host < 0 ? pos0 : o.pos_host;
  const bool embed = o.embed;
  // causal (query, key) pairs per (sequence, head) and the attention traffic
  const double pairs = (double)T * pos_host + 0.5 * (double)T * (T + 1);
  const double at_flops = 4.0 * d.hd * d.H * B * pairs;
  const double at_bytes = (double)B * (2.0 * T * d.qd() + 2.0 * (pos_host + T) * d.kvd()) * 4;
  const int64_t xplane = (int64_t)rows * d.D, aplane = (int64_t)rows * d.qd();
  const int64_t hplane = (int64_t)rows * d.dff;
  // ssq partials per row after the attention-output RESID
  const int nt_resid = gemm_ssq_parts(rows, d.D, d.qd());
  const int64_t pos_items = o.pos_cnt ? attn_items(d, B, T, pos0) : 0;

  if (embed)  // (else x already holds the embedded rows)
    timed(m, s, FG_K_OTHER, 0, (double)rows * d.D * (gm ? 10 : 6), [&] {
      launch_embed_norm(s, d, m->w.wte, ids, rows, ws.x, gm ? ws.xs : nullptr, xplane,
                        gm ? ws.ssq : nullptr, o.d_rows, f16);
    });
  int nt = 1;  // partial sums of squares per row of the current residual
  for (int l = 0; l < d.L; ++l) {
    // null: no persistent cache (gpt_forward); lstride counts elements
    const int64_t loff = o.kv16 ? l * lstride / 2 : l * lstride;  // in floats
    float* lk = kc ? kc + loff : nullptr;
    float* lv = vc ? vc + loff : nullptr;
    GemvArgs a = base_args(m, ws);
    a.M = rows;
    a.d_M = o.d_rows;
    a.T = T;
    a.pos0 = pos0;
    a.kc = lk;
    a.kv16 = o.kv16 ? 1 : 0;
    a.vc = lv;
    a.maxT = maxT;
    // q, k, v = rmsnorm(x) Wqkv^T, RoPE on q and k, k/v appended to the cache
    // (and, for a chunk, written as bf16 hi/lo planes for the MFMA attention)
    const bool one = (T == 1 || o.rows_single) && lk != nullptr;
    const int npos = npos_pad(pos0 + T);
    if (!one) {
      a.qs = m->qs;
      a.q_plane = aplane;
      a.ks = m->ks;
      a.vt = m->vt;
      a.npos = npos;
      a.kv_plane = (int64_t)B * npos * d.kvd();
    }
    a.x = ws.x; a.xs = ws.xs; a.xs_plane = xplane; a.ssq_in = ws.ssq; a.ssq_n = nt;
    a.f16 = f16 ? 1 : 0;
    a.ovf = f16 ? m->d_ovf : nullptr;
    a.wscale = m->w16_inv;
    a.w = W(m->w.qkv(l)); a.N = d.nqkv(); a.K = d.D; a.norm = 1; a.y = ws.q;
    // Batched cached steps (split-K GEMM, one query row per sequence): the
    // decode attention finishes the QKV's split-K sums itself (row norm,
    // RoPE, the k/v append) in place of the reduce launch
    QkvFold qf;
    bool fold = false;
    if (one && gm && T == 1 && !o.d_rows && !f16 &&
        attn_decode_takes_qkv(d, B, maxT, d_pos != nullptr, pos0 + 1, o.kv16)) {
      int sp = 0;
      const double M = a.M, N = a.N, K = a.K;  // (linear()'s units)
      timed(m, s, FG_K_GEMM, 2.0 * M * N * K, N * K * 2 + M * K * 4 + M * N * 4, [&] {
        sp = launch_gemm_partials(s, GV_QKV, a, d_pos);
      });
      if (sp > 0) {
        fold = true;
        qf.part = a.part;
        qf.splits = sp;
        qf.rows = rows;
        qf.N = a.N;
        qf.K = a.K;
        qf.ssq_n = a.ssq_n;
        qf.ssq_in = a.ssq_in;
        qf.eps = a.eps;
        qf.cosb = a.cosb;
        qf.sinb = a.sinb;
      }
    }
    if (!fold) linear(m, s, GV_QKV, a, d_pos, gm);
    a.qs = nullptr;
    a.ks = a.vt = nullptr;
    uint16_t* aos = gm ? ws.aos : nullptr;
    if (one) {
      timed(m, s, FG_K_ATTN_DECODE, at_flops, at_bytes, [&] {
        launch_attn_decode_pos(s, d, ws.q, lk, lv, o.kv16, B, maxT, d_pos, pos0 + 1, dec_part,
                               o.dec_cnt, ws.ao, aos,
                               aplane, T, o.d_rows, fold ? &qf : nullptr);
      });
    } else {
      if (pos0 > 0)  // earlier cache positions enter the chunk's key planes
        timed(m, s, FG_K_OTHER, 0, (double)B * pos0 * d.kvd() * 16, [&] {
          launch_split_cache(s, d, lk, lv, o.kv16, B, maxT, pos0, npos,
                             (int64_t)B * npos * d.kvd(),
                             m->ks, m->vt);
        });
      timed(m, s, FG_K_ATTN_CHUNK, at_flops, at_bytes, [&] {
        launch_attn_mfma(s, d, m->qs, m->ks, m->vt, B, T, npos, pos0, aplane,
                         (int64_t)B * npos * d.kvd(), m->attn_part, ws.ao, aos, aplane, f16,
                         o.pos_cnt ? o.pos_cnt + l * pos_items : nullptr);
      });
    }
    // x += attn_out Wproj^T (GEMM path: also the split x and its row sums)
    a.x = ws.ao; a.xs = ws.aos; a.xs_plane = aplane; a.ssq_n = 0;
    a.w = W(m->w.proj(l)); a.N = d.D; a.K = d.qd(); a.norm = 0; a.y = ws.x;
    a.ys = ws.xs; a.ys_plane = xplane; a.ssq_out = ws.ssq;
    linear(m, s, GV_RESID, a, d_pos, gm);
    nt = nt_resid;
    // h = relu(rmsnorm(x) Wfc^T)^2
    a.x = ws.x; a.xs = ws.xs; a.xs_plane = xplane; a.ssq_in = ws.ssq; a.ssq_n = nt;
    a.w = W(m->w.fc(l)); a.N = d.dff; a.K = d.D; a.norm = 1; a.y = ws.h;
    a.ys = ws.hs; a.ys_plane = hplane; a.ssq_out = nullptr;
    linear(m, s, GV_RELU2, a, d_pos, gm);
    // x += h Wproj2^T
    a.x = ws.h; a.xs = ws.hs; a.xs_plane = hplane; a.ssq_n = 0;
    a.w = W(m->w.proj2(l)); a.N = d.D; a.K = d.dff; a.norm = 0; a.y = ws.x;
    a.ys = ws.xs; a.ys_plane = xplane; a.ssq_out = ws.ssq;
    linear(m, s, GV_RESID, a, d_pos, gm);
    nt = gemm_ssq_parts(rows, d.D, d.dff);
  }
  GemvArgs a = base_args(m, ws);
  a.M = rows; a.T = T; a.d_M = o.d_rows;
  a.x = ws.x; a.xs = ws.xs; a.xs_plane = xplane; a.ssq_in = ws.ssq; a.ssq_n = nt;
  a.f16 = f16 ? 1 : 0;
  a.ovf = f16 ? m->d_ovf : nullptr;
  a.wscale = m->w16_inv;
  a.w = W(m->w.lm); a.N = d.V; a.K = d.D; a.norm = 1; a.y = logits;
  a.nll_part = gm ? o.nll_part : nullptr;
  linear(m, s, GV_STORE, a, d_pos, gm);
}

int32_t check_rope(fg_model* m, int64_t upto) {
  if (upto > m->rope_n)
    return seterr(FG_EROPE, "RoPE rows set for positions < %d; position %lld needed",
                  m->rope_n, (long long)upto - 1);
  return FG_OK;
}

int32_t forward_core(fg_model* m, const int32_t* d_ids, int B, int T, float* d_logits,
                     const int32_t* d_tgt, float* d_nll, hipStream_t s,
                     uint32_t* d_pos_cnt = nullptr) {
  if (B < 1 || T < 1) return seterr(FG_EARG, "B and T must be >= 1");
  RCCHK(check_rope(m, T));
  const int64_t rows = (int64_t)B * T;
  if (rows > (1ll << 30) / m->d.V) return seterr(FG_EARG, "B*T too large");
  RCCHK(ensure_work(m, rows));
  RCCHK(ensure_split(m, (int64_t)B * npos_pad(T) * m->d.kvd()));
  RCCHK(ensure_attn(m, B, T, 0));
  float* logits = d_logits ? d_logits : m->ws.logits;
  const double vb = (double)rows * m->d.V * 4;
  PassOpts o;
  o.f16 = m->fwd_f16;
  // the cross-entropy from lm_head's log-sum-exp partials where the GEMM
  // writes them (no second pass over the logits), else from the logits
  const bool nll_parts = d_tgt && d_nll && m->ws.nllp && use_gemm(m->d, rows) &&
                         gemm_store_nll(rows, m->d.V);
  if (nll_parts) o.nll_part = m->ws.nllp;
  o.pos_cnt = d_pos_cnt;
  layer_stack(m, s, d_ids, B, T, 0, nullptr, nullptr, nullptr, T, 0, nullptr, logits, o);
  if (nll_parts)
    timed(m, s, FG_K_OTHER, 0, (double)rows * (m->d.V / NLL_GROUP_COLS) * 8 + rows * 12, [&] {
      launch_nll_parts(s, logits, m->ws.nllp, d_tgt, rows, m->d.V, d_nll);
    });
  else if (d_tgt && d_nll)
    timed(m, s, FG_K_OTHER, 0, vb, [&] { launch_nll(s, logits, d_tgt, rows, m->d.V, d_nll); });
  HIPCHK(hipGetLastError());
  return FG_OK;
}

int32_t model_new(const fg_dims* dims, fg_model** out, fg_model** pm) {
  if (!out) return seterr(FG_EARG, "out is NULL");
  *out = nullptr;
  Dims d;
  RCCHK(check_dims(dims, &d));
  int dev = 0;
  RCCHK(check_device(&dev));
  fg_model* m = new fg_model();
  m->d = d;
  m->device = dev;
  hipError_t e = hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete m;
    return seterr(FG_EHIP, "hipStreamCreate: %s", hipGetErrorString(e));
  }
  *pm = m;
  return FG_OK;
}

}  // namespace

// ------------------------------------------------------------------ model
extern "C" int32_t fg_model_create(const fg_dims* dims, const float* wte, const float* c_q,
                                   const float* c_k, const float* c_v, const float* c_proj,
                                   const float* c_fc, const float* c_proj2,
                                   const float* lm_head, fg_model** out) {
  fg_model* m = nullptr;
  RCCHK(model_new(dims, out, &m));
  const float* st[8] = {wte, c_q, c_k, c_v, c_proj, c_fc, c_proj2, lm_head};
  int32_t rc = upload_weights(m, st);
  if (rc != FG_OK) {
    fg_model_destroy(m);
    return rc;
  }
  *out = m;
  return FG_OK;
}

extern "C" int32_t fg_model_load(const fg_dims* dims, const char* weights_dir, fg_model** out) {
  if (!weights_dir) return seterr(FG_EARG, "weights_dir is NULL");
  Dims d;
  RCCHK(check_dims(dims, &d));
  const size_t D = d.D, qd = d.qd(), kd = d.kvd(), dff = d.dff, V = d.V, L = d.L;
  std::vector<float> wte(V * D), lm(V * D), cq(L * qd * D), ck(L * kd * D), cv(L * kd * D),
      cp(L * D * qd), cf(L * dff * D), cp2(L * D * dff);
  RCCHK(fg_weights_read(dims, weights_dir, wte.data(), cq.data(), ck.data(), cv.data(), cp.data(),
                        cf.data(), cp2.data(), lm.data()));
  return fg_model_create(dims, wte.data(), cq.data(), ck.data(), cv.data(), cp.data(), cf.data(),
                         cp2.data(), lm.data(), out);
}

extern "C" int32_t fg_model_destroy(fg_model* m) {
  if (!m) return FG_OK;
  (void)hipSetDevice(m->device);
  if (m->stream) (void)hipStreamSynchronize(m->stream);
  free_work(m);
  if (m->ks) (void)hipFree(m->ks);
  if (m->vt) (void)hipFree(m->vt);
  if (m->attn_part) (void)hipFree(m->attn_part);
  if (m->d_pos) (void)hipFree(m->d_pos);
  if (m->d_ovf) (void)hipFree(m->d_ovf);
  if (m->samp) (void)hipFree(m->samp);
  if (m->w.base) (void)hipFree(m->w.base);
  if (m->fused_w) (void)hipFree(m->fused_w);
  if (m->w16) (void)hipFree(m->w16);
  if (m->fused_slots) (void)hipFree(m->fused_slots);
  if (m->fused_err) (void)hipFree(m->fused_err);
  if (m->d_cos) (void)hipFree(m->d_cos);
  if (m->d_sin) (void)hipFree(m->d_sin);
  for (int i = 0; i < 2; ++i) {
    if (m->pin[i]) (void)hipHostFree(m->pin[i]);
    if (m->pin_ev[i]) (void)hipEventDestroy(m->pin_ev[i]);
  }
  for (auto& r : m->trecs) {
    (void)hipEventDestroy(r.a);
    (void)hipEventDestroy(r.b);
  }
  for (auto e : m->evpool) (void)hipEventDestroy(e);
  if (m->stream) (void)hipStreamDestroy(m->stream);
  delete m;
  return FG_OK;
}

extern "C" int32_t fg_set_rope(fg_model* m, int32_t pos0, int32_t n_pos, const float* cos_buf,
                               const float* sin_buf) {
  if (!m || !cos_buf || !sin_buf) return seterr(FG_EARG, "NULL argument");
  if (pos0 < 0 || n_pos < 1) return seterr(FG_EARG, "bad row range");
  if (pos0 > m->rope_n)
    return seterr(FG_EROPE, "RoPE rows must be set contiguously from 0 (have %d, asked %d)",
                  m->rope_n, pos0);
  GUARD(m);
  const int half = m->d.hd / 2;
  const int need = pos0 + n_pos;
  if (need > m->rope_cap) {
    int cap = m->rope_cap ? m->rope_cap : 64;
    while (cap < need) cap *= 2;
    float *nc = nullptr, *ns = nullptr;
    HIPCHK(hipMalloc((void**)&nc, (size_t)cap * half * 4));
    HIPCHK(hipMalloc((void**)&ns, (size_t)cap * half * 4));
    RCCHK(quiesce(m));
    RCCHK(dev_zero(m, nc, (size_t)cap * half * 4));
    RCCHK(dev_zero(m, ns, (size_t)cap * half * 4));
    if (m->rope_n > 0) {
      RCCHK(dev_copy(m, nc, m->d_cos, (size_t)m->rope_n * half * 4, hipMemcpyDeviceToDevice));
      RCCHK(dev_copy(m, ns, m->d_sin, (size_t)m->rope_n * half * 4, hipMemcpyDeviceToDevice));
    }
    HIPCHK(hipStreamSynchronize(m->stream));
    if (m->d_cos) HIPCHK(hipFree(m->d_cos));
    if (m->d_sin) HIPCHK(hipFree(m->d_sin));
    m->d_cos = nc;
    m->d_sin = ns;
    m->rope_cap = cap;
    m->gen++;
  }
  // rows being replaced may still be read by queued work on any stream
  RCCHK(quiesce(m));
  RCCHK(dev_copy(m, m->d_cos + (size_t)pos0 * half, cos_buf, (size_t)n_pos * half * 4,
                 hipMemcpyHostToDevice));
  RCCHK(dev_copy(m, m->d_sin + (size_t)pos0 * half, sin_buf, (size_t)n_pos * half * 4,
                 hipMemcpyHostToDevice));
  if (need > m->rope_n) m->rope_n = need;
  return FG_OK;
}

namespace {

// After a pass queued on s: FG_ERANGE when a single-term fp16 epilogue
// raised the overflow flag (the flag is cleared again).
int32_t check_f16_range(fg_model* m, hipStream_t s) {
  if (!m->fwd_f16) return FG_OK;
  uint32_t f = 0;
  HIPCHK(hipMemcpyAsync(&f, m->d_ovf, 4, hipMemcpyDeviceToHost, s));
  HIPCHK(hipStreamSynchronize(s));
  if (f == 0) return FG_OK;
  launch_zero_u32(s, m->d_ovf, 1);
  HIPCHK(hipStreamSynchronize(s));
  return seterr(FG_ERANGE, "an activation of the single-term fp16 pass reached fp16's range "
                           "limit (|x| >= 65520): results invalid; run without "
                           "FG_OPT_FORWARD_F16");
}

// fg_forward, and with npos set attn_sgemm's positive-score statistic.
int32_t forward_host(fg_model* m, const int32_t* ids, int32_t B, int32_t T, float* logits,
                     const int32_t* targets, float* nll, int32_t* npos) {
  if (!m || !ids) return seterr(FG_EARG, "NULL argument");
  if (B < 1 || T < 1) return seterr(FG_EARG, "B and T must be >= 1");
  const int64_t rows = (int64_t)B * T;
  for (int64_t i = 0; i < rows; ++i)
    if (ids[i] < 0 || ids[i] >= m->d.V)
      return seterr(FG_EARG, "id %d at %lld outside [0, %d)", ids[i], (long long)i, m->d.V);
  if (targets)
    for (int64_t i = 0; i < rows; ++i)
      if (targets[i] < 0 || targets[i] >= m->d.V)
        return seterr(FG_EARG, "target %d at %lld outside [0, %d)", targets[i], (long long)i,
                      m->d.V);
  GUARD(m);
  RCCHK(ensure_work(m, rows));
  hipStream_t s = m->stream;
  const int64_t items = npos ? attn_items(m->d, B, T, 0) : 0;
  if (npos && items * m->d.L > m->pos_cap) {
    RCCHK(quiesce(m));
    if (m->d_pos) HIPCHK(hipFree(m->d_pos));
    m->d_pos = nullptr;
    m->pos_cap = 0;
    HIPCHK(hipMalloc((void**)&m->d_pos, (size_t)items * m->d.L * 4));
    RCCHK(dev_zero(m, m->d_pos, (size_t)items * m->d.L * 4));
    m->pos_cap = items * m->d.L;
  }
  HIPCHK(hipMemcpyAsync(m->ws.ids, ids, rows * 4, hipMemcpyHostToDevice, s));
  if (targets) HIPCHK(hipMemcpyAsync(m->ws.tgt, targets, rows * 4, hipMemcpyHostToDevice, s));
  if (m->fwd_f16) launch_zero_u32(s, m->d_ovf, 1);
  RCCHK(forward_core(m, m->ws.ids, B, T, m->ws.logits, targets ? m->ws.tgt : nullptr,
                     targets ? m->ws.nll : nullptr, s, npos ? m->d_pos : nullptr));
  RCCHK(check_f16_range(m, s));
  if (logits) RCCHK(copy_out(m, logits, m->ws.logits, (size_t)rows * m->d.V * 4, s));
  if (targets && nll) HIPCHK(hipMemcpyAsync(nll, m->ws.nll, rows * 4, hipMemcpyDeviceToHost, s));
  std::vector<uint32_t> cnt(npos ? (size_t)items * m->d.L : 0);
  if (npos) HIPCHK(hipMemcpyAsync(cnt.data(), m->d_pos, cnt.size() * 4, hipMemcpyDeviceToHost, s));
  HIPCHK(hipStreamSynchronize(s));
  if (npos) {
    // item i of a layer belongs to (row * H + head) = i % (B * H); its
    // counts are whole numbers of scores, so the sums are exact
    const int64_t nbh = (int64_t)B * m->d.H;
    std::vector<int64_t> sum((size_t)nbh);
    for (int l = 0; l < m->d.L; ++l) {
      std::fill(sum.begin(), sum.end(), 0);
      for (int64_t i = 0; i < items; ++i) sum[i % nbh] += cnt[(size_t)l * items + i];
      for (int64_t bh = 0; bh < nbh; ++bh) npos[l * nbh + bh] = (int32_t)sum[bh];
    }
  }
  return FG_OK;
}

}  // namespace

extern "C" int32_t fg_forward(fg_model* m, const int32_t* ids, int32_t B, int32_t T,
                              float* logits, const int32_t* targets, float* nll) {
  return forward_host(m, ids, B, T, logits, targets, nll, nullptr);
}

extern "C" int32_t fg_forward_pos(fg_model* m, const int32_t* ids, int32_t B, int32_t T,
                                  float* logits, const int32_t* targets, float* nll,
                                  int32_t* npos) {
  if (!npos) return seterr(FG_EARG, "npos is NULL");
  if (T > 65535) return seterr(FG_EARG, "T %d: the counts of T(T+1)/2 scores overflow", T);
  return forward_host(m, ids, B, T, logits, targets, nll, npos);
}

extern "C" int32_t fg_eval_bpb(fg_model* m, const int32_t* rows, int32_t n_rows, int32_t T,
                               int32_t batch, const int32_t* token_bytes, int32_t n_token_bytes,
                               float* nll, double* row_nats, int64_t* row_bytes,
                               double* total_nats, int64_t* total_bytes) {
  if (!m || !rows || !token_bytes || !total_nats || !total_bytes)
    return seterr(FG_EARG, "NULL argument");
  if (n_rows < 1 || T < 1) return seterr(FG_EARG, "n_rows and T must be >= 1");
  if (batch < 1 || batch > 64) return seterr(FG_EARG, "require 1 <= batch <= 64");
  if (n_token_bytes < 1) return seterr(FG_EARG, "empty token_bytes");
  const int64_t W = (int64_t)T + 1;
  for (int64_t r = 0; r < n_rows; ++r)
    for (int64_t t = 0; t < W; ++t) {
      const int32_t id = rows[r * W + t];
      if (t < T && (id < 0 || id >= m->d.V))
        return seterr(FG_EARG, "row %lld: id %d at %lld outside [0, %d)", (long long)r, id,
                      (long long)t, m->d.V);
      if (t > 0 && (id < 0 || id >= m->d.V || id >= n_token_bytes))
        return seterr(FG_EARG, "row %lld: token id %d at %lld out of token_bytes range (%d)",
                      (long long)r, id, (long long)t, n_token_bytes);
    }
  GUARD(m);
  const int64_t cap = (int64_t)batch * T;
  RCCHK(ensure_work(m, cap));
  hipStream_t s = m->stream;
  int32_t* d_tb = nullptr;
  double* d_rn = nullptr;
  long long* d_rb = nullptr;
  HIPCHK(hipMalloc((void**)&d_tb, (size_t)n_token_bytes * 4));
  int32_t rc = FG_OK;
  auto run = [&]() -> int32_t {
    HIPCHK(hipMalloc((void**)&d_rn, (size_t)batch * sizeof(double)));
    HIPCHK(hipMalloc((void**)&d_rb, (size_t)batch * sizeof(long long)));
    HIPCHK(hipMemcpyAsync(d_tb, token_bytes, (size_t)n_token_bytes * 4, hipMemcpyHostToDevice, s));
    std::vector<int32_t> ids(cap), tgt(cap);
    std::vector<double> rn(batch);
    std::vector<long long> rb(batch);
    double tn = 0.0;
    int64_t tbt = 0;
    for (int64_t r0 = 0; r0 < n_rows; r0 += batch) {
      const int nb = (int)std::min<int64_t>(batch, n_rows - r0);
      for (int b = 0; b < nb; ++b) {
        const int32_t* row = rows + (r0 + b) * W;
        std::copy(row, row + T, ids.data() + (int64_t)b * T);          // inputs ids[0:T]
        std::copy(row + 1, row + W, tgt.data() + (int64_t)b * T);      // targets ids[1:T+1]
      }
      const int64_t n = (int64_t)nb * T;
      HIPCHK(hipMemcpyAsync(m->ws.ids, ids.data(), n * 4, hipMemcpyHostToDevice, s));
      HIPCHK(hipMemcpyAsync(m->ws.tgt, tgt.data(), n * 4, hipMemcpyHostToDevice, s));
      if (m->fwd_f16) launch_zero_u32(s, m->d_ovf, 1);
      RCCHK(forward_core(m, m->ws.ids, nb, T, m->ws.logits, m->ws.tgt, m->ws.nll, s));
      timed(m, s, FG_K_OTHER, 0, (double)n * 12, [&] {
        launch_bpb_rows(s, m->ws.nll, m->ws.tgt, nb, T, d_tb, d_rn, d_rb);
      });
      if (nll) HIPCHK(hipMemcpyAsync(nll + r0 * T, m->ws.nll, n * 4, hipMemcpyDeviceToHost, s));
      HIPCHK(hipMemcpyAsync(rn.data(), d_rn, nb * sizeof(double), hipMemcpyDeviceToHost, s));
      HIPCHK(hipMemcpyAsync(rb.data(), d_rb, nb * sizeof(long long), hipMemcpyDeviceToHost, s));
      HIPCHK(hipStreamSynchronize(s));
      RCCHK(check_f16_range(m, s));
      for (int b = 0; b < nb; ++b) {  // rows in order, as bpb_agg adds them
        if (row_nats) row_nats[r0 + b] = rn[b];
        if (row_bytes) row_bytes[r0 + b] = rb[b];
        tn += rn[b];
        tbt += rb[b];
      }
    }
    *total_nats = tn;
    *total_bytes = tbt;
    return FG_OK;
  };
  rc = run();
  (void)hipStreamSynchronize(s);
  (void)hipFree(d_tb);
  if (d_rn) (void)hipFree(d_rn);
  if (d_rb) (void)hipFree(d_rb);
  return rc;
}

extern "C" int32_t fg_forward_dev(fg_model* m, const int32_t* d_ids, int32_t B, int32_t T,
                                  float* d_logits, const int32_t* d_targets, float* d_nll,
                                  void* stream) {
  if (!m || !d_ids) return seterr(FG_EARG, "NULL argument");
  GUARD(m);
  hipStream_t s = stream ? (hipStream_t)stream : m->stream;
  return forward_core(m, d_ids, B, T, d_logits, d_targets, d_nll, s);
}

// ------------------------------------------------------------------ KV
extern "C" int32_t fg_kv_create(fg_model* m, int32_t B, int32_t maxT, fg_kv** out) {
  return fg_kv_create_ex(m, B, maxT, 0, out);
}

extern "C" int32_t fg_kv_create_ex(fg_model* m, int32_t B, int32_t maxT, int32_t flags,
                                   fg_kv** out) {
  if (!m || !out) return seterr(FG_EARG, "NULL argument");
  *out = nullptr;
  if (B < 1 || maxT < 1) return seterr(FG_EARG, "B and maxT must be >= 1");
  if (flags & ~FG_KV_BF16) return seterr(FG_EARG, "unknown cache flags 0x%x", flags);
  // the largest cache this build is tested with
  if (maxT > 16000) return seterr(FG_EARG, "maxT %d above the 16000 this build supports", maxT);
  // the decode attention addresses a sequence's cache rows with 32-bit offsets
  if ((int64_t)maxT * m->d.kvd() * ((flags & FG_KV_BF16) ? 2 : 4) >= ((int64_t)1 << 31))
    return seterr(FG_EARG, "a sequence's cache (maxT %d x %d values) exceeds 2 GiB", maxT,
                  m->d.kvd());
  GUARD(m);
  fg_kv* kv = new fg_kv();
  kv->m = m;
  kv->B = B;
  kv->maxT = maxT;
  kv->kv16 = (flags & FG_KV_BF16) != 0;
  const size_t n = (size_t)m->d.L * B * maxT * m->d.kvd(), esz = kv->kv16 ? 2 : 4;
  hipError_t e = hipMalloc((void**)&kv->k, n * esz);
  if (e == hipSuccess) e = hipMalloc((void**)&kv->v, n * esz);
  if (e == hipSuccess) e = hipMalloc((void**)&kv->d_len, 8);
  if (e == hipSuccess) e = hipMalloc((void**)&kv->d_ids, (size_t)B * 4);
  const size_t part_bytes = (size_t)attn_decode_scratch_floats(m->d, B, maxT) * 4;
  if (e == hipSuccess) e = hipMalloc((void**)&kv->d_part, part_bytes);
  const size_t cnt_bytes = (size_t)attn_decode_counters(m->d, std::max(B, GEMV_MAX_ROWS)) * 4;
  if (e == hipSuccess) e = hipMalloc((void**)&kv->d_dcnt, cnt_bytes);
  // zeroed on the handle's stream, and finished before the cache is handed
  // out (its first user may be a caller's stream); the reference's callers
  // zero their caches too
  if (e == hipSuccess) e = hipMemsetAsync(kv->k, 0, n * esz, m->stream);
  if (e == hipSuccess) e = hipMemsetAsync(kv->v, 0, n * esz, m->stream);
  if (e == hipSuccess) e = hipMemsetAsync(kv->d_len, 0, 8, m->stream);
  if (e == hipSuccess) e = hipMemsetAsync(kv->d_ids, 0, (size_t)B * 4, m->stream);
  if (e == hipSuccess) e = hipMemsetAsync(kv->d_part, 0, part_bytes, m->stream);
  if (e == hipSuccess) e = hipMemsetAsync(kv->d_dcnt, 0, cnt_bytes, m->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
  if (e != hipSuccess) {
    (void)hipStreamSynchronize(m->stream);
    if (kv->k) (void)hipFree(kv->k);
    if (kv->v) (void)hipFree(kv->v);
    if (kv->d_len) (void)hipFree(kv->d_len);
    if (kv->d_ids) (void)hipFree(kv->d_ids);
    if (kv->d_part) (void)hipFree(kv->d_part);
    if (kv->d_dcnt) (void)hipFree(kv->d_dcnt);
    delete kv;
    return seterr(FG_EHIP, "KV cache allocation (%zu bytes): %s", 2 * n * esz,
                  hipGetErrorString(e));
  }
  *out = kv;
  return FG_OK;
}

extern "C" int32_t fg_kv_destroy(fg_kv* kv) {
  if (!kv) return FG_OK;
  (void)hipSetDevice(kv->m->device);
  (void)hipStreamSynchronize(kv->m->stream);
  for (auto& g : kv->graphs) (void)hipGraphExecDestroy(g.second);
  void* ptrs[] = {kv->k,     kv->v,      kv->d_len, kv->d_ids,   kv->d_out,  kv->d_lgs,
                  kv->d_part, kv->d_sst, kv->d_sids, kv->d_spart, kv->d_smp, kv->d_dcnt};
  for (void* p : ptrs)
    if (p) (void)hipFree(p);
  if (kv->h_sst) (void)hipHostFree(kv->h_sst);
  if (kv->h_smp) (void)hipHostFree(kv->h_smp);
  delete kv;
  return FG_OK;
}

extern "C" int32_t fg_kv_len(const fg_kv* kv, int32_t* len) {
  if (!kv || !len) return seterr(FG_EARG, "NULL argument");
  *len = kv->len;
  return FG_OK;
}

extern "C" int32_t fg_kv_set_len(fg_kv* kv, int32_t len) {
  if (!kv) return seterr(FG_EARG, "NULL argument");
  if (len < 0 || len > kv->maxT) return seterr(FG_EARG, "len %d outside [0, %d]", len, kv->maxT);
  if (len > kv->filled)
    return seterr(FG_EARG, "len %d: this cache has computed only %d positions", len, kv->filled);
  kv->len = len;
  return FG_OK;
}

extern "C" int32_t fg_kv_read(fg_kv* kv, float* k_out, float* v_out) {
  if (!kv) return seterr(FG_EARG, "NULL argument");
  fg_model* m = kv->m;
  GUARD(m);
  const size_t n = (size_t)m->d.L * kv->B * kv->maxT * m->d.kvd();
  HIPCHK(hipStreamSynchronize(m->stream));
  if (!kv->kv16) {
    if (k_out) HIPCHK(hipMemcpy(k_out, kv->k, n * 4, hipMemcpyDeviceToHost));
    if (v_out) HIPCHK(hipMemcpy(v_out, kv->v, n * 4, hipMemcpyDeviceToHost));
    return FG_OK;
  }
  // bf16 elements widened on the host
  std::vector<uint16_t> h(n);
  float* outs[2] = {k_out, v_out};
  const float* src[2] = {kv->k, kv->v};
  for (int t = 0; t < 2; ++t) {
    if (!outs[t]) continue;
    HIPCHK(hipMemcpy(h.data(), src[t], n * 2, hipMemcpyDeviceToHost));
    for (size_t i = 0; i < n; ++i) {
      const uint32_t u = (uint32_t)h[i] << 16;
      memcpy(outs[t] + i, &u, 4);
    }
  }
  return FG_OK;
}

namespace {

int32_t check_ids(const fg_model* m, const int32_t* ids, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= m->d.V)
      return seterr(FG_EARG, "id %d at %lld outside [0, %d)", ids[i], (long long)i, m->d.V);
  return FG_OK;
}

// TB tokens for each of the kv's B sequences at host position kv->len.
int32_t kv_pass(fg_model* m, fg_kv* kv, const int32_t* h_ids, int TB, float* logits,
                int32_t* next_ids) {
  const int B = kv->B;
  if (TB < 1) return seterr(FG_EARG, "TB must be >= 1");
  if (kv->len + TB > kv->maxT)
    return seterr(FG_EFULL, "cache full (raise maxT): len %d + %d > %d", kv->len, TB, kv->maxT);
  RCCHK(check_rope(m, kv->len + TB));
  const int64_t rows = (int64_t)B * TB;
  RCCHK(ensure_work(m, rows));
  if (TB > 1) {
    RCCHK(ensure_split(m, (int64_t)B * npos_pad(kv->len + TB) * m->d.kvd()));
    RCCHK(ensure_attn(m, B, TB, kv->len));
  }
  // (TB == 1 runs the single-query kernel on the cache)
  hipStream_t s = m->stream;
  HIPCHK(hipMemcpyAsync(m->ws.ids, h_ids, rows * 4, hipMemcpyHostToDevice, s));
  const int64_t lstride = (int64_t)B * kv->maxT * m->d.kvd();
  PassOpts o;
  o.kv16 = kv->kv16;
  o.dec_cnt = kv->d_dcnt;
  layer_stack(m, s, m->ws.ids, B, TB, kv->len, nullptr, kv->k, kv->v, kv->maxT, lstride,
              kv->d_part, m->ws.logits, o);
  HIPCHK(hipGetLastError());
  if (next_ids && TB == 1) {
    launch_argmax(s, m->ws.logits, B, m->d.V, m->ws.amax);
    HIPCHK(hipMemcpyAsync(next_ids, m->ws.amax, (size_t)B * 4, hipMemcpyDeviceToHost, s));
  } else if (next_ids) {
    // argmax of each sequence's last row: rows b*TB + TB-1
    for (int b = 0; b < B; ++b)
      launch_argmax(s, m->ws.logits + ((int64_t)b * TB + TB - 1) * m->d.V, 1, m->d.V,
                    m->ws.amax + b);
    HIPCHK(hipMemcpyAsync(next_ids, m->ws.amax, (size_t)B * 4, hipMemcpyDeviceToHost, s));
  }
  if (logits) RCCHK(copy_out(m, logits, m->ws.logits, (size_t)rows * m->d.V * 4, s));
  HIPCHK(hipStreamSynchronize(s));
  kv->len += TB;
  kv->filled = std::max(kv->filled, kv->len);
  return FG_OK;
}

// One greedy step whose position is read from kv->d_len on the device:
// embed(d_ids) -> layers -> lm_head -> argmax into d_ids and d_out[(len -
// len0) * B], logits copied to d_lgs at the same slot when wanted, len += 1.
// Nothing in it depends on the step index, so a captured run of steps can
// be replayed back to back.
void greedy_step_launches(fg_model* m, fg_kv* kv, hipStream_t s, bool with_logits,
                          int pos_host) {
  const int B = kv->B;
  const int64_t lstride = (int64_t)B * kv->maxT * m->d.kvd();
  if (use_gemm(m->d, B)) {
    PassOpts o;
    o.pos_host = pos_host;
    o.kv16 = kv->kv16;
    o.dec_cnt = kv->d_dcnt;
    layer_stack(m, s, kv->d_ids, B, 1, 0, kv->d_len, kv->k, kv->v, kv->maxT, lstride,
                kv->d_part, m->ws.logits, o);
    timed(m, s, FG_K_OTHER, 0, (double)B * m->d.V * 4 * (with_logits ? 2 : 1), [&] {
      launch_argmax_step(s, m->ws.logits, B, m->d.V, kv->d_ids, kv->d_out, kv->d_len,
                         kv->d_len + 1, with_logits ? kv->d_lgs : nullptr);
    });
  } else {
    // GEMV path: x of this step was embedded by the previous step's tail (or
    // before the first step); the tail does argmax, the next embedding and
    // the length update in one launch
    PassOpts o;
    o.pos_host = pos_host;
    o.embed = false;
    o.kv16 = kv->kv16;
    o.dec_cnt = kv->d_dcnt;
    layer_stack(m, s, kv->d_ids, B, 1, 0, kv->d_len, kv->k, kv->v, kv->maxT, lstride,
                kv->d_part, m->ws.logits, o);
    timed(m, s, FG_K_OTHER, 0, (double)B * (m->d.V * 4 * (with_logits ? 2 : 1) + 6 * m->d.D),
          [&] {
            launch_greedy_tail(s, m->d, m->ws.logits, B, m->w.wte, kv->d_ids, kv->d_out,
                               kv->d_len, kv->d_len + 1, with_logits ? kv->d_lgs : nullptr,
                               m->ws.x);
          });
  }
}

// Replay (capturing on first use) a graph of `steps` greedy steps.
int32_t run_greedy_graph(fg_model* m, fg_kv* kv, hipStream_t s, int steps, bool with_logits) {
  const auto key = std::make_pair(steps, with_logits ? 1 : 0);
  auto it = kv->graphs.find(key);
  if (it == kv->graphs.end()) {
    hipGraph_t g = nullptr;
    HIPCHK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    for (int st = 0; st < steps; ++st) greedy_step_launches(m, kv, s, with_logits, -1);
    HIPCHK(hipStreamEndCapture(s, &g));
    hipGraphExec_t ge = nullptr;
    hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return seterr(FG_EHIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
    it = kv->graphs.emplace(key, ge).first;
  }
  HIPCHK(hipGraphLaunch(it->second, s));
  return FG_OK;
}

// Per-kernel path: runs of captured steps (or eager launches under timing).
int32_t graph_decode(fg_model* m, fg_kv* kv, const int32_t* ids, int n_steps, int with_logits) {
  const int B = kv->B;
  hipStream_t s = m->stream;
  const int32_t lens[2] = {kv->len, kv->len};
  HIPCHK(hipMemcpyAsync(kv->d_ids, ids, (size_t)B * 4, hipMemcpyHostToDevice, s));
  HIPCHK(hipMemcpyAsync(kv->d_len, lens, 8, hipMemcpyHostToDevice, s));
  if (!use_gemm(m->d, B))  // the GEMV-path steps expect x embedded (see greedy_step_launches)
    launch_embed_norm(s, m->d, m->w.wte, kv->d_ids, B, m->ws.x, nullptr, 0, nullptr);
  HIPCHK(hipStreamSynchronize(s));
  if (m->timing) {  // eager launches so every kernel can be bracketed by events
    for (int st = 0; st < n_steps; ++st) greedy_step_launches(m, kv, s, with_logits, lens[0] + st);
  } else {
    // runs of captured steps replayed back to back; ~2k kernel nodes per
    // graph (a GEMM-path step has about twice the launches of a GEMV step)
    const int kGraphSteps = use_gemm(m->d, B) ? 16 : 32;
    int done = 0;
    while (done < n_steps) {
      const int run = n_steps - done < kGraphSteps ? n_steps - done : kGraphSteps;
      RCCHK(run_greedy_graph(m, kv, s, run, with_logits));
      done += run;
    }
  }
  return FG_OK;
}

bool fused_applies(const fg_model* m, const fg_kv* kv, int n_steps) {
  return m->fused_on && m->fused_w && kv->B == 1 && !kv->kv16 &&
         kv->len + n_steps <= m->fl.max_len;
}

// n_steps greedy steps as one persistent launch from the id at d_id0 (on
// the device) at position len0: the steps' argmax ids go to ids_out, their
// logits (when logits_out is set) to logits_out, the cache rows of the
// n_steps positions are written in place. The launch's placement counters
// are cleared first, and its error flag too when clear_err is set (a caller
// running several launches clears it once and reads it after the last).
int32_t fused_launch(fg_model* m, fg_kv* kv, const int32_t* d_id0, int len0, int n_steps,
                     int32_t* ids_out, float* logits_out, bool clear_err) {
  hipStream_t s = m->stream;
  const uint32_t eps = fused_epochs(m->d, n_steps);
  if ((uint64_t)m->fused_ep + eps >= 0xFFFFFF00ull) {  // epochs would wrap: start over
    HIPCHK(hipMemsetAsync(m->fused_slots, 0, (size_t)m->fl.slots * 8, s));
    m->fused_ep = 1;
  }
  if (clear_err)
    HIPCHK(hipMemsetAsync(m->fused_err, 0, 4 * (1 + FUSED_NX), s));
  else
    HIPCHK(hipMemsetAsync(m->fused_err + 1, 0, 4 * FUSED_NX, s));
  FusedArgs a;
  a.arena = m->fused_w;
  a.wte = m->w.wte;
  a.cosb = m->d_cos;
  a.sinb = m->d_sin;
  a.kc = kv->k;
  a.vc = kv->v;
  a.maxT = kv->maxT;
  a.len0 = len0;
  a.n_steps = n_steps;
  a.d_id0 = d_id0;
  a.ids_out = ids_out;
  a.logits_out = logits_out;
  a.slots = m->fused_slots;
  a.ep_base = m->fused_ep;
  a.err = m->fused_err;
  a.cnt = m->fused_err + 1;
  a.D = m->d.D;
  a.H = m->d.H;
  a.KH = m->d.KH;
  a.L = m->d.L;
  a.V = m->d.V;
  a.dff = m->d.dff;
  a.eps = m->d.eps;
  // algorithmic traffic of the loop: per step every weight but the
  // embedding table once, one embedding row, the cache rows read and written
  const Dims& d = m->d;
  const double wbytes = (double)m->w.bytes - 2.0 * d.V * d.D;
  double bytes = 0, flops = 0;
  for (int st = 0; st < n_steps; ++st) {
    const double len = len0 + st + 1;
    bytes += wbytes + 2.0 * d.D + (double)d.L * d.kvd() * 4 * 2 * (len + 1);
    flops += wbytes + (double)d.L * 4 * d.hd * d.H * len;
  }
  // FGPT_FUSED_TRACE=<file>: append the phase timestamps of one step (the
  // second, when there is one) of every workgroup to <file> (diagnostic)
  const char* tpath = getenv("FGPT_FUSED_TRACE");
  const size_t tn = (size_t)FUSED_NWG * (d.L + 1) * 32;
  a.trace = nullptr;  // (null: the kernel built without timestamps)
  a.trace_step = n_steps > 1 ? 1 : 0;
  if (tpath && *tpath) {
    HIPCHK(hipMalloc((void**)&a.trace, tn * 8));
    HIPCHK(hipMemsetAsync(a.trace, 0, tn * 8, s));
  }
  hipError_t e = hipSuccess;
  timed_stream(m, s, FG_K_DECODE_FUSED, flops, bytes,
               [&] { e = launch_fused_decode(s, d, m->fl, a); });
  m->fused_ep += eps;
  if (a.trace) {
    std::vector<uint64_t> ht(tn);
    if (e == hipSuccess) e = hipMemcpyAsync(ht.data(), a.trace, tn * 8, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipFree(a.trace);
    if (e == hipSuccess) {
      FILE* fp = fopen(tpath, "ab");
      if (fp) {
        const int32_t hdr[4] = {FUSED_NWG, d.L + 1, 32 | (m->fl.kind << 16), n_steps};
        fwrite(hdr, 4, 4, fp);
        fwrite(ht.data(), 8, tn, fp);
        fclose(fp);
      }
    }
  }
  if (e != hipSuccess) return seterr(FG_EHIP, "persistent decode launch: %s", hipGetErrorString(e));
  return FG_OK;
}

// The whole greedy loop as one persistent launch: ids go to kv->d_out,
// logits (when wanted) to kv->d_lgs.
int32_t fused_decode(fg_model* m, fg_kv* kv, const int32_t* ids, int n_steps, int with_logits) {
  HIPCHK(hipMemcpyAsync(kv->d_ids, ids, 4, hipMemcpyHostToDevice, m->stream));
  return fused_launch(m, kv, kv->d_ids, kv->len, n_steps, kv->d_out,
                      with_logits ? kv->d_lgs : nullptr, true);
}

// The persistent launch's error flag, after the device is idle: 0, or the
// engine error for it.
int32_t fused_check(fg_model* m) {
  uint32_t err = 0;
  HIPCHK(hipMemcpy(&err, m->fused_err, 4, hipMemcpyDeviceToHost));
  if (err != 0)
    return seterr(FG_EHIP, "persistent decode: %s",
                  err == 2 ? "an XCD held more than 32 of its workgroups"
                           : "a hand-over between workgroups timed out");
  return FG_OK;
}

}  // namespace

extern "C" int32_t fg_step(fg_model* m, fg_kv* kv, const int32_t* ids, float* logits,
                           int32_t* next_ids) {
  if (!m || !kv || !ids || kv->m != m) return seterr(FG_EARG, "bad argument");
  RCCHK(check_ids(m, ids, kv->B));
  GUARD(m);
  return kv_pass(m, kv, ids, 1, logits, next_ids);
}

// ------------------------------------------------------------ no-allocation step
// fg_step_dev_noalloc keeps the step's activations (x, q, attention output,
// relu2(fc)) and the single-query attention's per-chunk partials in this
// file-scope device array, one copy per GPU, instead of memory the library
// allocates. Its device address is taken once per device with
// hipGetSymbolAddress; host code uses only that address, never the name.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)4 << 20;
constexpr size_t NOALLOC_CNT_BYTES = 4096;  // at the start: attention arrival counters
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];
constexpr int NOALLOC_MAX_DEVICES = 64;
static std::mutex g_scratch_mu;  // also held while a call enqueues its work
static uint8_t* g_scratch_ptr[NOALLOC_MAX_DEVICES];
// The last uncaptured call on each device's array: its stream and an event
// recorded after its work, so that a call on another stream while that work
// is queued or running is refused (FG_EBUSY) instead of racing on the array.
struct ScratchUse {
  hipEvent_t ev = nullptr;
  hipStream_t last = nullptr;
  bool pending = false;
};
static ScratchUse g_scratch_use[NOALLOC_MAX_DEVICES];

namespace {

// The scratch array's address on device dev (current), looked up on first use.
int32_t scratch_on(int dev, uint8_t** out) {
  if (dev < 0 || dev >= NOALLOC_MAX_DEVICES)
    return seterr(FG_EARG, "device %d beyond the %d this build tracks", dev, NOALLOC_MAX_DEVICES);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return seterr(FG_EHIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    hipEvent_t ev = nullptr;
    const hipError_t e2 = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e2 != hipSuccess) return seterr(FG_EHIP, "hipEventCreate: %s", hipGetErrorString(e2));
    g_scratch_use[dev].ev = ev;
    g_scratch_ptr[dev] = (uint8_t*)p;
  }
  *out = g_scratch_ptr[dev];
  return FG_OK;
}

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

}  // namespace

// gpt_step for the kv's B sequences on device buffers with no allocation:
// the kernels of fg_step's single-row path (GEMV linears, single-query
// attention, argmax), their scratch in the array above.
extern "C" int32_t fg_step_dev_noalloc(fg_model* m, fg_kv* kv, const int32_t* d_ids,
                                       float* d_logits, int32_t* d_next, void* stream) {
  if (!m || !kv || !d_ids || !d_logits || kv->m != m) return seterr(FG_EARG, "bad argument");
  GUARD(m);
  const Dims& d = m->d;
  const int B = kv->B;
  if (use_gemm(d, B))
    return seterr(FG_EARG, "fg_step_dev_noalloc serves the single-row path: %d sequences at "
                           "d_model %d need the GEMM path (at most %d here)",
                  B, d.D, d.dff * 4 * 4 > 65536 ? 65536 / (d.dff * 4) : 4);
  if (kv->len + 1 > kv->maxT)
    return seterr(FG_EFULL, "cache full (raise maxT): len %d + 1 > %d", kv->len, kv->maxT);
  RCCHK(check_rope(m, kv->len + 1));
  // [arrival counters][activations][attention partials]: the counters sit
  // at a fixed place nothing else writes, so they stay zero between calls
  const size_t act = align256((size_t)B * (d.D + 2 * d.qd() + d.dff) * 4);
  const size_t part = (size_t)attn_decode_scratch_floats(d, B, kv->maxT) * 4;
  if (NOALLOC_CNT_BYTES + act + part > NOALLOC_SCRATCH_BYTES)
    return seterr(FG_EARG, "this step needs %zu bytes of scratch (B=%d, maxT=%d), above the %zu "
                           "the library holds",
                  NOALLOC_CNT_BYTES + act + part, B, kv->maxT, NOALLOC_SCRATCH_BYTES);
  uint8_t* sp = nullptr;
  RCCHK(scratch_on(m->device, &sp));
  Work w;
  w.rows = B;
  w.x = (float*)(sp + NOALLOC_CNT_BYTES);
  w.q = w.x + (size_t)B * d.D;
  w.ao = w.q + (size_t)B * d.qd();
  w.h = w.ao + (size_t)B * d.qd();
  float* dec_part = (float*)(sp + NOALLOC_CNT_BYTES + act);
  hipStream_t s = stream ? (hipStream_t)stream : m->stream;
  // Calls under graph capture are not tracked (their replays are ordered
  // by the caller); an uncaptured call waits for no one: it is refused if
  // another stream's call may still be using the array.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  HIPCHK(hipStreamIsCapturing(s, &cap));
  const bool track = cap == hipStreamCaptureStatusNone;
  std::lock_guard<std::mutex> use_lk(g_scratch_mu);
  ScratchUse& use = g_scratch_use[m->device];
  if (track && use.pending && use.last != s) {
    const hipError_t q = hipEventQuery(use.ev);
    if (q == hipErrorNotReady)
      return seterr(FG_EBUSY, "the no-allocation scratch of device %d is in use by a call on "
                              "another stream that has not finished",
                    m->device);
    if (q != hipSuccess) return seterr(FG_EHIP, "hipEventQuery: %s", hipGetErrorString(q));
  }
  const bool tm = m->timing;  // (timing records events: not on this path)
  m->timing = false;
  PassOpts o;
  o.kv16 = kv->kv16;
  // (beyond the counters' room the attention merges in a kernel of its own)
  if ((size_t)attn_decode_counters(d, B) * 4 <= NOALLOC_CNT_BYTES) o.dec_cnt = (uint32_t*)sp;
  layer_stack(m, s, d_ids, B, 1, kv->len, nullptr, kv->k, kv->v, kv->maxT,
              (int64_t)B * kv->maxT * d.kvd(), dec_part, d_logits, o, &w);
  if (d_next) launch_argmax(s, d_logits, B, d.V, d_next);
  m->timing = tm;
  HIPCHK(hipGetLastError());
  if (track) {
    HIPCHK(hipEventRecord(use.ev, s));
    use.last = s;
    use.pending = true;
  }
  kv->len += 1;
  kv->filled = std::max(kv->filled, kv->len);
  return FG_OK;
}

extern "C" int32_t fg_step_multi(fg_model* m, fg_kv* kv, const int32_t* ids, int32_t TB,
                                 float* logits, int32_t* next_ids) {
  if (!m || !kv || !ids || kv->m != m) return seterr(FG_EARG, "bad argument");
  if (TB < 1) return seterr(FG_EARG, "TB must be >= 1");
  RCCHK(check_ids(m, ids, (int64_t)kv->B * TB));
  GUARD(m);
  return kv_pass(m, kv, ids, TB, logits, next_ids);
}

extern "C" int32_t fg_decode_greedy(fg_model* m, fg_kv* kv, const int32_t* ids, int32_t n_steps,
                                    int32_t* ids_out, float* logits_out) {
  if (!m || !kv || !ids || !ids_out || kv->m != m) return seterr(FG_EARG, "bad argument");
  if (n_steps < 1) return seterr(FG_EARG, "n_steps must be >= 1");
  RCCHK(check_ids(m, ids, kv->B));
  GUARD(m);
  const int B = kv->B;
  if (kv->len + n_steps > kv->maxT)
    return seterr(FG_EFULL, "cache full (raise maxT): len %d + %d > %d", kv->len, n_steps,
                  kv->maxT);
  if (n_steps > (1 << 20)) return seterr(FG_EARG, "n_steps %d above 2^20", n_steps);
  RCCHK(check_rope(m, kv->len + n_steps));
  RCCHK(ensure_work(m, B));
  hipStream_t s = m->stream;
  const int64_t nout = (int64_t)n_steps * B;
  if (nout > kv->cap_out) {
    if (kv->d_out) HIPCHK(hipFree(kv->d_out));
    HIPCHK(hipMalloc((void**)&kv->d_out, nout * 4));
    RCCHK(dev_zero(m, kv->d_out, (size_t)nout * 4));
    kv->cap_out = nout;
    for (auto& g : kv->graphs) (void)hipGraphExecDestroy(g.second);
    kv->graphs.clear();
  }
  const int with_logits = logits_out ? 1 : 0;
  const int64_t nlg = with_logits ? nout * m->d.V : (int64_t)B * m->d.V;
  if (nlg > kv->cap_lgs) {
    if (kv->d_lgs) HIPCHK(hipFree(kv->d_lgs));
    HIPCHK(hipMalloc((void**)&kv->d_lgs, nlg * 4));
    RCCHK(dev_zero(m, kv->d_lgs, (size_t)nlg * 4));
    kv->cap_lgs = nlg;
    for (auto& g : kv->graphs) (void)hipGraphExecDestroy(g.second);
    kv->graphs.clear();
  }
  if (kv->graphs_gen != m->gen) {
    for (auto& g : kv->graphs) (void)hipGraphExecDestroy(g.second);
    kv->graphs.clear();
    kv->graphs_gen = m->gen;
  }
  const bool fused = fused_applies(m, kv, n_steps);
  if (fused) {
    RCCHK(fused_decode(m, kv, ids, n_steps, with_logits));
  } else {
    RCCHK(graph_decode(m, kv, ids, n_steps, with_logits));
  }
  HIPCHK(hipMemcpyAsync(ids_out, kv->d_out, nout * 4, hipMemcpyDeviceToHost, s));
  if (logits_out) RCCHK(copy_out(m, logits_out, kv->d_lgs, (size_t)nout * m->d.V * 4, s));
  HIPCHK(hipStreamSynchronize(s));
  if (fused) RCCHK(fused_check(m));
  kv->len += n_steps;
  kv->filled = std::max(kv->filled, kv->len);
  return FG_OK;
}


namespace {

// One round of the speculative loop, all on the device: draft (lookup and
// the pass's ids), the verification pass over up to `maxr` rows (the live
// count and the cache length come from the state: every row a single step,
// as gpt_step computes it), commit (argmax, accept, controller).
void spec_round_launches(fg_model* m, fg_kv* kv, hipStream_t s, int maxr, int pos_host) {
  SpecDev* st = kv->d_sst;
  timed(m, s, FG_K_OTHER, 0, 0, [&] { launch_spec_draft(s, st, kv->d_sids); });
  PassOpts o;
  o.pos_host = pos_host;
  o.rows_single = true;
  o.d_rows = &st->rows;
  o.kv16 = kv->kv16;
  o.dec_cnt = kv->d_dcnt;
  layer_stack(m, s, st->inp, 1, maxr, 0, &st->len, kv->k, kv->v, kv->maxT,
              (int64_t)kv->maxT * m->d.kvd(), kv->d_spart, m->ws.logits, o);
  timed(m, s, FG_K_OTHER, 0, (double)maxr * m->d.V * 4, [&] {
    launch_spec_commit(s, st, m->ws.logits, m->d.V, kv->d_sids);
  });
}

// `rounds` rounds, replayed from a graph captured on first use (eager when
// timing is on).
int32_t spec_rounds(fg_model* m, fg_kv* kv, int rounds, int maxr, int pos_host) {
  hipStream_t s = m->stream;
  if (m->timing) {
    for (int r = 0; r < rounds; ++r) spec_round_launches(m, kv, s, maxr, pos_host);
    return FG_OK;
  }
  const auto key = std::make_pair(rounds, 100 + maxr);
  auto it = kv->graphs.find(key);
  if (it == kv->graphs.end()) {
    hipGraph_t g = nullptr;
    HIPCHK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    for (int r = 0; r < rounds; ++r) spec_round_launches(m, kv, s, maxr, -1);
    HIPCHK(hipStreamEndCapture(s, &g));
    hipGraphExec_t ge = nullptr;
    hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return seterr(FG_EHIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
    it = kv->graphs.emplace(key, ge).first;
  }
  HIPCHK(hipGraphLaunch(it->second, s));
  return FG_OK;
}

}  // namespace

// The draft/verify/commit loop of src/app/chat_text.f90:293-422 at
// temperature 0 with the prompt-lookup drafter and the sliding-window
// controller, resident on the device: the host replays runs of captured
// rounds and reads the state back once per run. Every round commits at
// least one id, so a run never holds more rounds than ids remain and no
// round is spent past n_total.
extern "C" int32_t fg_decode_spec(fg_model* m, fg_kv* kv, int32_t* ids, int32_t n_known,
                                  int32_t n_total, const fg_spec_cfg* cfg,
                                  fg_spec_stats* stats) {
  if (!m || !kv || !ids || !cfg || kv->m != m) return seterr(FG_EARG, "bad argument");
  if (kv->B != 1) return seterr(FG_EARG, "speculative decoding runs one sequence (B=1), not %d",
                                kv->B);
  if (cfg->k < 1 || cfg->k > GEMV_MAX_ROWS - 1)
    return seterr(FG_EARG, "k = %d outside [1, %d]", cfg->k, GEMV_MAX_ROWS - 1);
  if (cfg->match < 1) return seterr(FG_EARG, "match = %d must be >= 1", cfg->match);
  if (cfg->probe < 1) return seterr(FG_EARG, "probe = %d must be >= 1", cfg->probe);
  if (n_known < 1 || n_total < n_known)
    return seterr(FG_EARG, "need 1 <= n_known (%d) <= n_total (%d)", n_known, n_total);
  if (kv->len != n_known - 1)
    return seterr(FG_EARG, "cache holds %d positions, expected n_known-1 = %d", kv->len,
                  n_known - 1);
  if (n_total > kv->maxT)
    return seterr(FG_EFULL, "cache full (raise maxT): n_total %d > %d", n_total, kv->maxT);
  RCCHK(check_ids(m, ids, n_known));
  GUARD(m);
  if (stats) *stats = fg_spec_stats{0, 0, 0, 0, 0};
  if (n_total == n_known) return FG_OK;
  const int maxr = cfg->k + 1;
  RCCHK(check_rope(m, n_total));
  RCCHK(ensure_work(m, maxr));
  if (!kv->d_sids) {
    HIPCHK(hipMalloc((void**)&kv->d_sids, (size_t)kv->maxT * 4));
    RCCHK(dev_zero(m, kv->d_sids, (size_t)kv->maxT * 4));
  }
  if (!kv->d_sst) {
    const size_t spb = (size_t)attn_decode_scratch_floats(m->d, GEMV_MAX_ROWS, kv->maxT) * 4;
    HIPCHK(hipMalloc((void**)&kv->d_sst, sizeof(SpecDev)));
    HIPCHK(hipHostMalloc((void**)&kv->h_sst, sizeof(SpecDev), hipHostMallocDefault));
    HIPCHK(hipMalloc((void**)&kv->d_spart, spb));
    RCCHK(dev_zero(m, kv->d_sst, sizeof(SpecDev)));
    RCCHK(dev_zero(m, kv->d_spart, spb));
  }
  if (kv->graphs_gen != m->gen) {
    for (auto& g : kv->graphs) (void)hipGraphExecDestroy(g.second);
    kv->graphs.clear();
    kv->graphs_gen = m->gen;
  }
  SpecDev* h = kv->h_sst;
  memset(h, 0, sizeof *h);
  h->pp = n_known;
  h->n_total = n_total;
  h->len = n_known - 1;
  h->mode_spec = 1;
  h->k = cfg->k;
  h->match = cfg->match;
  h->probe = cfg->probe;
  h->min_acc = cfg->min_acc;
  hipStream_t s = m->stream;
  HIPCHK(hipMemcpyAsync(kv->d_sids, ids, (size_t)n_known * 4, hipMemcpyHostToDevice, s));
  HIPCHK(hipMemcpyAsync(kv->d_sst, h, sizeof *h, hipMemcpyHostToDevice, s));
  HIPCHK(hipStreamSynchronize(s));
  int pp = n_known;
  while (pp < n_total) {
    int rounds = 16;
    while (rounds > n_total - pp) rounds >>= 1;
    const int32_t rc = spec_rounds(m, kv, rounds, maxr, pp - 1);
    if (rc == FG_OK) {
      HIPCHK(hipMemcpyAsync(h, kv->d_sst, sizeof *h, hipMemcpyDeviceToHost, s));
      HIPCHK(hipStreamSynchronize(s));
    }
    if (rc != FG_OK || h->pp <= pp) {  // (every round commits at least one id)
      kv->len = pp - 1;
      return rc != FG_OK ? rc : seterr(FG_EHIP, "speculative rounds made no progress");
    }
    pp = h->pp;
  }
  HIPCHK(hipMemcpyAsync(ids + n_known, kv->d_sids + n_known, (size_t)(n_total - n_known) * 4,
                        hipMemcpyDeviceToHost, s));
  HIPCHK(hipStreamSynchronize(s));
  kv->len = n_total - 1;
  kv->filled = std::max(kv->filled, kv->len);
  if (stats) *stats = fg_spec_stats{h->passes, h->accepted, h->proposed, h->plain, h->pauses};
  return FG_OK;
}

// ------------------------------------------------------------------ sampling
namespace {

int32_t check_sample_cfg(const fg_sample_cfg* c, int V, SampleCfg* out) {
  if (!c) return seterr(FG_EARG, "NULL sampling config");
  if (V < 1 || V > SAMPLE_MAX_V)
    return seterr(FG_EDIMS, "sampling takes 1 <= V <= %d ids, not %d", SAMPLE_MAX_V, V);
  if (c->nblock < 0 || c->pwin < 0) return seterr(FG_EARG, "nblock and pwin must be >= 0");
  out->temp = c->temp;
  out->topp = c->topp;
  out->pres = c->pres;
  out->freq = c->freq;
  out->rep = c->rep;
  out->plen = c->plen;
  out->pwin = c->pwin;
  out->nblock = c->nblock;
  out->byte_space = c->byte_space != 0;
  return FG_OK;
}

}  // namespace

// sample_next (src/lib/sample.f90:153-233) over one host row of V logits on
// the device: history gen[0:ngen], the generator state advanced in place.
extern "C" int32_t fg_sample(fg_model* m, const float* logits, int32_t V, const int32_t* gen,
                             int32_t ngen, const fg_sample_cfg* cfg, int64_t* state,
                             int32_t* id) {
  if (!m || !logits || !state || !id || ngen < 0 || (ngen > 0 && !gen))
    return seterr(FG_EARG, "bad argument");
  SampleCfg c;
  RCCHK(check_sample_cfg(cfg, V, &c));
  GUARD(m);
  const int64_t need = (int64_t)V * 4 + (int64_t)ngen * 4 + 64;
  if (need > m->samp_bytes) {
    if (m->samp) HIPCHK(hipFree(m->samp));
    m->samp = nullptr;
    m->samp_bytes = 0;
    HIPCHK(hipMalloc((void**)&m->samp, need));
    RCCHK(dev_zero(m, m->samp, (size_t)need));
    m->samp_bytes = need;
  }
  int64_t* d_state = (int64_t*)m->samp;
  int32_t* d_id = (int32_t*)(m->samp + 8);
  float* d_lg = (float*)(m->samp + 64);
  int32_t* d_gen = (int32_t*)(m->samp + 64 + (int64_t)V * 4);
  hipStream_t s = m->stream;
  HIPCHK(hipMemcpyAsync(d_state, state, 8, hipMemcpyHostToDevice, s));
  HIPCHK(hipMemcpyAsync(d_lg, logits, (size_t)V * 4, hipMemcpyHostToDevice, s));
  if (ngen > 0) HIPCHK(hipMemcpyAsync(d_gen, gen, (size_t)ngen * 4, hipMemcpyHostToDevice, s));
  launch_sample_one(s, d_lg, V, d_gen, ngen, c, d_state, d_id);
  HIPCHK(hipGetLastError());
  HIPCHK(hipMemcpyAsync(state, d_state, 8, hipMemcpyDeviceToHost, s));
  HIPCHK(hipMemcpyAsync(id, d_id, 4, hipMemcpyDeviceToHost, s));
  HIPCHK(hipStreamSynchronize(s));
  return FG_OK;
}

namespace {

// One step of the sampling loop: the pass over inp[0] at the device-held
// cache length, then the sampled id (history = the ids generated so far).
void sample_step_launches(fg_model* m, fg_kv* kv, hipStream_t s, int pos_host) {
  SampleDev* sd = kv->d_smp;
  PassOpts o;
  o.pos_host = pos_host;
  o.kv16 = kv->kv16;
  o.dec_cnt = kv->d_dcnt;
  layer_stack(m, s, sd->inp, 1, 1, 0, &sd->len, kv->k, kv->v, kv->maxT,
              (int64_t)kv->maxT * m->d.kvd(), kv->d_part, m->ws.logits, o);
  timed(m, s, FG_K_OTHER, 0, (double)m->d.V * 4, [&] {
    launch_sample_step(s, sd, m->ws.logits, m->d.V, kv->d_sids);
  });
}

int32_t sample_steps(fg_model* m, fg_kv* kv, int steps, int pos_host) {
  hipStream_t s = m->stream;
  if (m->timing) {
    for (int r = 0; r < steps; ++r) sample_step_launches(m, kv, s, pos_host + r);
    return FG_OK;
  }
  const auto key = std::make_pair(steps, 200);
  auto it = kv->graphs.find(key);
  if (it == kv->graphs.end()) {
    hipGraph_t g = nullptr;
    HIPCHK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    for (int r = 0; r < steps; ++r) sample_step_launches(m, kv, s, -1);
    HIPCHK(hipStreamEndCapture(s, &g));
    hipGraphExec_t ge = nullptr;
    hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return seterr(FG_EHIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
    it = kv->graphs.emplace(key, ge).first;
  }
  HIPCHK(hipGraphLaunch(it->second, s));
  return FG_OK;
}

}  // namespace

// The plain decode loop of src/app/chat_text.f90:423-462 with sample_next:
// one cached step per id, each id drawn from that step's logits with the
// ids generated so far as the penalty history, on the device. Captured runs
// of steps are replayed; every step commits one id, so the runs add up to
// exactly n_total - n_known steps.
extern "C" int32_t fg_decode_sample(fg_model* m, fg_kv* kv, int32_t* ids, int32_t n_known,
                                    int32_t n_total, const fg_sample_cfg* cfg, int64_t* state) {
  if (!m || !kv || !ids || !state || kv->m != m) return seterr(FG_EARG, "bad argument");
  if (kv->B != 1) return seterr(FG_EARG, "sampled decoding runs one sequence (B=1), not %d", kv->B);
  SampleCfg c;
  RCCHK(check_sample_cfg(cfg, m->d.V, &c));
  if (n_known < 1 || n_total < n_known)
    return seterr(FG_EARG, "need 1 <= n_known (%d) <= n_total (%d)", n_known, n_total);
  if (kv->len != n_known - 1)
    return seterr(FG_EARG, "cache holds %d positions, expected n_known-1 = %d", kv->len,
                  n_known - 1);
  if (n_total > kv->maxT)
    return seterr(FG_EFULL, "cache full (raise maxT): n_total %d > %d", n_total, kv->maxT);
  RCCHK(check_ids(m, ids, n_known));
  GUARD(m);
  if (n_total == n_known) return FG_OK;
  RCCHK(check_rope(m, n_total));
  RCCHK(ensure_work(m, 1));
  if (!kv->d_sids) {
    HIPCHK(hipMalloc((void**)&kv->d_sids, (size_t)kv->maxT * 4));
    RCCHK(dev_zero(m, kv->d_sids, (size_t)kv->maxT * 4));
  }
  if (!kv->d_smp) {
    HIPCHK(hipMalloc((void**)&kv->d_smp, sizeof(SampleDev)));
    RCCHK(dev_zero(m, kv->d_smp, sizeof(SampleDev)));
    HIPCHK(hipHostMalloc((void**)&kv->h_smp, sizeof(SampleDev), hipHostMallocDefault));
  }
  if (kv->graphs_gen != m->gen) {
    for (auto& g : kv->graphs) (void)hipGraphExecDestroy(g.second);
    kv->graphs.clear();
    kv->graphs_gen = m->gen;
  }
  SampleDev* h = kv->h_smp;
  memset(h, 0, sizeof *h);
  h->pp = n_known;
  h->n_total = n_total;
  h->len = n_known - 1;
  h->n_known = n_known;
  h->rng = *state;
  h->inp[0] = ids[n_known - 1];
  h->cfg = c;
  hipStream_t s = m->stream;
  HIPCHK(hipMemcpyAsync(kv->d_sids, ids, (size_t)n_known * 4, hipMemcpyHostToDevice, s));
  HIPCHK(hipMemcpyAsync(kv->d_smp, h, sizeof *h, hipMemcpyHostToDevice, s));
  int done = 0;
  const int total = n_total - n_known;
  const bool fused = fused_applies(m, kv, total);
  if (fused) {
    // each step the persistent kernel for one step (its logits; its own
    // argmax goes to the spare inp[1]), then the draw, which leaves the next
    // input in inp[0]; the error flag is cleared once and read at the end
    int32_t* inp = (int32_t*)((char*)kv->d_smp + offsetof(SampleDev, inp));
    HIPCHK(hipMemsetAsync(m->fused_err, 0, 4, s));
    for (; done < total; ++done) {
      const int32_t rc = fused_launch(m, kv, inp, n_known - 1 + done, 1, inp + 1,
                                      m->ws.logits, false);
      if (rc != FG_OK) {
        (void)hipStreamSynchronize(s);
        kv->len = n_known - 1;
        return rc;
      }
      timed(m, s, FG_K_OTHER, 0, (double)m->d.V * 4, [&] {
        launch_sample_step(s, kv->d_smp, m->ws.logits, m->d.V, kv->d_sids);
      });
    }
  }
  while (done < total) {
    int run = 32;
    while (run > total - done) run >>= 1;
    const int32_t rc = sample_steps(m, kv, run, n_known - 1 + done);
    if (rc != FG_OK) {
      (void)hipStreamSynchronize(s);
      kv->len = n_known - 1;
      return rc;
    }
    done += run;
  }
  HIPCHK(hipMemcpyAsync(h, kv->d_smp, sizeof *h, hipMemcpyDeviceToHost, s));
  HIPCHK(hipMemcpyAsync(ids + n_known, kv->d_sids + n_known, (size_t)total * 4,
                        hipMemcpyDeviceToHost, s));
  HIPCHK(hipStreamSynchronize(s));
  if (fused) {
    const int32_t rc = fused_check(m);
    if (rc != FG_OK) {
      kv->len = n_known - 1;
      return rc;
    }
  }
  if (h->pp != n_total) return seterr(FG_EHIP, "sampling loop ended at %d of %d", h->pp, n_total);
  *state = h->rng;
  kv->len = n_total - 1;
  kv->filled = std::max(kv->filled, kv->len);
  return FG_OK;
}

namespace {

// The fp16 copy of the GEMM weights for FG_OPT_FORWARD_F16: every bf16
// weight times 2^k, k the largest integer <= 15 with max|w| 2^k <= 32768,
// so the copy holds each weight exactly unless it is below ~2^-(24+k-7)
// (a bf16 has 8 significant bits; fp16 resolves 2^-24).
int32_t ensure_w16(fg_model* m) {
  if (m->w16) return FG_OK;
  int k = 15;
  while (k > -15 && m->wmax * std::ldexp(1.0f, k) > 32768.f) --k;
  if (m->wmax * std::ldexp(1.0f, k) > 32768.f)
    return seterr(FG_EARG, "weights up to %g exceed what fp16 holds", (double)m->wmax);
  const size_t n = m->w.layer_stride * m->d.L + (size_t)m->d.V * m->d.D;  // layers + lm_head
  HIPCHK(hipMalloc((void**)&m->w16, m->w.bytes));  // (the arena's size: offsets stay valid)
  m->w16_scale = std::ldexp(1.0f, k);
  m->w16_inv = std::ldexp(1.0f, -k);
  launch_to_f16(m->stream, m->w.base, m->w16, (int64_t)n, m->w16_scale);
  HIPCHK(hipStreamSynchronize(m->stream));
  return FG_OK;
}

}  // namespace

extern "C" int32_t fg_set_option(fg_model* m, int32_t key, int32_t value) {
  if (!m) return seterr(FG_EARG, "NULL argument");
  if (key != FG_OPT_FUSED_DECODE && key != FG_OPT_FORWARD_F16)
    return seterr(FG_EARG, "unknown option %d", key);
  GUARD(m);
  if (key == FG_OPT_FUSED_DECODE) {
    m->fused_on = value != 0;
  } else {
    if (value) {
      RCCHK(ensure_w16(m));
    } else if (m->w16) {
      // the copy goes with the option; passes queued on any stream (the
      // device-pointer entries take the caller's) may still read it
      HIPCHK(hipDeviceSynchronize());
      HIPCHK(hipFree(m->w16));
      m->w16 = nullptr;
    }
    m->fwd_f16 = value != 0;
  }
  return FG_OK;
}

extern "C" int32_t fg_get_option(fg_model* m, int32_t key, int32_t* value, char* why,
                                 int32_t len) {
  if (!m || !value) return seterr(FG_EARG, "NULL argument");
  if (key == FG_OPT_FORWARD_F16) {
    *value = m->fwd_f16 ? 1 : 0;
    if (why && len > 0) why[0] = '\0';
    return FG_OK;
  }
  if (key != FG_OPT_FUSED_DECODE) return seterr(FG_EARG, "unknown option %d", key);
  *value = (m->fused_on && m->fused_w) ? 1 : 0;
  if (why && len > 0) {
    const char* r = !m->fused_on ? "disabled by fg_set_option" : m->fused_w ? "" : m->fused_why.c_str();
    strncpy(why, r, (size_t)len - 1);
    why[len - 1] = '\0';
  }
  return FG_OK;
}

extern "C" int32_t fg_sync(fg_model* m) {
  if (!m) return seterr(FG_EARG, "NULL argument");
  GUARD(m);
  HIPCHK(hipStreamSynchronize(m->stream));
  return check_f16_range(m, m->stream);
}

extern "C" int32_t fg_timing(fg_model* m, int32_t enable) {
  if (!m) return seterr(FG_EARG, "NULL argument");
  GUARD(m);
  HIPCHK(hipStreamSynchronize(m->stream));
  for (auto& r : m->trecs) {
    m->evpool.push_back(r.a);
    m->evpool.push_back(r.b);
  }
  m->trecs.clear();
  m->timing = enable != 0;
  return FG_OK;
}

extern "C" int32_t fg_timing_read(fg_model* m, int32_t kind, int64_t* launches, double* ms,
                                  double* flops, double* bytes) {
  if (!m) return seterr(FG_EARG, "NULL argument");
  if (kind < 0 || kind >= FG_K_NKINDS) return seterr(FG_EARG, "kind %d out of range", kind);
  GUARD(m);
  HIPCHK(hipStreamSynchronize(m->stream));
  int64_t n = 0;
  double t = 0, f = 0, b = 0;
  for (auto& r : m->trecs) {
    if (r.kind != kind) continue;
    float e = 0.f;
    // (launches on a caller's stream: wait for the record's own end event)
    HIPCHK(hipEventSynchronize(r.b));
    HIPCHK(hipEventElapsedTime(&e, r.a, r.b));
    ++n;
    t += e;
    f += r.flops;
    b += r.bytes;
  }
  if (launches) *launches = n;
  if (ms) *ms = t;
  if (flops) *flops = f;
  if (bytes) *bytes = b;
  return FG_OK;
}

extern "C" int32_t fg_model_bytes(const fg_model* m, int64_t* weight_bytes, int64_t* work_bytes) {
  if (!m) return seterr(FG_EARG, "NULL argument");
  if (weight_bytes) *weight_bytes = (int64_t)m->w.bytes * (m->w16 ? 2 : 1);  // + the fp16 copy
  if (work_bytes) *work_bytes = m->work_bytes;
  return FG_OK;
}
