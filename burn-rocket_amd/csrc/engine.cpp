// C-ABI engine: process-global device context, resident weight registry,
// per-shape scratch and the op entry points declared in burn_rocket_amd.h.
//
// Mirrors the reference extension's engine (crates/burn-rocket/src/ext.rs:
// Engine ext.rs:518-535, init ext.rs:561-580, weight kinds ext.rs:1156-1181,
// matmul_impl ext.rs:1208-1232, attention_impl ext.rs:1669-1858) with the
// NPU driver calls replaced by HIP kernel launches on one stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <mutex>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "../../include/burn_rocket_amd.h"
#include "kernels.hpp"
#include "stage.hpp"

static inline int64_t round_up_i(int64_t a, int64_t b) { return (a + b - 1) / b * b; }

namespace {

thread_local std::string g_last_error;

const char *status_text(int rc) {
  switch (rc) {
    case RK_E_SHAPE: return "unsupported shape";
    case RK_E_TILING: return "shape not tileable";
    case RK_E_NOMEM: return "allocation failed";
    case RK_E_DEVICE: return "device/driver failure";
    case RK_E_UNSUPPORTED: return "unsupported feature";
    case RK_E_RANGE: return "value out of range";
    case RK_E_IO: return "i/o failure";
  }
  return "unknown error";
}

int fail(int rc, const char *op, const std::string &detail) {
  g_last_error = std::string(op) + " failed: " + status_text(rc) + " (rc=" + std::to_string(rc) +
                 ")" + (detail.empty() ? "" : ": " + detail);
  return rc;
}

int hip_fail(hipError_t e, const char *op) {
  const int rc = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) ? RK_E_NOMEM
                                                                             : RK_E_DEVICE;
  return fail(rc, op, hipGetErrorString(e));
}

#define HIP_TRY(expr, op)                         \
  do {                                            \
    hipError_t e_ = (expr);                       \
    if (e_ != hipSuccess) return hip_fail(e_, op); \
  } while (0)

#define RK_TRY(expr)          \
  do {                        \
    int rc_ = (expr);         \
    if (rc_ != RK_OK) return rc_; \
  } while (0)

// A named device scratch buffer and the point after the last call that used
// it: a call on another stream first waits for that point, and the buffer is
// freed only once it has passed. On a caller's stream the point is an event
// recorded when the call returns. On a stream the library owns (its own, or
// one from rk_stream_create) nothing is recorded per call: the event is
// recorded on that stream only when another stream or a free needs the point
// (everything enqueued there by then includes the last use). An event record
// costs the GPU ~5 µs after the preceding kernel on MI355X, a large share of
// the short ops when it was paid per call and buffer.
struct DevBuf {
  void *p = nullptr;
  size_t bytes = 0;
  hipEvent_t ev = nullptr;
  hipStream_t ev_stream = nullptr;  // stream of the last call that used the buffer
  bool recorded = false;            // ev marks the end of that call's work
  bool pending = false;             // that call ran on a library stream; ev not recorded yet
  uint64_t epoch = 0;               // Engine::epoch at its last use
};

struct Weight {
  int kind = 0;
  int64_t n = 0, k = 0, group = 0;
  void *codes = nullptr;     // fp16 [N,K] or int8 [N,K]
  float *scales = nullptr;   // I8: [N, ws_stride] per 32-block; QAT: [N]
  int ws_stride = 0;
  bool ws_f16 = false;       // I8: every block scale is an fp16 value (GGUF Q8_0 d)
  int64_t glu_n = 0;  // > 0: gate|up rows interleaved for rk_matmul_w8a8_glu_dev, n = glu_n outputs
  float in_scale = 0.f, out_scale = 0.f;
  size_t bytes = 0;
  // MoE expert stack (kind 0, moe = true)
  bool moe = false;
  int n_experts = 0;
  int64_t hidden = 0, inter = 0;
  int8_t *gu_codes = nullptr, *dn_codes = nullptr;
  float *gu_scales = nullptr, *dn_scales = nullptr;
  int gu_ws_stride = 0, dn_ws_stride = 0;
};

struct Engine {
  int device = 0;
  hipStream_t stream = nullptr;
  std::unordered_set<hipStream_t> own_streams;  // made by rk_stream_create
  int num_cus = 256;
  std::unordered_map<uint64_t, Weight> weights;
  uint64_t next_id = 1;
  std::unordered_map<std::string, DevBuf> scratch;
  double convert_s = 0, device_s = 0;
  uint64_t calls = 0;
  rkstage::HostStage stage;  // page-locked staging of the host-buffer entries
  uint64_t epoch = 0;        // rk_trim_scratch: scratch not used since the last trim goes
};

std::mutex g_mu;
Engine *g_eng = nullptr;

using Clock = std::chrono::steady_clock;
double secs(Clock::time_point a, Clock::time_point b) {
  return std::chrono::duration<double>(b - a).count();
}

int ensure(const char *op) {
  if (!g_eng) return fail(RK_E_DEVICE, op, "rk_init() has not been called");
  HIP_TRY(hipSetDevice(g_eng->device), op);
  return RK_OK;
}

bool own_stream(hipStream_t s) { return s == g_eng->stream || g_eng->own_streams.count(s) != 0; }

// The stream of one entry-point call and the scratch buffers it took: when the
// call returns (its work is enqueued) each buffer notes the stream, and on a
// caller's stream gets its event recorded there (DevBuf).
struct CallScope {
  hipStream_t st;
  std::vector<DevBuf *> used;
  explicit CallScope(hipStream_t s) : st(s) {}
  CallScope(const CallScope &) = delete;
  CallScope &operator=(const CallScope &) = delete;
  ~CallScope() {
    const bool own = own_stream(st);
    for (DevBuf *b : used) {
      b->ev_stream = st;
      b->pending = own;
      b->recorded = false;
      if (!own && hipEventRecord(b->ev, st) == hipSuccess) b->recorded = true;
    }
  }
};

// Make b.ev mark the end of the buffer's last use (see DevBuf).
int fence_point(DevBuf &b, const char *op) {
  if (b.pending) {
    HIP_TRY(hipEventRecord(b.ev, b.ev_stream), op);
    b.pending = false;
    b.recorded = true;
  }
  return RK_OK;
}

// Grow-only named device scratch, ordered after its last use on any stream.
// *fresh (when given) tells whether this call allocated it.
int scratch(CallScope &c, const char *name, size_t bytes, void **out, bool *fresh = nullptr) {
  if (fresh) *fresh = false;
  DevBuf &b = g_eng->scratch[name];
  if (!b.ev) HIP_TRY(hipEventCreateWithFlags(&b.ev, hipEventDisableTiming), "scratch");
  if (b.bytes < bytes) {
    if (b.p) {
      RK_TRY(fence_point(b, "scratch"));
      if (b.recorded) HIP_TRY(hipEventSynchronize(b.ev), "scratch");
      HIP_TRY(hipFree(b.p), "scratch");
    }
    b.p = nullptr;
    b.bytes = 0;
    b.recorded = false;
    b.pending = false;
    const size_t want = std::max<size_t>(bytes, 256);
    HIP_TRY(hipMalloc(&b.p, want), "scratch");
    b.bytes = want;
    if (fresh) *fresh = true;
  } else if ((b.recorded || b.pending) && b.ev_stream != c.st) {
    RK_TRY(fence_point(b, "scratch"));
    HIP_TRY(hipStreamWaitEvent(c.st, b.ev, 0), "scratch");
  }
  if (std::find(c.used.begin(), c.used.end(), &b) == c.used.end()) c.used.push_back(&b);
  b.epoch = g_eng->epoch;
  *out = b.p;
  return RK_OK;
}

hipStream_t pick(rk_stream s) { return s ? (hipStream_t)s : g_eng->stream; }

// A host-buffer op through the page-locked staging (stage.hpp): `ins` go up,
// compute(r0, r1) enqueues the kernels of rows [r0, r1) on cs.st and returns
// an RK status, `outs` come down; row-sliced transfers move chunk by chunk so
// that uploads, kernels and downloads overlap. The op's kernel time (events
// around each chunk's kernels) is device_s; the rest of its wall time
// (copies and waits not hidden behind kernels) is convert_s.
int staged(CallScope &cs, const std::vector<rkstage::Xfer> &ins,
           const std::vector<rkstage::Xfer> &outs, int64_t rows, int64_t chunk_rows,
           const std::function<int(int64_t, int64_t)> &compute, const char *op) {
  HIP_TRY(g_eng->stage.setup(g_eng->device), op);
  const auto t0 = Clock::now();
  int crc = RK_OK;
  bool ok = true;
  float kms = 0.f;
  const hipError_t e = g_eng->stage.run(
      cs.st, ins, outs, rows, chunk_rows,
      [&](int64_t r0, int64_t r1) {
        crc = compute(r0, r1);
        return crc == RK_OK;
      },
      &ok, &kms);
  if (e != hipSuccess) return hip_fail(e, op);
  if (!ok) return crc;
  const double wall = secs(t0, Clock::now());
  g_eng->device_s += 1e-3 * kms;
  g_eng->convert_s += std::max(0.0, wall - 1e-3 * kms);
  return RK_OK;
}

// Rows per staged chunk: about 8 MiB of the larger of a row's input and
// output bytes, at most HostStage::kMaxChunks chunks, a multiple of 16 rows
// (so every chunk's device offsets keep 64-byte alignment).
int64_t stage_chunk_rows(int64_t rows, size_t in_row, size_t out_row) {
  const size_t per = std::max<size_t>({in_row, out_row, (size_t)1});
  int64_t c = std::max<int64_t>(1, (int64_t)(((size_t)8 << 20) / per));
  c = std::max<int64_t>(c, (rows + rkstage::HostStage::kMaxChunks - 1) / rkstage::HostStage::kMaxChunks);
  c = round_up_i(c, 16);
  return std::min<int64_t>(c, std::max<int64_t>(rows, 1));
}

Weight *find(uint64_t id) {
  auto it = g_eng->weights.find(id);
  return it == g_eng->weights.end() ? nullptr : &it->second;
}

uint64_t insert(Weight w) {
  const uint64_t id = g_eng->next_id++;
  g_eng->weights.emplace(id, w);
  return id;
}

// The device buffers of a weight being packed, freed if the pack fails before
// the weight is registered (register() hands them to the registry).
struct PackGuard {
  Weight &w;
  bool kept = false;
  explicit PackGuard(Weight &w_) : w(w_) {}
  PackGuard(const PackGuard &) = delete;
  PackGuard &operator=(const PackGuard &) = delete;
  uint64_t register_weight() {
    kept = true;
    return insert(w);
  }
  ~PackGuard() {
    if (kept) return;
    void *bufs[] = {w.codes, w.scales, w.gu_codes, w.dn_codes, w.gu_scales, w.dn_scales};
    for (void *b : bufs)
      if (b) (void)hipFree(b);
  }
};

int ws_stride_for(int64_t k) { return (int)round_up_i(k / 32, 4); }

}  // namespace

namespace {

// Upload per-block scales [n][kb] (kb = K/32 values per row) into a padded
// [n][ws_stride] device array.
int upload_block_scales(const std::vector<float> &blk, int64_t n, int64_t kb, float **dev,
                        int *stride_out, const char *op) {
  const int stride = ws_stride_for(kb * 32);
  std::vector<float> pad((size_t)n * stride, 0.f);
  for (int64_t r = 0; r < n; ++r)
    std::memcpy(&pad[(size_t)r * stride], &blk[(size_t)r * kb], sizeof(float) * kb);
  HIP_TRY(hipMalloc((void **)dev, pad.size() * sizeof(float)), op);
  HIP_TRY(hipMemcpy(*dev, pad.data(), pad.size() * sizeof(float), hipMemcpyHostToDevice), op);
  *stride_out = stride;
  return RK_OK;
}

int pack_f16_dev(const void *src_f16_dev, int64_t n, int64_t k, uint64_t *id) {
  Weight w;
  PackGuard guard(w);
  w.kind = RK_WEIGHT_F16;
  w.n = n;
  w.k = k;
  w.bytes = (size_t)n * k * 2;
  HIP_TRY(hipMalloc(&w.codes, w.bytes), "rk_pack");
  HIP_TRY(hipMemcpyAsync(w.codes, src_f16_dev, w.bytes, hipMemcpyDeviceToDevice, g_eng->stream),
          "rk_pack");
  HIP_TRY(hipStreamSynchronize(g_eng->stream), "rk_pack");
  *id = guard.register_weight();
  return RK_OK;
}

int check_f16_shape(int64_t n, int64_t k, const char *op) {
  if (n <= 0 || k <= 0) return fail(RK_E_SHAPE, op, "empty weight");
  if (k % 8 != 0) return fail(RK_E_SHAPE, op, "K must be a multiple of 8 (16-byte rows)");
  if (n > INT32_MAX || k > INT32_MAX) return fail(RK_E_SHAPE, op, "dimension too large");
  return RK_OK;
}

int check_i8_shape(int64_t n, int64_t k, int64_t group, const char *op) {
  if (n <= 0 || k <= 0) return fail(RK_E_SHAPE, op, "empty weight");
  if (group <= 0 || group % 32 != 0 || k % group != 0)
    return fail(RK_E_SHAPE, op, "group must be a positive multiple of 32 dividing K");
  return RK_OK;
}

}  // namespace

// =========================================================================
// Engine
// =========================================================================
extern "C" int rk_init(int device) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_eng) return RK_OK;
  int count = 0;
  HIP_TRY(hipGetDeviceCount(&count), "rk_init");
  if (device < 0 || device >= count)
    return fail(RK_E_DEVICE, "rk_init", "no HIP device " + std::to_string(device));
  HIP_TRY(hipSetDevice(device), "rk_init");
  // The static scratch of rk_attention_dev_noalloc, looked up once per device.
  HIP_TRY(rk_noalloc_setup(device), "rk_init");
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, device), "rk_init");
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(RK_E_UNSUPPORTED, "rk_init",
                std::string("kernels are built for gfx950, device is ") + prop.gcnArchName);
  Engine *e = new Engine();
  e->device = device;
  e->num_cus = prop.multiProcessorCount;
  hipError_t err = hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking);
  if (err != hipSuccess) {
    delete e;
    return hip_fail(err, "rk_init");
  }
  g_eng = e;
  return RK_OK;
}

extern "C" const char *rk_last_error(void) { return g_last_error.c_str(); }

extern "C" int rk_is_fallback(int rc) { return rc == RK_E_TILING ? 1 : 0; }

extern "C" int rk_stats(rk_stats_t *out) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_stats"));
  out->convert_s = g_eng->convert_s;
  out->device_s = g_eng->device_s;
  out->calls = g_eng->calls;
  return RK_OK;
}

extern "C" int rk_stats_reset(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_stats_reset"));
  g_eng->convert_s = g_eng->device_s = 0;
  g_eng->calls = 0;
  return RK_OK;
}

extern "C" int rk_mem_stats(rk_mem_stats_t *out) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_mem_stats"));
  out->weights_bytes = 0;
  out->scratch_bytes = 0;
  out->attention_bytes = 0;
  out->n_weights = g_eng->weights.size();
  out->n_scratch = g_eng->scratch.size();
  for (auto &kv : g_eng->weights) out->weights_bytes += kv.second.bytes;
  for (auto &kv : g_eng->scratch) {
    out->scratch_bytes += kv.second.bytes;
    if (kv.first.rfind("at", 0) == 0 || kv.first.rfind("fa_", 0) == 0)
      out->attention_bytes += kv.second.bytes;
  }
  out->host_bytes = g_eng->stage.pinned_bytes();
  return RK_OK;
}

namespace {
// Frees one named scratch buffer once its last use has completed.
int free_scratch(const std::string &name, const char *op) {
  DevBuf &b = g_eng->scratch[name];
  RK_TRY(fence_point(b, op));
  if (b.recorded) HIP_TRY(hipEventSynchronize(b.ev), op);
  HIP_TRY(hipFree(b.p), op);
  if (b.ev) (void)hipEventDestroy(b.ev);
  g_eng->scratch.erase(name);
  return RK_OK;
}
}  // namespace

extern "C" int rk_trim_scratch_to(uint64_t budget) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_trim_scratch_to"));
  // Largest buffers go first until the rest fits the budget.
  std::vector<std::pair<size_t, std::string>> order;
  uint64_t total = 0;
  for (auto &kv : g_eng->scratch) {
    order.push_back({kv.second.bytes, kv.first});
    total += kv.second.bytes;
  }
  std::sort(order.rbegin(), order.rend());
  for (auto &o : order) {
    if (total <= budget) break;
    RK_TRY(free_scratch(o.second, "rk_trim_scratch_to"));
    total -= o.first;
  }
  // A zero budget also returns the page-locked staging slots.
  if (budget == 0) HIP_TRY(g_eng->stage.release(), "rk_trim_scratch_to");
  return RK_OK;
}

extern "C" int rk_trim_scratch(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_trim_scratch"));
  // Scratch no call has used since the previous rk_trim_scratch goes; what
  // the calls in between used stays (the reference keeps the just-used shape
  // set, ext.rs:254-265).
  std::vector<std::string> old;
  for (auto &kv : g_eng->scratch)
    if (kv.second.epoch < g_eng->epoch) old.push_back(kv.first);
  for (auto &name : old) RK_TRY(free_scratch(name, "rk_trim_scratch"));
  g_eng->epoch++;
  return RK_OK;
}

extern "C" int rk_clear_scratch(void) { return rk_trim_scratch_to(0); }

// =========================================================================
// Weights
// =========================================================================
extern "C" int rk_pack(const float *w, int64_t n, int64_t k, rk_weight_id *id) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_pack"));
  RK_TRY(check_f16_shape(n, k, "rk_pack"));
  CallScope cs(g_eng->stream);
  void *x32, *x16;
  RK_TRY(scratch(cs, "pack_f32", (size_t)n * k * 4, &x32));
  RK_TRY(scratch(cs, "pack_f16", (size_t)n * k * 2, &x16));
  HIP_TRY(hipMemcpyAsync(x32, w, (size_t)n * k * 4, hipMemcpyHostToDevice, g_eng->stream), "rk_pack");
  HIP_TRY(rk_launch_f32_to_f16((const float *)x32, x16, n * k, g_eng->stream), "rk_pack");
  return pack_f16_dev(x16, n, k, id);
}

extern "C" int rk_pack_f16(const uint16_t *w, int64_t n, int64_t k, rk_weight_id *id) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_pack_f16"));
  RK_TRY(check_f16_shape(n, k, "rk_pack_f16"));
  CallScope cs(g_eng->stream);
  void *x16;
  RK_TRY(scratch(cs, "pack_f16", (size_t)n * k * 2, &x16));
  HIP_TRY(hipMemcpyAsync(x16, w, (size_t)n * k * 2, hipMemcpyHostToDevice, g_eng->stream),
          "rk_pack_f16");
  return pack_f16_dev(x16, n, k, id);
}

extern "C" int rk_pack_seg(const float *const *parts, const int64_t *ns, int nparts, int64_t k,
                           rk_weight_id *id) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_pack_seg"));
  if (nparts <= 0) return fail(RK_E_SHAPE, "rk_pack_seg", "no parts");
  int64_t n = 0;
  for (int i = 0; i < nparts; ++i) {
    if (ns[i] <= 0) return fail(RK_E_SHAPE, "rk_pack_seg", "empty part");
    n += ns[i];
  }
  RK_TRY(check_f16_shape(n, k, "rk_pack_seg"));
  CallScope cs(g_eng->stream);
  void *x32, *x16;
  RK_TRY(scratch(cs, "pack_f32", (size_t)n * k * 4, &x32));
  RK_TRY(scratch(cs, "pack_f16", (size_t)n * k * 2, &x16));
  int64_t off = 0;
  for (int i = 0; i < nparts; ++i) {
    HIP_TRY(hipMemcpyAsync((char *)x32 + off * k * 4, parts[i], (size_t)ns[i] * k * 4,
                           hipMemcpyHostToDevice, g_eng->stream),
            "rk_pack_seg");
    off += ns[i];
  }
  HIP_TRY(rk_launch_f32_to_f16((const float *)x32, x16, n * k, g_eng->stream), "rk_pack_seg");
  return pack_f16_dev(x16, n, k, id);
}

namespace {
int pack_i8_host(const int8_t *codes, const std::vector<float> &block_scales, int64_t n,
                 int64_t k, int64_t group, rk_weight_id *id, const char *op) {
  Weight w;
  PackGuard guard(w);
  w.kind = RK_WEIGHT_I8;
  w.n = n;
  w.k = k;
  w.group = group;
  HIP_TRY(hipMalloc(&w.codes, (size_t)n * k), op);
  HIP_TRY(hipMemcpy(w.codes, codes, (size_t)n * k, hipMemcpyHostToDevice), op);
  RK_TRY(upload_block_scales(block_scales, n, k / 32, &w.scales, &w.ws_stride, op));
  w.ws_f16 = std::all_of(block_scales.begin(), block_scales.end(),
                         [](float d) { return (float)(_Float16)d == d; });
  w.bytes = (size_t)n * k + (size_t)n * w.ws_stride * 4;
  *id = guard.register_weight();
  return RK_OK;
}

// Per-group scales [n, K/group] repeated over each group's 32-value blocks;
// null scales (codes packed alone, I8Context::pack_weight_gw) give zeros.
std::vector<float> expand_group_scales(const float *scales, int64_t n, int64_t k, int64_t group) {
  const int64_t kb = k / 32, ng = k / group, gb = group / 32;
  std::vector<float> blk((size_t)n * kb, 0.f);
  if (scales)
    for (int64_t r = 0; r < n; ++r)
      for (int64_t b = 0; b < kb; ++b) blk[r * kb + b] = scales[r * ng + b / gb];
  return blk;
}
}  // namespace

extern "C" int rk_pack_i8(const float *w, int64_t n, int64_t k, int64_t group, rk_weight_id *id) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_pack_i8"));
  RK_TRY(check_i8_shape(n, k, group, "rk_pack_i8"));
  CallScope cs(g_eng->stream);
  // Quantize on the device with the activation quantizer (same formula as
  // quantize_i8_weight, ext.rs:1001-1012), then keep codes and scales.
  void *x32, *q, *s;
  const int64_t ng = k / group;
  RK_TRY(scratch(cs, "pack_f32", (size_t)n * k * 4, &x32));
  RK_TRY(scratch(cs, "pack_q", (size_t)n * k, &q));
  RK_TRY(scratch(cs, "pack_s", (size_t)n * ng * 4, &s));
  HIP_TRY(hipMemcpyAsync(x32, w, (size_t)n * k * 4, hipMemcpyHostToDevice, g_eng->stream),
          "rk_pack_i8");
  HIP_TRY(rk_launch_quantize_rows((const float *)x32, n, k, group, (int8_t *)q, (float *)s,
                                  g_eng->stream),
          "rk_pack_i8");
  std::vector<int8_t> codes((size_t)n * k);
  std::vector<float> scales((size_t)n * ng);
  HIP_TRY(hipMemcpyAsync(codes.data(), q, codes.size(), hipMemcpyDeviceToHost, g_eng->stream),
          "rk_pack_i8");
  HIP_TRY(hipMemcpyAsync(scales.data(), s, scales.size() * 4, hipMemcpyDeviceToHost,
                         g_eng->stream),
          "rk_pack_i8");
  HIP_TRY(hipStreamSynchronize(g_eng->stream), "rk_pack_i8");
  return pack_i8_host(codes.data(), expand_group_scales(scales.data(), n, k, group), n, k, group,
                      id, "rk_pack_i8");
}

extern "C" int rk_pack_i8_codes(const int8_t *codes, const float *scales, int64_t n, int64_t k,
                                int64_t group, rk_weight_id *id) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_pack_i8_codes"));
  RK_TRY(check_i8_shape(n, k, group, "rk_pack_i8_codes"));
  return pack_i8_host(codes, expand_group_scales(scales, n, k, group), n, k, group, id,
                      "rk_pack_i8_codes");
}

extern "C" int rk_rewrite_i8(rk_weight_id id, const int8_t *codes, const float *scales) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_rewrite_i8"));
  Weight *w = find(id);
  if (!w || w->kind != RK_WEIGHT_I8)
    return fail(RK_E_SHAPE, "rk_rewrite_i8", "id is not a resident int8 weight");
  HIP_TRY(hipStreamSynchronize(g_eng->stream), "rk_rewrite_i8");
  HIP_TRY(hipMemcpy(w->codes, codes, (size_t)w->n * w->k, hipMemcpyHostToDevice), "rk_rewrite_i8");
  // Null scales: the codes alone (I8Context::rewrite_weight_gw, int8.rs:482-526).
  if (!scales) return RK_OK;
  std::vector<float> blk = expand_group_scales(scales, w->n, w->k, w->group);
  const int64_t kb = w->k / 32;
  std::vector<float> pad((size_t)w->n * w->ws_stride, 0.f);
  for (int64_t r = 0; r < w->n; ++r)
    std::memcpy(&pad[(size_t)r * w->ws_stride], &blk[(size_t)r * kb], sizeof(float) * kb);
  HIP_TRY(hipMemcpy(w->scales, pad.data(), pad.size() * 4, hipMemcpyHostToDevice), "rk_rewrite_i8");
  return RK_OK;
}

namespace {
// Resident Q8_0 weight of `rows` rows from GGUF blocks that are uploaded once and
// split into codes and f32 scales on the device. Each (blocks, grp_off) source
// lands at rows (r/16)·grp_stride + grp_off + r%16; other rows stay zero.
int pack_q8_0_blocks(CallScope &cs, const uint8_t *const *srcs, const int *grp_offs, int nsrc,
                     int64_t n, int64_t k, int64_t rows, int grp_stride, Weight &wt,
                     const char *op) {
  wt.kind = RK_WEIGHT_I8;
  wt.ws_f16 = true;  // GGUF Q8_0: fp16 d per block
  wt.n = rows;
  wt.k = k;
  wt.group = 32;
  wt.ws_stride = ws_stride_for(k);
  const size_t blk_bytes = (size_t)n * (k / 32) * 34;
  void *dblk;
  RK_TRY(scratch(cs, "pack_blk", blk_bytes, &dblk));
  HIP_TRY(hipMalloc(&wt.codes, (size_t)rows * k), op);
  HIP_TRY(hipMalloc((void **)&wt.scales, (size_t)rows * wt.ws_stride * 4), op);
  HIP_TRY(hipMemsetAsync(wt.codes, 0, (size_t)rows * k, cs.st), op);
  HIP_TRY(hipMemsetAsync(wt.scales, 0, (size_t)rows * wt.ws_stride * 4, cs.st), op);
  for (int i = 0; i < nsrc; ++i) {
    HIP_TRY(hipMemcpyAsync(dblk, srcs[i], blk_bytes, hipMemcpyHostToDevice, cs.st), op);
    HIP_TRY(rk_launch_q8_0_unpack(dblk, n, k, grp_stride, grp_offs[i], (int8_t *)wt.codes, wt.scales,
                                  wt.ws_stride, false, cs.st),
            op);
  }
  HIP_TRY(hipStreamSynchronize(cs.st), op);
  wt.bytes = (size_t)rows * k + (size_t)rows * wt.ws_stride * 4;
  return RK_OK;
}
}  // namespace

extern "C" int rk_pack_q8_0(const uint8_t *blocks, int64_t n, int64_t k, rk_weight_id *id) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_pack_q8_0"));
  RK_TRY(check_i8_shape(n, k, 32, "rk_pack_q8_0"));
  CallScope cs(g_eng->stream);
  Weight wt;
  PackGuard guard(wt);
  const int off = 0;
  RK_TRY(pack_q8_0_blocks(cs, &blocks, &off, 1, n, k, n, 16, wt, "rk_pack_q8_0"));
  *id = guard.register_weight();
  return RK_OK;
}

extern "C" int rk_pack_q8_0_f32(const float *w, int64_t n, int64_t k, rk_weight_id *id) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_pack_q8_0_f32"));
  RK_TRY(check_i8_shape(n, k, 32, "rk_pack_q8_0_f32"));
  CallScope cs(g_eng->stream);
  Weight wt;
  PackGuard guard(wt);
  wt.kind = RK_WEIGHT_I8;
  wt.ws_f16 = true;  // GGUF Q8_0: fp16 d per block
  wt.n = n;
  wt.k = k;
  wt.group = 32;
  wt.ws_stride = ws_stride_for(k);
  void *x32;
  RK_TRY(scratch(cs, "pack_f32", (size_t)n * k * 4, &x32));
  HIP_TRY(hipMalloc(&wt.codes, (size_t)n * k), "rk_pack_q8_0_f32");
  HIP_TRY(hipMalloc((void **)&wt.scales, (size_t)n * wt.ws_stride * 4), "rk_pack_q8_0_f32");
  HIP_TRY(hipMemsetAsync(wt.scales, 0, (size_t)n * wt.ws_stride * 4, g_eng->stream), "rk_pack_q8_0_f32");
  HIP_TRY(hipMemcpyAsync(x32, w, (size_t)n * k * 4, hipMemcpyHostToDevice, g_eng->stream),
          "rk_pack_q8_0_f32");
  HIP_TRY(rk_launch_q8_0_quantize((const float *)x32, n, k, 16, 0, (int8_t *)wt.codes, wt.scales,
                                  wt.ws_stride, false, g_eng->stream),
          "rk_pack_q8_0_f32");
  HIP_TRY(hipStreamSynchronize(g_eng->stream), "rk_pack_q8_0_f32");
  wt.bytes = (size_t)n * k + (size_t)n * wt.ws_stride * 4;
  *id = guard.register_weight();
  return RK_OK;
}

// Gate and up Q8_0 weights of one gated MLP as one resident weight whose rows
// alternate 16 gate rows and the same 16 up rows (32·ceil(n/16) rows, padding
// rows zero), the layout rk_matmul_w8a8_glu_dev pairs in its epilogue.
namespace {
int64_t glu_rows(int64_t n) { return 32 * ((n + 15) / 16); }
int64_t glu_row(int64_t r, int part) { return (r / 16) * 32 + 16 * part + r % 16; }
}  // namespace

extern "C" int rk_pack_q8_0_glu(const uint8_t *gate_blocks, const uint8_t *up_blocks, int64_t n,
                                int64_t k, rk_weight_id *id) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_pack_q8_0_glu"));
  RK_TRY(check_i8_shape(n, k, 32, "rk_pack_q8_0_glu"));
  CallScope cs(g_eng->stream);
  Weight wt;
  PackGuard guard(wt);
  const uint8_t *srcs[2] = {gate_blocks, up_blocks};
  const int offs[2] = {0, 16};  // gate rows at 32t + j, up rows at 32t + 16 + j
  RK_TRY(pack_q8_0_blocks(cs, srcs, offs, 2, n, k, glu_rows(n), 32, wt, "rk_pack_q8_0_glu"));
  wt.glu_n = n;
  *id = guard.register_weight();
  return RK_OK;
}

extern "C" int rk_pack_q8_0_glu_f32(const float *gate, const float *up, int64_t n, int64_t k,
                                    rk_weight_id *id) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_pack_q8_0_glu_f32"));
  RK_TRY(check_i8_shape(n, k, 32, "rk_pack_q8_0_glu_f32"));
  CallScope cs(g_eng->stream);
  const int64_t rows = glu_rows(n);
  Weight wt;
  PackGuard guard(wt);
  wt.kind = RK_WEIGHT_I8;
  wt.ws_f16 = true;  // GGUF Q8_0: fp16 d per block
  wt.n = rows;
  wt.k = k;
  wt.group = 32;
  wt.glu_n = n;
  wt.ws_stride = ws_stride_for(k);
  void *x32;
  RK_TRY(scratch(cs, "pack_f32", (size_t)n * k * 4, &x32));
  HIP_TRY(hipMalloc(&wt.codes, (size_t)rows * k), "rk_pack_q8_0_glu_f32");
  HIP_TRY(hipMalloc((void **)&wt.scales, (size_t)rows * wt.ws_stride * 4), "rk_pack_q8_0_glu_f32");
  HIP_TRY(hipMemsetAsync(wt.codes, 0, (size_t)rows * k, g_eng->stream), "rk_pack_q8_0_glu_f32");
  HIP_TRY(hipMemsetAsync(wt.scales, 0, (size_t)rows * wt.ws_stride * 4, g_eng->stream),
          "rk_pack_q8_0_glu_f32");
  for (int part = 0; part < 2; ++part) {
    HIP_TRY(hipMemcpyAsync(x32, part ? up : gate, (size_t)n * k * 4, hipMemcpyHostToDevice,
                           g_eng->stream),
            "rk_pack_q8_0_glu_f32");
    // rows land at (r/16)·32 + 16·part + r%16
    HIP_TRY(rk_launch_q8_0_quantize((const float *)x32, n, k, 32, 16 * part, (int8_t *)wt.codes,
                                    wt.scales, wt.ws_stride, false, g_eng->stream),
            "rk_pack_q8_0_glu_f32");
  }
  HIP_TRY(hipStreamSynchronize(g_eng->stream), "rk_pack_q8_0_glu_f32");
  wt.bytes = (size_t)rows * k + (size_t)rows * wt.ws_stride * 4;
  *id = guard.register_weight();
  return RK_OK;
}

// fp16 gate|up weight for rk_matmul_f16_glu_dev: rows interleaved per 16 as
// rk_pack_q8_0_glu lays them out, padding rows zero.
extern "C" int rk_pack_f16_glu(const float *gate, const float *up, int64_t n, int64_t k,
                               rk_weight_id *id) {
  std::lock_guard<std::mutex> lk(g_mu);
  const char *op = "rk_pack_f16_glu";
  RK_TRY(ensure(op));
  RK_TRY(check_f16_shape(n, k, op));
  if (!gate || !up) return fail(RK_E_SHAPE, op, "null weight");
  CallScope cs(g_eng->stream);
  const int64_t rows = glu_rows(n);
  Weight w;
  PackGuard guard(w);
  w.kind = RK_WEIGHT_F16;
  w.n = rows;
  w.k = k;
  w.glu_n = n;
  w.bytes = (size_t)rows * k * 2;
  void *x32;
  RK_TRY(scratch(cs, "pack_f32", (size_t)n * k * 4, &x32));
  HIP_TRY(hipMalloc(&w.codes, w.bytes), op);
  HIP_TRY(hipMemsetAsync(w.codes, 0, w.bytes, cs.st), op);
  for (int part = 0; part < 2; ++part) {
    HIP_TRY(hipMemcpyAsync(x32, part ? up : gate, (size_t)n * k * 4, hipMemcpyHostToDevice, cs.st), op);
    HIP_TRY(rk_launch_f32_to_f16_rows((const float *)x32, n, k, 32, 16 * part, w.codes, cs.st), op);
  }
  HIP_TRY(hipStreamSynchronize(cs.st), op);
  *id = guard.register_weight();
  return RK_OK;
}

extern "C" int rk_pack_qat(const int8_t *codes, const float *w_scale, int64_t n, int64_t k,
                           float in_scale, float out_scale, rk_weight_id *id) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_pack_qat"));
  if (n <= 0 || k <= 0 || k % 32 != 0)
    return fail(RK_E_SHAPE, "rk_pack_qat", "the int8 path needs K % 32 == 0");
  if (!(in_scale >= 0.f)) return fail(RK_E_SHAPE, "rk_pack_qat", "input scale must not be negative");
  Weight w;
  PackGuard guard(w);
  w.kind = RK_WEIGHT_QAT;
  w.n = n;
  w.k = k;
  w.group = k;
  w.in_scale = in_scale;
  w.out_scale = out_scale;
  HIP_TRY(hipMalloc(&w.codes, (size_t)n * k), "rk_pack_qat");
  HIP_TRY(hipMemcpy(w.codes, codes, (size_t)n * k, hipMemcpyHostToDevice), "rk_pack_qat");
  HIP_TRY(hipMalloc((void **)&w.scales, (size_t)n * 4), "rk_pack_qat");
  HIP_TRY(hipMemcpy(w.scales, w_scale, (size_t)n * 4, hipMemcpyHostToDevice), "rk_pack_qat");
  w.bytes = (size_t)n * k + (size_t)n * 4;
  *id = guard.register_weight();
  return RK_OK;
}

extern "C" int rk_weight_info(rk_weight_id id, int *kind, int64_t *n, int64_t *k,
                              int64_t *group) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_weight_info"));
  Weight *w = find(id);
  if (!w) return fail(RK_E_SHAPE, "rk_weight_info", "weight id is not packed");
  *kind = w->moe ? 0 : w->kind;
  *n = w->n;
  *k = w->k;
  *group = w->group;
  return RK_OK;
}

// =========================================================================
// Matmul
// =========================================================================
namespace {
int launch_i8(const Weight &w, const int8_t *a, const float *as, int as_stride, int a_gb,
              int mode, bool out_f16, int64_t m, void *c, hipStream_t st, const char *op) {
  I8GemmArgs g;
  g.A = a;
  g.AS = as;
  g.as_stride = as_stride;
  g.a_gb = a_gb;
  g.W = (const int8_t *)w.codes;
  g.WS = w.scales;
  g.ws_stride = w.ws_stride;
  g.ws_f16 = w.ws_f16;
  g.gb = (int)(w.group / 32);
  g.C = c;
  g.M = (int)m;
  g.N = (int)w.n;
  g.K = (int)w.k;
  g.mode = mode;
  g.out_f16 = out_f16;
  g.num_cus = g_eng->num_cus;
  HIP_TRY(rk_launch_gemm_i8(g, st), op);
  return RK_OK;
}

// One fp16 GEMM launch (glu: the gate|up epilogue form) with its split-K
// workspace from the call's scratch: partial tiles, and arrival counters
// zeroed when first allocated (every launch leaves them at zero).
int gemm_f16_run(CallScope &cs, const void *a, const void *b, void *c, int64_t m, int64_t n, int64_t k,
                 const char *op, int glu = 0, int64_t n_out = 0, bool out_f16 = true) {
  const F16Plan p = rk_gemm_f16_plan((int)m, (int)n, (int)k, g_eng->num_cus, glu != 0);
  float *part = nullptr;
  unsigned *cnt = nullptr;
  if (p.ksplit > 1) {
    bool fresh = false;
    const size_t cnt_bytes = std::max<size_t>((size_t)p.n_cnt * 4, 256);
    RK_TRY(scratch(cs, "f16_part", (size_t)p.part_floats * 4, (void **)&part));
    RK_TRY(scratch(cs, "f16_cnt", cnt_bytes, (void **)&cnt, &fresh));
    if (fresh) HIP_TRY(hipMemsetAsync(cnt, 0, cnt_bytes, cs.st), op);
  }
  if (glu)
    HIP_TRY(rk_launch_gemm_f16_glu(p, a, b, c, (int)m, (int)n, (int)k, (int)n_out, glu, out_f16, part, cnt, cs.st),
            op);
  else
    HIP_TRY(rk_launch_gemm_f16(p, a, b, c, (int)m, (int)n, (int)k, part, cnt, cs.st), op);
  return RK_OK;
}

int check_m(int64_t m, int64_t k, const Weight *w, const char *op) {
  if (!w) return fail(RK_E_SHAPE, op, "weight id is not packed");
  if (m < 0) return fail(RK_E_SHAPE, op, "M must not be negative");
  if (m > INT32_MAX) return fail(RK_E_SHAPE, op, "M too large");
  if (k != w->k)
    return fail(RK_E_SHAPE, op, "activation K " + std::to_string(k) + " != weight K " +
                                    std::to_string(w->k));
  return RK_OK;
}
}  // namespace

extern "C" int rk_matmul(rk_weight_id id, const float *x, int64_t m, int64_t k, float *y) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_matmul"));
  Weight *w = find(id);
  RK_TRY(check_m(m, k, w, "rk_matmul"));
  if (w->moe) return fail(RK_E_UNSUPPORTED, "rk_matmul", "an expert stack is not a matmul weight");
  if (w->glu_n > 0)
    return fail(RK_E_UNSUPPORTED, "rk_matmul", "gate|up weight: use rk_matmul_w8a8_glu_dev");
  if (m == 0) return RK_OK;  // an empty batch: nothing to compute (the reference returns [.., 0, N])
  hipStream_t st = g_eng->stream;
  CallScope cs(st);
  const int64_t n = w->n;
  float *x32, *y32;
  RK_TRY(scratch(cs, "mm_x32", (size_t)m * k * 4, (void **)&x32));
  RK_TRY(scratch(cs, "mm_y32", (size_t)m * n * 4, (void **)&y32));
  // Row chunks of x go up, are converted or quantized and multiplied, and
  // their rows of y come down while the next chunk is in flight.
  std::function<int(int64_t, int64_t)> compute;
  if (w->kind == RK_WEIGHT_F16) {
    uint16_t *a16, *c16;
    RK_TRY(scratch(cs, "mm_a16", (size_t)m * k * 2, (void **)&a16));
    RK_TRY(scratch(cs, "mm_c16", (size_t)m * n * 2, (void **)&c16));
    compute = [=, &cs](int64_t r0, int64_t r1) {
      const int64_t rows = r1 - r0;
      HIP_TRY(rk_launch_f32_to_f16(x32 + r0 * k, a16 + r0 * k, rows * k, st), "rk_matmul");
      RK_TRY(gemm_f16_run(cs, a16 + r0 * k, w->codes, c16 + r0 * n, rows, n, k, "rk_matmul_fp16"));
      HIP_TRY(rk_launch_f16_to_f32(c16 + r0 * n, y32 + r0 * n, rows * n, st), "rk_matmul");
      return RK_OK;
    };
  } else if (w->kind == RK_WEIGHT_I8) {
    int8_t *q;
    float *s;
    const int64_t ng = k / w->group;
    RK_TRY(scratch(cs, "mm_q", (size_t)m * k, (void **)&q));
    RK_TRY(scratch(cs, "mm_s", (size_t)m * ng * 4, (void **)&s));
    compute = [=](int64_t r0, int64_t r1) {
      HIP_TRY(rk_launch_quantize_rows(x32 + r0 * k, r1 - r0, k, w->group, q + r0 * k, s + r0 * ng, st),
              "rk_matmul");
      return launch_i8(*w, q + r0 * k, s + r0 * ng, (int)ng, (int)(w->group / 32), I8_PER_GROUP, false,
                       r1 - r0, y32 + r0 * n, st, "rk_matmul_int8_gw");
    };
  } else {  // QAT
    int8_t *q;
    float *rs;
    int32_t *acc;
    RK_TRY(scratch(cs, "mm_q", (size_t)m * k, (void **)&q));
    RK_TRY(scratch(cs, "mm_rs", (size_t)m * 4, (void **)&rs));
    RK_TRY(scratch(cs, "mm_acc", (size_t)m * n * 4, (void **)&acc));
    compute = [=](int64_t r0, int64_t r1) {
      const int64_t rows = r1 - r0;
      HIP_TRY(rk_launch_quantize_static(x32 + r0 * k, rows, k, w->in_scale, q + r0 * k, rs + r0, st),
              "rk_matmul");
      RK_TRY(launch_i8(*w, q + r0 * k, nullptr, 0, 1, I8_RAW, false, rows, acc + r0 * n, st,
                       "rk_matmul_int8_qat"));
      HIP_TRY(rk_launch_qat_epilogue(acc + r0 * n, rs + r0, w->scales, rows, n, w->out_scale,
                                     y32 + r0 * n, st),
              "rk_matmul");
      return RK_OK;
    };
  }
  RK_TRY(staged(cs, {{x, nullptr, x32, (size_t)k * 4, 0}}, {{nullptr, y, y32, (size_t)n * 4, 0}}, m,
                stage_chunk_rows(m, (size_t)k * 4, (size_t)n * 4), compute, "rk_matmul"));
  g_eng->calls++;
  return RK_OK;
}

// RocketCtx::matmul_prepacked (crates/burn-rocket/src/lib.rs:244-254) on host
// fp16 buffers.
extern "C" int rk_matmul_f16(rk_weight_id id, const uint16_t *a, int64_t m, int64_t k, uint16_t *c) {
  std::lock_guard<std::mutex> lk(g_mu);
  const char *op = "rk_matmul_f16";
  RK_TRY(ensure(op));
  Weight *w = find(id);
  RK_TRY(check_m(m, k, w, op));
  if (w->kind != RK_WEIGHT_F16 || w->moe || w->glu_n > 0)
    return fail(RK_E_UNSUPPORTED, op, "weight is not a plain fp16 weight");
  if (m == 0) return RK_OK;  // an empty batch: nothing to compute (the reference returns [.., 0, N])
  if (!a || !c) return fail(RK_E_SHAPE, op, "null buffer");
  hipStream_t st = g_eng->stream;
  CallScope cs(st);
  const int64_t n = w->n;
  uint16_t *a16, *c16;
  RK_TRY(scratch(cs, "mm_a16", (size_t)m * k * 2, (void **)&a16));
  RK_TRY(scratch(cs, "mm_c16", (size_t)m * n * 2, (void **)&c16));
  auto compute = [&](int64_t r0, int64_t r1) {
    RK_TRY(gemm_f16_run(cs, a16 + r0 * k, w->codes, c16 + r0 * n, r1 - r0, n, k, "rocket_matmul_fp16"));
    return RK_OK;
  };
  RK_TRY(staged(cs, {{a, nullptr, a16, (size_t)k * 2, 0}}, {{nullptr, c, c16, (size_t)n * 2, 0}}, m,
                stage_chunk_rows(m, (size_t)k * 2, (size_t)n * 2), compute, op));
  g_eng->calls++;
  return RK_OK;
}

// I8Context::matmul_gw (crates/rocket-npu/src/matmul/int8.rs:644-676) on host
// buffers, as Clef's gw_matmul calls it (src/clef/engine_npu.rs:75-110).
extern "C" int rk_matmul_i8_gw(rk_weight_id id, const int8_t *a, const float *a_scale,
                               const float *b_scale, int64_t m, int64_t k, float *cf) {
  std::lock_guard<std::mutex> lk(g_mu);
  const char *op = "rk_matmul_i8_gw";
  RK_TRY(ensure(op));
  Weight *w = find(id);
  RK_TRY(check_m(m, k, w, op));
  if (w->kind != RK_WEIGHT_I8 || w->moe || w->glu_n > 0)
    return fail(RK_E_UNSUPPORTED, op, "weight is not a group-wise int8 weight");
  if (m == 0) return RK_OK;  // an empty batch: nothing to compute (the reference returns [.., 0, N])
  if (!a || !a_scale || !cf) return fail(RK_E_SHAPE, op, "null buffer");
  hipStream_t st = g_eng->stream;
  CallScope cs(st);
  const int64_t n = w->n, ng = k / w->group;
  int8_t *q;
  float *s, *y32, *ws = w->scales;
  RK_TRY(scratch(cs, "mm_q", (size_t)m * k, (void **)&q));
  RK_TRY(scratch(cs, "mm_s", (size_t)m * ng * 4, (void **)&s));
  RK_TRY(scratch(cs, "mm_y32", (size_t)m * n * 4, (void **)&y32));
  // This call's weight scales [N, K/group], widened to the resident layout
  // (one f32 per 32-value block, rows padded to ws_stride) and uploaded with
  // the first chunk.
  std::vector<float> wpad;
  if (b_scale) {
    RK_TRY(scratch(cs, "mm_ws", (size_t)n * w->ws_stride * 4, (void **)&ws));
    const std::vector<float> blk = expand_group_scales(b_scale, n, k, w->group);
    const int64_t kb = k / 32;
    wpad.assign((size_t)n * w->ws_stride, 0.f);
    for (int64_t r = 0; r < n; ++r)
      std::memcpy(&wpad[(size_t)r * w->ws_stride], &blk[(size_t)r * kb], sizeof(float) * kb);
  }
  Weight wv = *w;
  wv.scales = ws;
  // The fold is the reference's (a_s·w_s)·P per group (int8.rs:663-667) for
  // any scale values (no fp16-scale fold order).
  wv.ws_f16 = false;
  std::vector<rkstage::Xfer> ins = {{a, nullptr, q, (size_t)k, 0}, {a_scale, nullptr, s, (size_t)ng * 4, 0}};
  if (b_scale) ins.push_back({wpad.data(), nullptr, ws, 0, wpad.size() * 4});
  auto compute = [&](int64_t r0, int64_t r1) {
    return launch_i8(wv, q + r0 * k, s + r0 * ng, (int)ng, (int)(w->group / 32), I8_PER_GROUP, false,
                     r1 - r0, y32 + r0 * n, st, "rk_matmul_int8_gw");
  };
  RK_TRY(staged(cs, ins, {{nullptr, cf, y32, (size_t)n * 4, 0}}, m,
                stage_chunk_rows(m, (size_t)k, (size_t)n * 4), compute, op));
  g_eng->calls++;
  return RK_OK;
}

// I8Context::matmul (int8.rs:606-640): raw int32 on host buffers.
extern "C" int rk_matmul_i8(rk_weight_id id, const int8_t *a, int64_t m, int64_t k, int32_t *c) {
  std::lock_guard<std::mutex> lk(g_mu);
  const char *op = "rk_matmul_i8";
  RK_TRY(ensure(op));
  Weight *w = find(id);
  RK_TRY(check_m(m, k, w, op));
  if ((w->kind != RK_WEIGHT_I8 && w->kind != RK_WEIGHT_QAT) || w->moe || w->glu_n > 0)
    return fail(RK_E_UNSUPPORTED, op, "weight is not int8");
  if (m == 0) return RK_OK;  // an empty batch: nothing to compute (the reference returns [.., 0, N])
  if (!a || !c) return fail(RK_E_SHAPE, op, "null buffer");
  hipStream_t st = g_eng->stream;
  CallScope cs(st);
  const int64_t n = w->n;
  int8_t *q;
  int32_t *acc;
  RK_TRY(scratch(cs, "mm_q", (size_t)m * k, (void **)&q));
  RK_TRY(scratch(cs, "mm_acc", (size_t)m * n * 4, (void **)&acc));
  auto compute = [&](int64_t r0, int64_t r1) {
    return launch_i8(*w, q + r0 * k, nullptr, 0, 1, I8_RAW, false, r1 - r0, acc + r0 * n, st, op);
  };
  RK_TRY(staged(cs, {{a, nullptr, q, (size_t)k, 0}}, {{nullptr, c, acc, (size_t)n * 4, 0}}, m,
                stage_chunk_rows(m, (size_t)k, (size_t)n * 4), compute, op));
  g_eng->calls++;
  return RK_OK;
}

extern "C" int rk_matmul_f16_dev(rk_weight_id id, const void *a, int64_t m, int64_t k, void *c,
                                 rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_matmul_f16_dev"));
  Weight *w = find(id);
  RK_TRY(check_m(m, k, w, "rk_matmul_f16_dev"));
  if (w->kind != RK_WEIGHT_F16 || w->moe)
    return fail(RK_E_UNSUPPORTED, "rk_matmul_f16_dev", "weight is not fp16");
  if (w->glu_n > 0)
    return fail(RK_E_UNSUPPORTED, "rk_matmul_f16_dev", "gate|up weight: use rk_matmul_f16_glu_dev");
  if (m == 0) return RK_OK;  // an empty batch: nothing to compute (the reference returns [.., 0, N])
  CallScope cs(pick(stream));
  RK_TRY(gemm_f16_run(cs, a, w->codes, c, m, w->n, k, "rk_matmul_f16_dev"));
  g_eng->calls++;
  return RK_OK;
}

extern "C" int rk_matmul_f16_glu_dev(rk_weight_id id, const void *a, int64_t m, int64_t k, int glu,
                                     void *out, int out_f16, rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  const char *op = "rk_matmul_f16_glu_dev";
  RK_TRY(ensure(op));
  Weight *w = find(id);
  RK_TRY(check_m(m, k, w, op));
  if (w->kind != RK_WEIGHT_F16 || w->moe || w->glu_n <= 0)
    return fail(RK_E_UNSUPPORTED, op, "weight was not packed by rk_pack_f16_glu");
  if (glu != RK_GLU_SILU && glu != RK_GLU_GELU) return fail(RK_E_SHAPE, op, "unknown glu kind");
  if (m == 0) return RK_OK;  // an empty batch: nothing to compute (the reference returns [.., 0, N])
  CallScope cs(pick(stream));
  RK_TRY(gemm_f16_run(cs, a, w->codes, out, m, w->n, k, op, glu, w->glu_n, out_f16 != 0));
  g_eng->calls++;
  return RK_OK;
}

extern "C" int rk_quantize_rows_dev(const float *x, int64_t m, int64_t k, int64_t group, int8_t *q,
                                    float *scale, rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_quantize_rows_dev"));
  if (m < 0 || k <= 0 || group <= 0 || k % group != 0)
    return fail(RK_E_SHAPE, "rk_quantize_rows_dev", "group must divide K");
  if (k / group > 1024) return fail(RK_E_SHAPE, "rk_quantize_rows_dev", "more than 1024 groups per row");
  if (m == 0) return RK_OK;
  HIP_TRY(rk_launch_quantize_rows(x, m, k, group, q, scale, pick(stream)), "rk_quantize_rows_dev");
  return RK_OK;
}

namespace {
int w8a8_dev(rk_weight_id id, const int8_t *a, const float *a_scale, int64_t a_group, int64_t m,
             int64_t k, void *c, bool out_f16, rk_stream stream, const char *op) {
  RK_TRY(ensure(op));
  Weight *w = find(id);
  RK_TRY(check_m(m, k, w, op));
  if (w->kind != RK_WEIGHT_I8 || w->moe) return fail(RK_E_UNSUPPORTED, op, "weight is not group-wise int8");
  if (w->glu_n > 0) return fail(RK_E_UNSUPPORTED, op, "gate|up weight: use rk_matmul_w8a8_glu_dev");
  int mode;
  if (a_group == k)
    mode = I8_PER_TOKEN;
  else if (a_group == w->group)
    mode = I8_PER_GROUP;
  else
    return fail(RK_E_SHAPE, op, "activation group must be K (per token) or the weight group");
  if (m == 0) return RK_OK;  // an empty batch: nothing to compute (the reference returns [.., 0, N])
  RK_TRY(launch_i8(*w, a, a_scale, (int)(k / a_group), (int)(a_group / 32), mode, out_f16, m, c,
                   pick(stream), op));
  g_eng->calls++;
  return RK_OK;
}
}  // namespace

extern "C" int rk_matmul_w8a8_glu_dev(rk_weight_id id, const int8_t *a, const float *a_scale,
                                      int64_t m, int64_t k, int glu, void *out, int out_f16,
                                      rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  const char *op = "rk_matmul_w8a8_glu_dev";
  RK_TRY(ensure(op));
  Weight *w = find(id);
  RK_TRY(check_m(m, k, w, op));
  if (w->glu_n <= 0) return fail(RK_E_UNSUPPORTED, op, "weight was not packed by rk_pack_q8_0_glu");
  if (glu != RK_GLU_SILU && glu != RK_GLU_GELU) return fail(RK_E_SHAPE, op, "unknown glu kind");
  if (m == 0) return RK_OK;  // an empty batch: nothing to compute (the reference returns [.., 0, N])
  I8GemmArgs g;
  g.A = a;
  g.AS = a_scale;
  g.as_stride = 1;
  g.a_gb = (int)(k / 32);
  g.W = (const int8_t *)w->codes;
  g.WS = w->scales;
  g.ws_stride = w->ws_stride;
  g.gb = 1;
  g.C = out;
  g.M = (int)m;
  g.N = (int)w->n;
  g.K = (int)w->k;
  g.mode = I8_PER_TOKEN;
  g.out_f16 = out_f16 != 0;
  g.num_cus = g_eng->num_cus;
  g.glu = glu;
  g.n_out = (int)w->glu_n;
  HIP_TRY(rk_launch_gemm_i8(g, pick(stream)), op);
  g_eng->calls++;
  return RK_OK;
}

extern "C" int rk_matmul_w8a8_dev(rk_weight_id id, const int8_t *a, const float *a_scale,
                                  int64_t a_group, int64_t m, int64_t k, float *c,
                                  rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  return w8a8_dev(id, a, a_scale, a_group, m, k, c, false, stream, "rk_matmul_w8a8_dev");
}

extern "C" int rk_matmul_w8a8_f16out_dev(rk_weight_id id, const int8_t *a, const float *a_scale,
                                         int64_t a_group, int64_t m, int64_t k, void *c,
                                         rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  return w8a8_dev(id, a, a_scale, a_group, m, k, c, true, stream, "rk_matmul_w8a8_f16out_dev");
}

extern "C" int rk_matmul_i8_raw_dev(rk_weight_id id, const int8_t *a, int64_t m, int64_t k,
                                    int32_t *c, rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_matmul_i8_raw_dev"));
  Weight *w = find(id);
  RK_TRY(check_m(m, k, w, "rk_matmul_i8_raw_dev"));
  if ((w->kind != RK_WEIGHT_I8 && w->kind != RK_WEIGHT_QAT) || w->moe)
    return fail(RK_E_UNSUPPORTED, "rk_matmul_i8_raw_dev", "weight is not int8");
  if (m == 0) return RK_OK;  // an empty batch: nothing to compute (the reference returns [.., 0, N])
  RK_TRY(launch_i8(*w, a, nullptr, 0, 1, I8_RAW, false, m, c, pick(stream), "rk_matmul_i8_raw_dev"));
  g_eng->calls++;
  return RK_OK;
}

extern "C" int rk_matmul_i8_partials_dev(rk_weight_id id, const int8_t *a, int64_t m, int64_t k,
                                         int32_t *p, rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_matmul_i8_partials_dev"));
  Weight *w = find(id);
  RK_TRY(check_m(m, k, w, "rk_matmul_i8_partials_dev"));
  if ((w->kind != RK_WEIGHT_I8 && w->kind != RK_WEIGHT_QAT) || w->moe)
    return fail(RK_E_UNSUPPORTED, "rk_matmul_i8_partials_dev", "weight is not int8");
  if (m == 0) return RK_OK;  // an empty batch: nothing to compute (the reference returns [.., 0, N])
  RK_TRY(launch_i8(*w, a, nullptr, 0, 1, I8_PARTIALS, false, m, p, pick(stream),
                   "rk_matmul_i8_partials_dev"));
  g_eng->calls++;
  return RK_OK;
}

// =========================================================================
// Attention
// =========================================================================
hipError_t rk_launch_v_transpose_strided(const void *v, int64_t tok_stride, int64_t head_stride,
                                         int64_t d_stride, int n_kv, int n_kv_pad,
                                         int n_kv_heads, int head_dim, int dv_pad, void *vt,
                                         hipStream_t st);
namespace {
// padded: also head dims 160, 192 and 224, which attn_dev_impl runs zero-padded.
int attn_check(int64_t n_q, int64_t n_kv, int n_head, int n_kv_heads, int head_dim, int *mode,
               int64_t window, const char *op, bool padded = false) {
  if (n_q <= 0 || n_kv <= 0) return fail(RK_E_SHAPE, op, "empty query or key axis");
  if (n_q > INT32_MAX || n_kv > INT32_MAX) return fail(RK_E_SHAPE, op, "sequence too long");
  if (n_head <= 0 || n_kv_heads <= 0 || n_head % n_kv_heads != 0)
    return fail(RK_E_SHAPE, op, "n_head must be a positive multiple of n_kv_heads");
  if (n_head / n_kv_heads > 128) return fail(RK_E_SHAPE, op, "GQA group above 128");
  switch (head_dim) {
    case 32: case 48: case 64: case 72: case 80: case 96: case 112: case 128: case 256: break;
    case 160: case 192: case 224:
      if (padded) break;
      [[fallthrough]];
    default:
      return fail(RK_E_UNSUPPORTED, op, "head_dim " + std::to_string(head_dim) +
                                            " (supported: 32, 48, 64, 72, 80, 96, 112, 128, 256)");
  }
  if (*mode < RK_MASK_NONE || *mode > RK_MASK_CAUSAL_WINDOW)
    return fail(RK_E_SHAPE, op, "unknown mask mode");
  // window < 0 disables the window (ext.rs:99-126).
  if (*mode == RK_MASK_WINDOW && window < 0) *mode = RK_MASK_NONE;
  if (*mode == RK_MASK_CAUSAL_WINDOW && window < 0) *mode = RK_MASK_CAUSAL;
  return RK_OK;
}

// cs: the call's scope, which provides the key-split workspace; null (the
// no-allocation entry) launches without a key split.
int attn_run(const void *q, const void *k, const void *vt, void *out, int64_t n_q, int64_t n_kv,
             int64_t n_kv_pad, int n_head, int n_kv_heads, int head_dim, float scale, float softcap,
             int mode, int64_t window, int64_t q0, int64_t k0, bool head_major, hipStream_t st,
             const char *op, CallScope *cs, int64_t q_ts = 0, int64_t k_ts = 0, int64_t o_ts = 0) {
  // K and Vᵀ of one kv head are addressed with 32-bit byte offsets.
  const int64_t k_tok = head_major ? head_dim : (k_ts ? k_ts : (int64_t)n_kv_heads * head_dim);
  if (((n_kv - 1) * k_tok + head_dim) * 2 >= ((int64_t)1 << 31) ||
      (int64_t)rk_attn_dv_pad(head_dim) * n_kv_pad * 2 >= ((int64_t)1 << 31))
    return fail(RK_E_SHAPE, op, "one kv head's K rows or Vᵀ reach 2 GiB");
  AttnArgs a{};
  a.q = q;
  a.k = k;
  a.vt = vt;
  a.out = out;
  if (head_major) {
    a.q_tok_stride = head_dim;
    a.q_head_stride = n_q * head_dim;
    a.k_tok_stride = head_dim;
    a.k_head_stride = n_kv * head_dim;
    a.o_tok_stride = head_dim;
    a.o_head_stride = n_q * head_dim;
  } else {
    a.q_tok_stride = q_ts ? q_ts : (int64_t)n_head * head_dim;
    a.q_head_stride = head_dim;
    a.k_tok_stride = k_ts ? k_ts : (int64_t)n_kv_heads * head_dim;
    a.k_head_stride = head_dim;
    a.o_tok_stride = o_ts ? o_ts : (int64_t)n_head * head_dim;
    a.o_head_stride = head_dim;
  }
  a.n_q = (int)n_q;
  a.n_kv = (int)n_kv;
  a.n_kv_pad = (int)n_kv_pad;
  a.n_head = n_head;
  a.n_kv_heads = n_kv_heads;
  a.head_dim = head_dim;
  a.scale = scale;
  a.softcap = softcap;
  a.mask_mode = mode;
  a.window = window;
  a.q0 = q0;
  a.k0 = k0;
  a.num_cus = g_eng->num_cus;
  const long split = cs ? rk_attn_split_tiles(a) : 0;
  if (split > 0) {
    // Partial states (two per split tile) and arrival counters. The counters
    // start at zero and every launch leaves them at zero.
    // A new counter buffer is zeroed whole: a later launch with more query
    // tiles uses counters past this one's.
    void *part, *cnt;
    bool fresh = false;
    const size_t cnt_bytes = std::max<size_t>((size_t)split * 4, 256);
    RK_TRY(scratch(*cs, "attn_part", (size_t)split * 2 * rk_attn_split_floats(head_dim) * 4, &part));
    RK_TRY(scratch(*cs, "attn_cnt", cnt_bytes, &cnt, &fresh));
    if (fresh) HIP_TRY(hipMemsetAsync(cnt, 0, cnt_bytes, st), op);
    a.part = (float *)part;
    a.cnt = (unsigned *)cnt;
    a.n_split = (int)split;
  }
  HIP_TRY(rk_launch_attention(a, st), op);
  return RK_OK;
}

// Token-major attention on device buffers: Vᵀ into scratch, then the kernel.
int attn_dev_impl(CallScope &cs, const void *q, const void *k, const void *v, int64_t n_q,
                  int64_t n_kv, int n_head, int n_kv_heads, int head_dim, float scale,
                  float softcap, int mode, int64_t window, int64_t q0, int64_t k0, void *out,
                  const char *op, int64_t q_ts = 0, int64_t k_ts = 0, int64_t v_ts = 0,
                  int64_t o_ts = 0) {
  // Head dims of the reference's contract (head_dim % 32, attn/mod.rs:1443)
  // between the kernel widths (160, 192, 224) run zero-padded to 256 on
  // packed token-major operands: zero q/k columns leave the scores, zero V
  // columns only give output columns that are not copied back.
  const int pad_w = head_dim > 128 && head_dim < 256 && head_dim % 32 == 0 ? 256 : 0;
  if (pad_w) {
    if ((q_ts && q_ts != (int64_t)n_head * head_dim) || (k_ts && k_ts != (int64_t)n_kv_heads * head_dim) ||
        (v_ts && v_ts != (int64_t)n_kv_heads * head_dim) || (o_ts && o_ts != (int64_t)n_head * head_dim))
      return fail(RK_E_UNSUPPORTED, op, "head_dim " + std::to_string(head_dim) + " with token strides");
    RK_TRY(attn_check(n_q, n_kv, n_head, n_kv_heads, pad_w, &mode, window, op));
    const size_t hd = (size_t)head_dim * 2, w = (size_t)pad_w * 2;
    void *qp, *kp, *vp, *op_;
    RK_TRY(scratch(cs, "attn_pad_q", (size_t)n_q * n_head * w, &qp));
    RK_TRY(scratch(cs, "attn_pad_k", (size_t)n_kv * n_kv_heads * w, &kp));
    RK_TRY(scratch(cs, "attn_pad_v", (size_t)n_kv * n_kv_heads * w, &vp));
    RK_TRY(scratch(cs, "attn_pad_o", (size_t)n_q * n_head * w, &op_));
    const struct {
      const void *src;
      void *dst;
      size_t rows;
    } in[3] = {{q, qp, (size_t)n_q * n_head}, {k, kp, (size_t)n_kv * n_kv_heads},
               {v, vp, (size_t)n_kv * n_kv_heads}};
    for (const auto &t : in) {
      HIP_TRY(hipMemsetAsync(t.dst, 0, t.rows * w, cs.st), op);
      HIP_TRY(hipMemcpy2DAsync(t.dst, w, t.src, hd, hd, t.rows, hipMemcpyDeviceToDevice, cs.st), op);
    }
    RK_TRY(attn_dev_impl(cs, qp, kp, vp, n_q, n_kv, n_head, n_kv_heads, pad_w, scale, softcap, mode,
                         window, q0, k0, op_, op));
    HIP_TRY(hipMemcpy2DAsync(out, hd, op_, w, hd, (size_t)n_q * n_head, hipMemcpyDeviceToDevice, cs.st),
            op);
    return RK_OK;
  }
  RK_TRY(attn_check(n_q, n_kv, n_head, n_kv_heads, head_dim, &mode, window, op));
  const int dvp = rk_attn_dv_pad(head_dim);
  const int64_t n_kv_pad = round_up_i(n_kv, rk_attn_kv_tile());
  if ((int64_t)dvp * n_kv_pad * 2 >= ((int64_t)1 << 31))
    return fail(RK_E_SHAPE, op, "one kv head's Vᵀ reaches 2 GiB");
  void *vt;
  RK_TRY(scratch(cs, "attn_vt", (size_t)n_kv_heads * dvp * n_kv_pad * 2, &vt));
  HIP_TRY(rk_launch_v_transpose(v, v_ts ? v_ts : (int64_t)n_kv_heads * head_dim, head_dim,
                                (int)n_kv, (int)n_kv_pad, n_kv_heads, head_dim, dvp, vt, cs.st),
          op);
  return attn_run(q, k, vt, out, n_q, n_kv, n_kv_pad, n_head, n_kv_heads, head_dim, scale, softcap,
                  mode, window, q0, k0, false, cs.st, op, &cs, q_ts, k_ts, o_ts);
}
}  // namespace

extern "C" int rk_attention_dev(const void *q, const void *k, const void *v, int64_t n_q,
                                int64_t n_kv, int n_head, int n_kv_heads, int head_dim,
                                float scale, float softcap, int mask_mode, int64_t window,
                                int64_t q0, int64_t k0, void *out, rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_attention_dev"));
  CallScope cs(pick(stream));
  RK_TRY(attn_dev_impl(cs, q, k, v, n_q, n_kv, n_head, n_kv_heads, head_dim, scale, softcap,
                       mask_mode, window, q0, k0, out, "rk_attention_dev"));
  g_eng->calls++;
  return RK_OK;
}

extern "C" int rk_attention_strided_dev(const void *q, int64_t q_stride, const void *k,
                                        int64_t k_stride, const void *v, int64_t v_stride,
                                        int64_t n_q, int64_t n_kv, int n_head, int n_kv_heads,
                                        int head_dim, float scale, float softcap, int mask_mode,
                                        int64_t window, int64_t q0, int64_t k0, void *out,
                                        int64_t out_stride, rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  const char *name = "rk_attention_strided_dev";
  RK_TRY(ensure(name));
  const int64_t qw = (int64_t)n_head * head_dim, kw = (int64_t)n_kv_heads * head_dim;
  if (q_stride < qw || out_stride < qw || k_stride < kw || v_stride < kw)
    return fail(RK_E_SHAPE, name, "a token stride is shorter than the token's heads");
  if ((q_stride | k_stride | v_stride | out_stride) % 8 != 0 ||
      (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) & 15) != 0)
    return fail(RK_E_SHAPE, name, "token strides must be multiples of 8 values, buffers 16-byte aligned");
  CallScope cs(pick(stream));
  RK_TRY(attn_dev_impl(cs, q, k, v, n_q, n_kv, n_head, n_kv_heads, head_dim, scale, softcap,
                       mask_mode, window, q0, k0, out, name, q_stride, k_stride, v_stride,
                       out_stride));
  g_eng->calls++;
  return RK_OK;
}

extern "C" int rk_attention_dev_noalloc(const void *q, const void *k, const void *v, int64_t n_q,
                                        int64_t n_kv, int n_head, int n_kv_heads, int head_dim,
                                        float scale, float softcap, int mask_mode, int64_t window,
                                        int64_t q0, int64_t k0, void *out, rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  const char *op = "rk_attention_dev_noalloc";
  RK_TRY(ensure(op));
  int mode = mask_mode;
  RK_TRY(attn_check(n_q, n_kv, n_head, n_kv_heads, head_dim, &mode, window, op));
  const int dvp = rk_attn_dv_pad(head_dim);
  const int64_t n_kv_pad = round_up_i(n_kv, rk_attn_kv_tile());
  const int64_t need = (int64_t)n_kv_heads * dvp * n_kv_pad * 2;
  if (need > (int64_t)RK_NOALLOC_SCRATCH_BYTES)
    return fail(RK_E_NOMEM, op,
                "V transposed needs " + std::to_string(need) + " bytes, above the " +
                    std::to_string(RK_NOALLOC_SCRATCH_BYTES) + "-byte static scratch");
  void *vt = rk_noalloc_scratch(g_eng->device);
  if (!vt) return fail(RK_E_DEVICE, op, "the static scratch was not set up on this device");
  hipStream_t st = pick(stream);
  // Every Vᵀ element the kernel reads (padding rows and keys included) is
  // written here first, so nothing is left from an earlier call.
  HIP_TRY(rk_launch_v_transpose(v, (int64_t)n_kv_heads * head_dim, head_dim, (int)n_kv,
                                (int)n_kv_pad, n_kv_heads, head_dim, dvp, vt, st),
          op);
  RK_TRY(attn_run(q, k, vt, out, n_q, n_kv, n_kv_pad, n_head, n_kv_heads, head_dim, scale, softcap,
                  mode, window, q0, k0, false, st, op, nullptr));
  g_eng->calls++;
  return RK_OK;
}

namespace {
// RK_E_RANGE after a host-buffer attention whose q or k held a value that
// fp16 cannot represent: the reference converts them to fp16 the same way
// and answers Status::Range when a score leaves fp16's range
// (attn/softmax.rs:462-475, attn/mod.rs:1044-1046). The scores themselves are
// f32 here and cannot saturate.
int range_flag(const int *flag, const char *op) {
  int h = 0;
  HIP_TRY(hipMemcpy(&h, flag, 4, hipMemcpyDeviceToHost), op);
  if (h) return fail(RK_E_RANGE, op, "q or k holds a value outside the fp16 range");
  return RK_OK;
}
}  // namespace

extern "C" int rk_attention(const float *q, const float *k, const float *v, int64_t n_q,
                            int64_t n_kv, int n_head, int n_kv_heads, int head_dim, float scale,
                            float softcap, int mask_mode, int64_t window, int64_t q0, int64_t k0,
                            float *out) {
  std::lock_guard<std::mutex> lk(g_mu);
  const char *op = "rk_attention";
  RK_TRY(ensure(op));
  int mode = mask_mode;
  RK_TRY(attn_check(n_q, n_kv, n_head, n_kv_heads, head_dim, &mode, window, op, true));
  hipStream_t st = g_eng->stream;
  CallScope cs(st);
  const size_t nq_el = (size_t)n_q * n_head * head_dim;
  const size_t nk_el = (size_t)n_kv * n_kv_heads * head_dim;
  float *f32;
  void *q16, *k16, *v16, *o16;
  int *flag;
  RK_TRY(scratch(cs, "at_f32", (nq_el + 2 * nk_el) * 4, (void **)&f32));
  RK_TRY(scratch(cs, "at_q16", nq_el * 2, &q16));
  RK_TRY(scratch(cs, "at_k16", nk_el * 2, &k16));
  RK_TRY(scratch(cs, "at_v16", nk_el * 2, &v16));
  RK_TRY(scratch(cs, "at_o16", nq_el * 2, &o16));
  RK_TRY(scratch(cs, "at_flag", 4, (void **)&flag));
  float *q32 = f32, *k32 = q32 + nq_el, *v32 = k32 + nk_el;
  auto compute = [&](int64_t, int64_t) {
    HIP_TRY(hipMemsetAsync(flag, 0, 4, st), op);
    HIP_TRY(rk_launch_f32_to_f16_checked(q32, q16, (int64_t)nq_el, flag, st), op);
    HIP_TRY(rk_launch_f32_to_f16_checked(k32, k16, (int64_t)nk_el, flag, st), op);
    HIP_TRY(rk_launch_f32_to_f16(v32, v16, (int64_t)nk_el, st), op);
    RK_TRY(attn_dev_impl(cs, q16, k16, v16, n_q, n_kv, n_head, n_kv_heads, head_dim, scale, softcap,
                         mode, window, q0, k0, o16, op));
    // the output overwrites q's f32 copy, which is no longer read
    HIP_TRY(rk_launch_f16_to_f32(o16, q32, (int64_t)nq_el, st), op);
    return RK_OK;
  };
  RK_TRY(staged(cs, {{q, nullptr, q32, 0, nq_el * 4}, {k, nullptr, k32, 0, nk_el * 4}, {v, nullptr, v32, 0, nk_el * 4}},
                {{nullptr, out, q32, 0, nq_el * 4}}, 1, 1, compute, op));
  RK_TRY(range_flag(flag, op));
  g_eng->calls++;
  return RK_OK;
}

namespace {
int flash_impl(int64_t n_q, int64_t n_kv, int head_dim, int dv, int n_head, int n_kv_heads, float scale,
               float softcap, int mask_mode, int64_t window, int64_t q0, int64_t k0, const uint16_t *q,
               const uint16_t *k, const uint16_t *v, uint16_t *out, const char *op) {
  RK_TRY(ensure(op));
  if (head_dim <= 0 || dv <= 0) return fail(RK_E_SHAPE, op, "head_dim and dv must be positive");
  // The kernel runs one width D for q, k and v, the smallest kernel width at
  // least max(head_dim, dv): zero columns added to q and k leave every score
  // unchanged, zero rows added to Vᵀ only add zero output columns, so the
  // first dv output columns are the attention of the given operands (the
  // reference pads Clef's 72-wide heads to head_dim 96 / dv 80 the same way,
  // src/clef/vision/npu.rs:211-230). Its own contract, head_dim % 32 and
  // dv % 16 with no upper bound (attn/mod.rs:1443), is met here up to 256.
  int D = 0;
  for (int w : {32, 48, 64, 72, 80, 96, 112, 128, 256})
    if (D == 0 && std::max(head_dim, dv) <= w) D = w;
  if (D == 0)
    return fail(RK_E_UNSUPPORTED, op,
                "head_dim " + std::to_string(head_dim) + " / dv " + std::to_string(dv) +
                    " above the widest kernel (256)");
  int mode = mask_mode;
  RK_TRY(attn_check(n_q, n_kv, n_head, n_kv_heads, D, &mode, window, op));
  hipStream_t st = g_eng->stream;
  CallScope cs(st);
  const size_t q_in = (size_t)n_head * n_q * head_dim, k_in = (size_t)n_kv_heads * n_kv * head_dim;
  const size_t v_in = (size_t)n_kv_heads * dv * n_kv, o_out = (size_t)n_head * n_q * dv;
  const size_t nq_el = (size_t)n_q * n_head * D, nk_el = (size_t)n_kv * n_kv_heads * D;
  const int dvp = rk_attn_dv_pad(D);
  const int64_t n_kv_pad = round_up_i(n_kv, rk_attn_kv_tile());
  char *raw;
  void *q16, *k16, *o16, *vt;
  RK_TRY(scratch(cs, "fa_raw", (q_in + k_in + v_in + o_out) * 2, (void **)&raw));
  RK_TRY(scratch(cs, "at_q16", nq_el * 2, &q16));
  RK_TRY(scratch(cs, "at_k16", nk_el * 2, &k16));
  RK_TRY(scratch(cs, "at_o16", nq_el * 2, &o16));
  RK_TRY(scratch(cs, "attn_vt", (size_t)n_kv_heads * dvp * n_kv_pad * 2, &vt));
  char *q_raw = raw, *k_raw = q_raw + q_in * 2, *v_raw = k_raw + k_in * 2, *o_raw = v_raw + v_in * 2;
  auto compute = [&](int64_t, int64_t) {
    // q [H][n_q][head_dim] and k [KV][n_kv][head_dim] into rows of D values.
    const struct {
      const char *src;
      void *dst;
      size_t rows;
    } qk[2] = {{q_raw, q16, (size_t)n_head * n_q}, {k_raw, k16, (size_t)n_kv_heads * n_kv}};
    for (const auto &t : qk) {
      if (head_dim < D) {
        HIP_TRY(hipMemsetAsync(t.dst, 0, t.rows * D * 2, st), op);
        HIP_TRY(hipMemcpy2DAsync(t.dst, (size_t)D * 2, t.src, (size_t)head_dim * 2, (size_t)head_dim * 2,
                                 t.rows, hipMemcpyDeviceToDevice, st),
                op);
      } else {
        HIP_TRY(hipMemcpyAsync(t.dst, t.src, t.rows * D * 2, hipMemcpyDeviceToDevice, st), op);
      }
    }
    // v is [KV][dv][n_kv]: element (key, head, d) at head·dv·n_kv + d·n_kv + key;
    // its dv rows fill Vᵀ, the rest of the D rows are zero.
    HIP_TRY(rk_launch_v_transpose_strided(v_raw, 1, (int64_t)dv * n_kv, n_kv, (int)n_kv, (int)n_kv_pad,
                                          n_kv_heads, dv, dvp, vt, st),
            op);
    RK_TRY(attn_run(q16, k16, vt, o16, n_q, n_kv, n_kv_pad, n_head, n_kv_heads, D, scale, softcap, mode,
                    window, q0, k0, true, st, op, &cs));
    // out [H][n_q][dv]: the first dv columns of each output row.
    HIP_TRY(hipMemcpy2DAsync(o_raw, (size_t)dv * 2, o16, (size_t)D * 2, (size_t)dv * 2, (size_t)n_head * n_q,
                             hipMemcpyDeviceToDevice, st),
            op);
    return RK_OK;
  };
  RK_TRY(staged(cs, {{q, nullptr, q_raw, 0, q_in * 2}, {k, nullptr, k_raw, 0, k_in * 2}, {v, nullptr, v_raw, 0, v_in * 2}},
                {{nullptr, out, o_raw, 0, o_out * 2}}, 1, 1, compute, op));
  g_eng->calls++;
  return RK_OK;
}

// The additive masks of masks.rs:11-114 (0 visible, -inf hidden) in the
// kernel's predicate form: each row's visible keys must be one interval and
// the rows' intervals those of one mode at one query-key offset d = q0 - k0
// (relative query i sees relative key j as absolute t = i + d against j).
struct MaskFit {
  int mode = RK_MASK_NONE;
  int64_t window = -1, q0 = 0, k0 = 0;
};

int classify_mask(const uint16_t *mask, int64_t n_q, int64_t n_kv, MaskFit *fit, const char *op) {
  std::vector<int64_t> lo(n_q), hi(n_q);  // visible interval per row; lo > hi: none
  bool all_full = true;
  for (int64_t i = 0; i < n_q; ++i) {
    const uint16_t *row = mask + i * n_kv;
    int64_t first = -1, last = -2, count = 0;
    for (int64_t j = 0; j < n_kv; ++j) {
      const uint16_t m = row[j];
      if ((m & 0x7fff) == 0) {
        if (first < 0) first = j;
        last = j;
        ++count;
      } else if (m != 0xfc00) {
        return fail(RK_E_UNSUPPORTED, op, "an additive mask value other than 0 and -inf");
      }
    }
    if (first < 0) first = 0, last = -1;
    if (count != last - first + 1)
      return fail(RK_E_UNSUPPORTED, op, "a mask row whose visible keys are not one interval");
    lo[i] = first;
    hi[i] = last;
    all_full = all_full && first == 0 && last == n_kv - 1;
  }
  if (all_full) return RK_OK;
  // Offsets of the unclipped ends: hi = i + dh (causal, window, causal window)
  // and lo = i + dl (window, causal window).
  bool has_h = false, has_l = false;
  int64_t dh = 0, dl = 0, first_full = -1;
  for (int64_t i = 0; i < n_q; ++i) {
    if (lo[i] > hi[i]) continue;
    if (!has_h && hi[i] < n_kv - 1) has_h = true, dh = hi[i] - i;
    if (!has_l && lo[i] > 0) has_l = true, dl = lo[i] - i;
    if (first_full < 0 && lo[i] == 0 && hi[i] == n_kv - 1) first_full = i;
  }
  const int64_t big = n_q + n_kv + 1;
  struct Cand {
    int mode;
    int64_t d, w;
  };
  std::vector<Cand> cands;
  if (has_h) cands.push_back({RK_MASK_CAUSAL, dh, -1});
  if (has_h && has_l && dh - dl + 1 >= 1) cands.push_back({RK_MASK_CAUSAL_WINDOW, dh, dh - dl + 1});
  if (has_h && has_l && (dh - dl) % 2 == 0 && dh >= dl)
    cands.push_back({RK_MASK_WINDOW, (dh + dl) / 2, (dh - dl) / 2});
  if (!has_h && has_l) {
    cands.push_back({RK_MASK_WINDOW, dl + big, big});
    cands.push_back({RK_MASK_CAUSAL_WINDOW, n_kv + big, n_kv + big - dl + 1});
  }
  if (!has_h && !has_l) {
    if (first_full >= 0) cands.push_back({RK_MASK_CAUSAL, n_kv - 1 - first_full, -1});
    cands.push_back({RK_MASK_CAUSAL, -(n_q + 1), -1});  // every row hidden
  }
  for (const Cand &c : cands) {
    bool ok = true;
    for (int64_t i = 0; i < n_q && ok; ++i) {
      const int64_t t = i + c.d;
      int64_t a, b;
      if (c.mode == RK_MASK_CAUSAL)
        a = 0, b = t;
      else if (c.mode == RK_MASK_WINDOW)
        a = t - c.w, b = t + c.w;
      else
        a = t - c.w + 1, b = t;
      a = std::max<int64_t>(a, 0);
      b = std::min<int64_t>(b, n_kv - 1);
      const bool empty = a > b, row_empty = lo[i] > hi[i];
      ok = empty ? row_empty : (!row_empty && a == lo[i] && b == hi[i]);
    }
    if (ok) {
      fit->mode = c.mode;
      fit->window = c.w;
      fit->q0 = std::max<int64_t>(c.d, 0);
      fit->k0 = std::max<int64_t>(-c.d, 0);
      return RK_OK;
    }
  }
  return fail(RK_E_UNSUPPORTED, op, "an additive mask that is not a causal, band or causal-window mask");
}
}  // namespace

extern "C" int rk_flash_attn_f16(int64_t n_q, int64_t n_kv, int head_dim, int dv, int n_head,
                                 int n_kv_heads, float scale, float softcap, int mask_mode,
                                 int64_t window, int64_t q0, int64_t k0, const uint16_t *q,
                                 const uint16_t *k, const uint16_t *v, uint16_t *out) {
  std::lock_guard<std::mutex> lk(g_mu);
  return flash_impl(n_q, n_kv, head_dim, dv, n_head, n_kv_heads, scale, softcap, mask_mode, window, q0, k0,
                    q, k, v, out, "rk_flash_attn_f16");
}

extern "C" int rk_flash_attn_f16_masked(int64_t n_q, int64_t n_kv, int head_dim, int dv, int n_head,
                                        int n_kv_heads, float scale, float softcap, const uint16_t *mask,
                                        const uint16_t *q, const uint16_t *k, const uint16_t *v,
                                        uint16_t *out) {
  std::lock_guard<std::mutex> lk(g_mu);
  const char *op = "rk_flash_attn_f16_masked";
  if (n_q <= 0 || n_kv <= 0) return fail(RK_E_SHAPE, op, "empty query or key axis");
  MaskFit fit;
  if (mask) RK_TRY(classify_mask(mask, n_q, n_kv, &fit, op));
  return flash_impl(n_q, n_kv, head_dim, dv, n_head, n_kv_heads, scale, softcap, fit.mode, fit.window, fit.q0,
                    fit.k0, q, k, v, out, op);
}

// =========================================================================
// MoE
// =========================================================================
extern "C" int rk_moe_route(const float *logits, int64_t s, int n_experts, int top_k,
                            int norm_topk, uint32_t *ids, float *wts) {
  if (s < 0 || n_experts <= 0 || top_k <= 0 || top_k > n_experts)
    return fail(RK_E_SHAPE, "rk_moe_route", "need 0 < top_k <= n_experts");
  std::vector<float> p(n_experts);
  std::vector<int> order(n_experts);
  for (int64_t t = 0; t < s; ++t) {
    const float *l = logits + t * n_experts;
    // softmax_row (src/clef/math.rs:138-148): max, exp(v - max), sum, divide.
    float mx = -INFINITY;
    for (int e = 0; e < n_experts; ++e) mx = std::max(mx, l[e]);
    float sum = 0.f;
    for (int e = 0; e < n_experts; ++e) {
      p[e] = std::exp(l[e] - mx);
      sum += p[e];
    }
    for (int e = 0; e < n_experts; ++e) p[e] /= sum;
    for (int e = 0; e < n_experts; ++e) order[e] = e;
    // Descending probability, ties to the lower id (model.rs:475).
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
      if (p[a] != p[b]) return p[a] > p[b];
      return a < b;
    });
    float sel = 0.f;
    for (int j = 0; j < top_k; ++j) sel += p[order[j]];
    for (int j = 0; j < top_k; ++j) {
      ids[t * top_k + j] = (uint32_t)order[j];
      wts[t * top_k + j] = norm_topk ? p[order[j]] / sel : p[order[j]];
    }
  }
  return RK_OK;
}

namespace {
// Bytes of one expert's fragment-major codes (blocks per row padded to a
// multiple of 4, q8_code_offset in kernels.hpp).
int64_t moe_gu_code_stride(const Weight &w) { return 2 * w.inter * w.gu_ws_stride * 32; }
int64_t moe_dn_code_stride(const Weight &w) { return w.hidden * w.dn_ws_stride * 32; }

}  // namespace

namespace {
int moe_alloc(Weight &w, int n_experts, int64_t H, int64_t I, const char *op) {
  w.moe = true;
  w.n_experts = n_experts;
  w.hidden = H;
  w.inter = I;
  w.n = H;
  w.k = H;
  w.group = 32;
  w.gu_ws_stride = ws_stride_for(H);
  w.dn_ws_stride = ws_stride_for(I);
  const int64_t E = n_experts;
  const size_t gu_codes = (size_t)E * moe_gu_code_stride(w), dn_codes = (size_t)E * moe_dn_code_stride(w);
  const size_t gu_sc = (size_t)E * 2 * I * w.gu_ws_stride, dn_sc = (size_t)E * H * w.dn_ws_stride;
  HIP_TRY(hipMalloc((void **)&w.gu_codes, gu_codes), op);
  HIP_TRY(hipMalloc((void **)&w.dn_codes, dn_codes), op);
  HIP_TRY(hipMalloc((void **)&w.gu_scales, gu_sc * 4), op);
  HIP_TRY(hipMalloc((void **)&w.dn_scales, dn_sc * 4), op);
  // Padding blocks of the fragment-major layout stay zero.
  HIP_TRY(hipMemset(w.gu_codes, 0, gu_codes), op);
  HIP_TRY(hipMemset(w.dn_codes, 0, dn_codes), op);
  HIP_TRY(hipMemset(w.gu_scales, 0, gu_sc * 4), op);
  HIP_TRY(hipMemset(w.dn_scales, 0, dn_sc * 4), op);
  w.bytes = gu_codes + dn_codes + (gu_sc + dn_sc) * 4;
  return RK_OK;
}
}  // namespace

extern "C" int rk_pack_moe_q8_0(const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                                int n_experts, int64_t hidden, int64_t inter, rk_weight_id *id) {
  std::lock_guard<std::mutex> lk(g_mu);
  const char *op = "rk_pack_moe_q8_0";
  RK_TRY(ensure(op));
  if (n_experts <= 0 || hidden <= 0 || inter <= 0 || hidden % 32 || inter % 32)
    return fail(RK_E_SHAPE, op, "hidden and inter must be multiples of 32");
  const int64_t H = hidden, I = inter, E = n_experts;
  Weight w;
  PackGuard guard(w);
  RK_TRY(moe_alloc(w, n_experts, H, I, op));
  CallScope cs(g_eng->stream);
  hipStream_t st = cs.st;
  // Per expert: one upload of its gate, up and down blocks, split on the device
  // into the fragment-major stacks (gate|up interleaved per 16-row slice).
  const size_t gblk = (size_t)I * (H / 32) * 34, dblk = (size_t)H * (I / 32) * 34;
  void *dev;
  RK_TRY(scratch(cs, "pack_blk", 2 * gblk + dblk, &dev));
  uint8_t *dg = (uint8_t *)dev, *du = dg + gblk, *dd = du + gblk;
  const int64_t gu_stride = moe_gu_code_stride(w), dn_stride = moe_dn_code_stride(w);
  for (int64_t e = 0; e < E; ++e) {
    HIP_TRY(hipMemcpyAsync(dg, gate + e * gblk, gblk, hipMemcpyHostToDevice, st), op);
    HIP_TRY(hipMemcpyAsync(du, up + e * gblk, gblk, hipMemcpyHostToDevice, st), op);
    HIP_TRY(hipMemcpyAsync(dd, down + e * dblk, dblk, hipMemcpyHostToDevice, st), op);
    int8_t *guc = w.gu_codes + e * gu_stride;
    float *gus = w.gu_scales + e * 2 * I * w.gu_ws_stride;
    HIP_TRY(rk_launch_q8_0_unpack(dg, I, H, 32, 0, guc, gus, w.gu_ws_stride, true, st), op);
    HIP_TRY(rk_launch_q8_0_unpack(du, I, H, 32, 16, guc, gus, w.gu_ws_stride, true, st), op);
    HIP_TRY(rk_launch_q8_0_unpack(dd, H, I, 16, 0, w.dn_codes + e * dn_stride,
                                  w.dn_scales + e * H * w.dn_ws_stride, w.dn_ws_stride, true, st),
            op);
  }
  HIP_TRY(hipStreamSynchronize(st), op);
  *id = guard.register_weight();
  return RK_OK;
}

extern "C" int rk_pack_moe_f32(const float *gate, const float *up, const float *down, int n_experts,
                               int64_t hidden, int64_t inter, rk_weight_id *id) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_pack_moe_f32"));
  if (n_experts <= 0 || hidden <= 0 || inter <= 0 || hidden % 32 || inter % 32)
    return fail(RK_E_SHAPE, "rk_pack_moe_f32", "hidden and inter must be multiples of 32");
  const int64_t H = hidden, I = inter, E = n_experts;
  Weight w;
  PackGuard guard(w);
  RK_TRY(moe_alloc(w, n_experts, H, I, "rk_pack_moe_f32"));
  CallScope cs(g_eng->stream);
  void *x32;
  RK_TRY(scratch(cs, "pack_f32", (size_t)I * H * 4, &x32));
  hipStream_t st = g_eng->stream;
  const int64_t gu_stride = moe_gu_code_stride(w), dn_stride = moe_dn_code_stride(w);
  for (int64_t e = 0; e < E; ++e) {
    int8_t *guc = w.gu_codes + e * gu_stride;
    float *gus = w.gu_scales + e * 2 * I * w.gu_ws_stride;
    const float *src[3] = {gate + e * I * H, up + e * I * H, down + e * H * I};
    for (int part = 0; part < 3; ++part) {
      HIP_TRY(hipMemcpyAsync(x32, src[part], (size_t)I * H * 4, hipMemcpyHostToDevice, st),
              "rk_pack_moe_f32");
      if (part < 2)
        HIP_TRY(rk_launch_q8_0_quantize((const float *)x32, I, H, 32, 16 * part, guc, gus,
                                        w.gu_ws_stride, true, st),
                "rk_pack_moe_f32");
      else
        HIP_TRY(rk_launch_q8_0_quantize((const float *)x32, H, I, 16, 0, w.dn_codes + e * dn_stride,
                                        w.dn_scales + e * H * w.dn_ws_stride, w.dn_ws_stride, true,
                                        st),
                "rk_pack_moe_f32");
    }
  }
  HIP_TRY(hipStreamSynchronize(st), "rk_pack_moe_f32");
  *id = guard.register_weight();
  return RK_OK;
}

namespace {
// Device-resident routing lists of one MoE call.
struct MoePlan {
  int64_t s = 0;
  int top_k = 0;
  int64_t rows = 0;
  int n_tiles = 0;
  int tile_rows = 128;        // rows per tile at most (the kernels' tile size)
  int32_t *tok = nullptr;     // [rows] token of each bucket row
  float *roww = nullptr;      // [rows] router weight of each bucket row
  int32_t *slot = nullptr;    // [s, top_k] bucket rows of a token, ascending expert id
  MoeTile *tiles = nullptr;   // [n_tiles] in expert order (down)
  MoeTile *tiles_gu = nullptr;  // [n_tiles] the same tiles, longest first (gate|up)
  uint64_t weight = 0;        // expert stack the plan was made for
  // Streams of the runs that read the lists: a library stream is
  // synchronized when the plan is destroyed; a caller's stream gets an event
  // recorded after each run there.
  mutable std::vector<std::pair<hipStream_t, hipEvent_t>> uses;
};

void plan_free(MoePlan *p) {
  if (!p) return;
  for (auto &u : p->uses)
    if (u.second) (void)hipEventDestroy(u.second);
  (void)hipFree(p->tok);
  (void)hipFree(p->roww);
  (void)hipFree(p->slot);
  (void)hipFree(p->tiles);
  (void)hipFree(p->tiles_gu);
  delete p;
}

// Bucket the (token, slot) pairs per expert in ascending token order
// (engine.rs:292-305), list tiles of ≤ rk_moe_tile_rows() rows (two tiles of
// one expert sit next to each other, so the second read of its weights is
// mostly served from cache), and sort each token's slot rows by
// expert id for the combine; the lists are copied into the plan's buffers.
int moe_plan(const Weight &w, int64_t s, int top_k, const uint32_t *ids, const float *wts,
             MoePlan *plan, hipStream_t st) {
  const char *op = "rk_moe_plan";
  const int E = w.n_experts;
  std::vector<int64_t> count(E, 0);
  for (int64_t i = 0; i < s * top_k; ++i) {
    if (ids[i] >= (uint32_t)E) return fail(RK_E_SHAPE, op, "expert id out of range");
    count[ids[i]]++;
  }
  std::vector<int64_t> off(E + 1, 0);
  for (int e = 0; e < E; ++e) off[e + 1] = off[e] + count[e];
  const int64_t R = off[E];
  std::vector<int32_t> tok(R), slot(s * top_k);
  std::vector<float> roww(R);
  std::vector<int64_t> fill(off.begin(), off.end() - 1);
  for (int64_t t = 0; t < s; ++t)
    for (int j = 0; j < top_k; ++j) {
      const int e = (int)ids[t * top_k + j];
      const int64_t row = fill[e]++;
      tok[row] = (int32_t)t;
      roww[row] = wts[t * top_k + j];
      slot[t * top_k + j] = (int32_t)row;
    }
  // Rows of one expert are contiguous and expert-major, so ordering a token's
  // slots by row is ordering them by expert id.
  for (int64_t t = 0; t < s; ++t) std::sort(slot.begin() + t * top_k, slot.begin() + (t + 1) * top_k);
  std::vector<MoeTile> tiles;
  const int tr = rk_moe_tile_rows();
  for (int e = 0; e < E; ++e)
    for (int64_t r = off[e]; r < off[e + 1]; r += tr)
      tiles.push_back(MoeTile{e, (int)r, (int)std::min<int64_t>(tr, off[e + 1] - r)});
  // gate|up takes the tiles longest first (a tile's time grows with its
  // 32-row blocks; ties in expert order): the kernels put tile t on XCD t mod 8
  // and each XCD takes its tiles in list order, so every XCD runs its longest
  // tiles first and the short ones fill the last round. Per-workgroup
  // timestamps of a 30B-A3B expert layer (1024 tokens, top-8 of 128) on
  // MI355X: gate|up 148 -> 141 us; the down kernel in the same order took
  // 98 -> 107 us (its shortest tiles, run last, then carry most of the
  // combine's merges), so it keeps expert order. Neither result depends on
  // the order: the combine sums a token's rows in ascending expert id.
  std::vector<MoeTile> tiles_gu(tiles);
  std::stable_sort(tiles_gu.begin(), tiles_gu.end(),
                   [](const MoeTile &x, const MoeTile &y) { return (x.rows + 31) / 32 > (y.rows + 31) / 32; });
  HIP_TRY(hipMalloc((void **)&plan->tok, std::max<size_t>(R, 1) * 4), op);
  HIP_TRY(hipMalloc((void **)&plan->roww, std::max<size_t>(R, 1) * 4), op);
  HIP_TRY(hipMalloc((void **)&plan->slot, std::max<size_t>(slot.size(), 1) * 4), op);
  HIP_TRY(hipMalloc((void **)&plan->tiles, std::max<size_t>(tiles.size(), 1) * sizeof(MoeTile)), op);
  HIP_TRY(hipMalloc((void **)&plan->tiles_gu, std::max<size_t>(tiles.size(), 1) * sizeof(MoeTile)), op);
  if (R) {
    HIP_TRY(hipMemcpyAsync(plan->tok, tok.data(), R * 4, hipMemcpyHostToDevice, st), op);
    HIP_TRY(hipMemcpyAsync(plan->roww, roww.data(), R * 4, hipMemcpyHostToDevice, st), op);
    HIP_TRY(hipMemcpyAsync(plan->tiles, tiles.data(), tiles.size() * sizeof(MoeTile),
                           hipMemcpyHostToDevice, st),
            op);
    HIP_TRY(hipMemcpyAsync(plan->tiles_gu, tiles_gu.data(), tiles_gu.size() * sizeof(MoeTile),
                           hipMemcpyHostToDevice, st),
            op);
  }
  if (!slot.empty())
    HIP_TRY(hipMemcpyAsync(plan->slot, slot.data(), slot.size() * 4, hipMemcpyHostToDevice, st), op);
  // The host vectors die at return: finish the copies first.
  HIP_TRY(hipStreamSynchronize(st), op);
  plan->s = s;
  plan->top_k = top_k;
  plan->rows = R;
  plan->n_tiles = (int)tiles.size();
  plan->tile_rows = tr;
  return RK_OK;
}

int moe_run(CallScope &cs, const Weight &w, const MoePlan &plan, const float *x, float *y,
            float *act_out = nullptr, bool accumulate = false) {
  hipStream_t st = cs.st;
  const int64_t H = w.hidden, I = w.inter, S = plan.s, R = std::max<int64_t>(plan.rows, 1);
  const int64_t KBh = H / 32, KBi = I / 32;  // 32-value activation groups per row
  void *xq, *xs, *act, *aq, *as, *yb, *cnt;
  RK_TRY(scratch(cs, "moe_xq", (size_t)S * H, &xq));
  RK_TRY(scratch(cs, "moe_xs", (size_t)S * KBh * 4, &xs));
  if (act_out)
    act = act_out;
  else
    RK_TRY(scratch(cs, "moe_act", (size_t)R * I * 4, &act));
  RK_TRY(scratch(cs, "moe_aq", (size_t)R * I, &aq));
  RK_TRY(scratch(cs, "moe_as", (size_t)R * KBi * 4, &as));
  RK_TRY(scratch(cs, "moe_yb", (size_t)R * H * 4, &yb));
  // One arrival counter per (token, 128-column slice) for the combine in the
  // down launch. Each launch leaves them at zero; a new buffer is zeroed once.
  const size_t cnt_bytes = (size_t)S * ((H + 127) / 128) * 4;
  bool fresh = false;
  RK_TRY(scratch(cs, "moe_cnt", cnt_bytes, &cnt, &fresh));
  const char *op = "rk_moe_experts_dev";
  if (fresh) HIP_TRY(hipMemsetAsync(cnt, 0, std::max<size_t>(cnt_bytes, 256), st), op);
  // x and the silu·up rows are quantized per row per 32-value group, as the
  // reference's expert workers do (engine.rs:1005-1006, 1034-1035).
  HIP_TRY(rk_launch_quantize_rows(x, S, H, 32, (int8_t *)xq, (float *)xs, st), op);
  HIP_TRY(rk_launch_moe_gemm_gu(plan.tile_rows, (const int8_t *)xq, (const float *)xs, (int)KBh, plan.tok, S,
                                plan.tiles_gu, plan.n_tiles, w.gu_codes, w.gu_scales,
                                moe_gu_code_stride(w), 2 * I * w.gu_ws_stride, w.gu_ws_stride,
                                (int)(2 * I), (int)H, (float *)act, st),
          op);
  if (!y) return RK_OK;  // stage 1 only
  HIP_TRY(rk_launch_quantize_rows((const float *)act, plan.rows, I, 32, (int8_t *)aq, (float *)as, st),
          op);
  MoeCombine cmb;
  cmb.tok = plan.tok;
  cmb.slot = plan.slot;
  cmb.cnt = (unsigned *)cnt;
  cmb.y = y;
  cmb.n_tok = (int)S;
  cmb.top_k = plan.top_k;
  cmb.accumulate = accumulate ? 1 : 0;
  HIP_TRY(rk_launch_moe_gemm_down(plan.tile_rows, (const int8_t *)aq, (const float *)as, (int)KBi, plan.rows,
                                  plan.tiles, plan.n_tiles, w.dn_codes, w.dn_scales,
                                  moe_dn_code_stride(w), H * w.dn_ws_stride, w.dn_ws_stride, (int)H,
                                  (int)I, plan.roww, (float *)yb, cmb, st),
          op);
  return RK_OK;
}

int plan_mark_used(const MoePlan &p, hipStream_t st) {
  auto it = std::find_if(p.uses.begin(), p.uses.end(), [&](const auto &u) { return u.first == st; });
  if (it == p.uses.end()) {
    p.uses.push_back({st, nullptr});
    it = p.uses.end() - 1;
  }
  if (own_stream(st)) return RK_OK;
  if (!it->second) HIP_TRY(hipEventCreateWithFlags(&it->second, hipEventDisableTiming), "rk_moe_plan");
  HIP_TRY(hipEventRecord(it->second, st), "rk_moe_plan");
  return RK_OK;
}

int moe_check(uint64_t id, int64_t s, int top_k, Weight **w, const char *op) {
  *w = find(id);
  if (!*w || !(*w)->moe) return fail(RK_E_SHAPE, op, "id is not an expert stack");
  if (s <= 0 || top_k <= 0 || top_k > (*w)->n_experts)
    return fail(RK_E_SHAPE, op, "need s > 0 and 0 < top_k <= n_experts");
  // The expert kernels address the int8 activations (x [s, hidden], the
  // quantized silu·up rows [s·top_k, inter]) with 32-bit byte offsets.
  if (s * (*w)->hidden >= ((int64_t)1 << 31) || s * top_k * (*w)->inter >= ((int64_t)1 << 31))
    return fail(RK_E_SHAPE, op, "s·hidden and s·top_k·inter must stay below 2^31");
  // The combine reads the per-slot f32 rows [s·top_k, hidden] the same way.
  if (s * top_k * (*w)->hidden * 4 >= ((int64_t)1 << 31))
    return fail(RK_E_SHAPE, op, "s·top_k·hidden f32 values must stay below 2^31 bytes");
  return RK_OK;
}
}  // namespace

namespace {
int moe_experts(rk_weight_id id, const float *x, int64_t s, int top_k, const uint32_t *ids,
                const float *wts, float *y, rk_stream stream, bool accumulate, const char *op) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure(op));
  Weight *w;
  RK_TRY(moe_check(id, s, top_k, &w, op));
  if (!x || !y || !ids || !wts) return fail(RK_E_SHAPE, op, "null buffer");
  hipStream_t st = pick(stream);
  CallScope cs(st);
  MoePlan *plan = new MoePlan();
  int rc = moe_plan(*w, s, top_k, ids, wts, plan, st);
  if (rc == RK_OK) rc = moe_run(cs, *w, *plan, x, y, nullptr, accumulate);
  // The plan's lists must outlive the kernels that read them.
  hipError_t e = hipStreamSynchronize(st);
  plan_free(plan);
  if (rc != RK_OK) return rc;
  HIP_TRY(e, op);
  g_eng->calls++;
  return RK_OK;
}

int moe_experts_planned(rk_weight_id id, const void *plan, const float *x, float *y, rk_stream stream,
                        bool accumulate, const char *op) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure(op));
  const MoePlan *p = (const MoePlan *)plan;
  if (!p) return fail(RK_E_SHAPE, op, "null plan");
  if (!x || !y) return fail(RK_E_SHAPE, op, "null buffer");
  Weight *w;
  RK_TRY(moe_check(id, p->s, p->top_k, &w, op));
  if (p->weight != id) return fail(RK_E_SHAPE, op, "plan was made for another expert stack");
  CallScope cs(pick(stream));
  RK_TRY(moe_run(cs, *w, *p, x, y, nullptr, accumulate));
  RK_TRY(plan_mark_used(*p, cs.st));
  g_eng->calls++;
  return RK_OK;
}
}  // namespace

extern "C" int rk_moe_experts_dev(rk_weight_id id, const float *x, int64_t s, int top_k,
                                  const uint32_t *ids, const float *wts, float *y,
                                  rk_stream stream) {
  return moe_experts(id, x, s, top_k, ids, wts, y, stream, false, "rk_moe_experts_dev");
}

extern "C" int rk_moe_experts_acc_dev(rk_weight_id id, const float *x, int64_t s, int top_k,
                                      const uint32_t *ids, const float *wts, float *y,
                                      rk_stream stream) {
  return moe_experts(id, x, s, top_k, ids, wts, y, stream, true, "rk_moe_experts_acc_dev");
}

extern "C" int rk_moe_plan_create(rk_weight_id id, int64_t s, int top_k, const uint32_t *ids,
                                  const float *wts, void **plan) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_moe_plan_create"));
  Weight *w;
  RK_TRY(moe_check(id, s, top_k, &w, "rk_moe_plan_create"));
  MoePlan *p = new MoePlan();
  const int rc = moe_plan(*w, s, top_k, ids, wts, p, g_eng->stream);
  if (rc != RK_OK) {
    plan_free(p);
    return rc;
  }
  p->weight = id;
  *plan = p;
  return RK_OK;
}

extern "C" int rk_moe_experts_planned_dev(rk_weight_id id, const void *plan, const float *x,
                                          float *y, rk_stream stream) {
  return moe_experts_planned(id, plan, x, y, stream, false, "rk_moe_experts_planned_dev");
}

extern "C" int rk_moe_experts_planned_acc_dev(rk_weight_id id, const void *plan, const float *x,
                                              float *y, rk_stream stream) {
  return moe_experts_planned(id, plan, x, y, stream, true, "rk_moe_experts_planned_acc_dev");
}

extern "C" int rk_moe_gate_up_dev(rk_weight_id id, const void *plan, const float *x, float *act,
                                  rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_moe_gate_up_dev"));
  const MoePlan *p = (const MoePlan *)plan;
  if (!p || !act) return fail(RK_E_SHAPE, "rk_moe_gate_up_dev", "null plan or output");
  Weight *w;
  RK_TRY(moe_check(id, p->s, p->top_k, &w, "rk_moe_gate_up_dev"));
  if (p->weight != id)
    return fail(RK_E_SHAPE, "rk_moe_gate_up_dev", "plan was made for another expert stack");
  CallScope cs(pick(stream));
  RK_TRY(moe_run(cs, *w, *p, x, nullptr, act));
  RK_TRY(plan_mark_used(*p, cs.st));
  return RK_OK;
}

extern "C" int rk_moe_plan_destroy(void *plan) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_moe_plan_destroy"));
  MoePlan *p = (MoePlan *)plan;
  // Runs on any stream that read the plan's lists must have finished (a
  // library stream destroyed since was synchronized then).
  if (p)
    for (auto &u : p->uses) {
      if (u.second) HIP_TRY(hipEventSynchronize(u.second), "rk_moe_plan_destroy");
      else if (own_stream(u.first)) HIP_TRY(hipStreamSynchronize(u.first), "rk_moe_plan_destroy");
    }
  HIP_TRY(hipStreamSynchronize(g_eng->stream), "rk_moe_plan_destroy");
  plan_free(p);
  return RK_OK;
}

// =========================================================================
// Device plumbing
// =========================================================================
extern "C" int rk_device_alloc(size_t bytes, void **ptr) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_device_alloc"));
  HIP_TRY(hipMalloc(ptr, std::max<size_t>(bytes, 1)), "rk_device_alloc");
  return RK_OK;
}
extern "C" int rk_device_free(void *ptr) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_device_free"));
  HIP_TRY(hipFree(ptr), "rk_device_free");
  return RK_OK;
}
extern "C" int rk_memcpy_htod(void *dst, const void *src, size_t bytes) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_memcpy_htod"));
  HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "rk_memcpy_htod");
  return RK_OK;
}
extern "C" int rk_memcpy_dtoh(void *dst, const void *src, size_t bytes) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_memcpy_dtoh"));
  HIP_TRY(hipStreamSynchronize(g_eng->stream), "rk_memcpy_dtoh");
  HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "rk_memcpy_dtoh");
  return RK_OK;
}
// =========================================================================
// MLP glue
// =========================================================================
namespace {
int glue_dev(int op, const void *a, const void *b, void *out, int64_t n, int dtype,
             rk_stream stream, const char *name) {
  RK_TRY(ensure(name));
  if (n < 0) return fail(RK_E_SHAPE, name, "negative element count");
  if (dtype < RK_DTYPE_F32 || dtype > RK_DTYPE_BF16) return fail(RK_E_SHAPE, name, "unknown dtype");
  if (n > 0 && (!a || !b || !out)) return fail(RK_E_SHAPE, name, "null buffer");
  HIP_TRY(rk_launch_glue(op, a, b, out, n, dtype, pick(stream)), name);
  return RK_OK;
}
int glue_host(int op, const float *a, const float *b, float *out, int64_t n, const char *name) {
  RK_TRY(ensure(name));
  if (n < 0) return fail(RK_E_SHAPE, name, "negative element count");
  if (n == 0) return RK_OK;
  if (!a || !b || !out) return fail(RK_E_SHAPE, name, "null buffer");
  hipStream_t st = g_eng->stream;
  CallScope cs(st);
  void *d = nullptr;
  RK_TRY(scratch(cs, "glue", (size_t)n * 12, &d));
  float *da = (float *)d, *db = da + n, *dout = db + n;
  auto compute = [&](int64_t r0, int64_t r1) {
    HIP_TRY(rk_launch_glue(op, da + r0, db + r0, dout + r0, r1 - r0, RK_DTYPE_F32, st), name);
    return RK_OK;
  };
  return staged(cs, {{a, nullptr, da, 4, 0}, {b, nullptr, db, 4, 0}}, {{nullptr, out, dout, 4, 0}}, n,
                stage_chunk_rows(n, 8, 4), compute, name);
}
}  // namespace

extern "C" int rk_silu_mul_dev(const void *a, const void *b, void *out, int64_t n, int dtype,
                               rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  return glue_dev(0, a, b, out, n, dtype, stream, "rk_silu_mul_dev");
}
extern "C" int rk_gelu_mul_dev(const void *a, const void *b, void *out, int64_t n, int dtype,
                               rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  return glue_dev(1, a, b, out, n, dtype, stream, "rk_gelu_mul_dev");
}
extern "C" int rk_silu_mul(const float *a, const float *b, float *out, int64_t n) {
  std::lock_guard<std::mutex> lk(g_mu);
  return glue_host(0, a, b, out, n, "rk_silu_mul");
}
extern "C" int rk_gelu_mul(const float *a, const float *b, float *out, int64_t n) {
  std::lock_guard<std::mutex> lk(g_mu);
  return glue_host(1, a, b, out, n, "rk_gelu_mul");
}

// =========================================================================
// RMSNorm and RoPE
// =========================================================================
namespace {
bool float_dtype(int dt) { return dt >= RK_DTYPE_F32 && dt <= RK_DTYPE_BF16; }
size_t dtype_bytes(int dt) { return dt == RK_DTYPE_F32 ? 4 : 2; }

int rms_check(const void *x, const void *out, int64_t rows, int64_t d, int dtype,
              const char *name) {
  if (rows < 0) return fail(RK_E_SHAPE, name, "negative row count");
  if (d <= 0 || d > INT32_MAX) return fail(RK_E_SHAPE, name, "the last dim must be in [1, 2^31)");
  if (!float_dtype(dtype)) return fail(RK_E_SHAPE, name, "unknown dtype");
  if (rows > 0 && (!x || !out)) return fail(RK_E_SHAPE, name, "null buffer");
  return RK_OK;
}
int rope_check(const void *x, const void *cs, const void *sn, const void *out, int64_t b,
               int64_t s, int64_t h, int64_t d, int dtype, int cs_dtype, const char *name) {
  if (b < 0 || s < 0 || h < 0 || d < 0) return fail(RK_E_SHAPE, name, "x must be [B, S, H, D]");
  if (d % 2 != 0) return fail(RK_E_SHAPE, name, "the head dim must be even");
  if (!float_dtype(dtype) || !float_dtype(cs_dtype)) return fail(RK_E_SHAPE, name, "unknown dtype");
  if (b * s * h > INT32_MAX || d > INT32_MAX)
    return fail(RK_E_SHAPE, name, "B·S·H and D must be below 2^31");
  if (b * s * h * d > 0 && (!x || !cs || !sn || !out)) return fail(RK_E_SHAPE, name, "null buffer");
  return RK_OK;
}
int rms_host(const float *x, const float *w, float *out, int64_t rows, int64_t d, double eps,
             const char *name) {
  RK_TRY(ensure(name));
  RK_TRY(rms_check(x, out, rows, d, RK_DTYPE_F32, name));
  if (rows == 0) return RK_OK;
  const size_t n = (size_t)(rows * d);
  hipStream_t st = g_eng->stream;
  CallScope cs(st);
  void *buf = nullptr;
  RK_TRY(scratch(cs, "norm", (n + (size_t)d) * 4, &buf));
  float *dx = (float *)buf, *dw = dx + n;
  std::vector<rkstage::Xfer> ins = {{x, nullptr, dx, (size_t)d * 4, 0}};
  if (w) ins.push_back({w, nullptr, dw, 0, (size_t)d * 4});
  auto compute = [&](int64_t r0, int64_t r1) {
    HIP_TRY(rk_launch_rms_norm(dx + r0 * d, w ? dw : nullptr, RK_DTYPE_F32, dx + r0 * d, r1 - r0, (int)d,
                               (float)eps, RK_DTYPE_F32, st),
            name);
    return RK_OK;
  };
  return staged(cs, ins, {{nullptr, out, dx, (size_t)d * 4, 0}}, rows,
                stage_chunk_rows(rows, (size_t)d * 4, (size_t)d * 4), compute, name);
}
}  // namespace

extern "C" int rk_rms_norm_dev(const void *x, const void *w, int w_dtype, void *out, int64_t rows,
                               int64_t d, double eps, int dtype, rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  const char *name = "rk_rms_norm_dev";
  RK_TRY(ensure(name));
  RK_TRY(rms_check(x, out, rows, d, dtype, name));
  if (!float_dtype(w_dtype)) return fail(RK_E_SHAPE, name, "unknown weight dtype");
  if (rows > 0 && !w) return fail(RK_E_SHAPE, name, "null weight");
  HIP_TRY(rk_launch_rms_norm(x, w, w_dtype, out, rows, (int)d, (float)eps, dtype, pick(stream)),
          name);
  return RK_OK;
}
extern "C" int rk_rms_norm_noscale_dev(const void *x, void *out, int64_t rows, int64_t d,
                                       double eps, int dtype, rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  const char *name = "rk_rms_norm_noscale_dev";
  RK_TRY(ensure(name));
  RK_TRY(rms_check(x, out, rows, d, dtype, name));
  HIP_TRY(rk_launch_rms_norm(x, nullptr, RK_DTYPE_F32, out, rows, (int)d, (float)eps, dtype,
                             pick(stream)), name);
  return RK_OK;
}
extern "C" int rk_rope_dev(const void *x, const void *cos, const void *sin, int cs_dtype, void *out,
                           int64_t b, int64_t s, int64_t h, int64_t d, int dtype,
                           rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  const char *name = "rk_rope_dev";
  RK_TRY(ensure(name));
  RK_TRY(rope_check(x, cos, sin, out, b, s, h, d, dtype, cs_dtype, name));
  HIP_TRY(rk_launch_rope(x, cos, sin, cs_dtype, out, (int)(b * s * h), (int)s, (int)h, (int)(d / 2),
                         dtype, pick(stream)), name);
  return RK_OK;
}
extern "C" int rk_qk_norm_rope_dev(void *qkv, int64_t s, int64_t row_stride, int n_q_heads,
                                   int n_kv_heads, int64_t head_dim, const void *q_norm_w,
                                   const void *k_norm_w, double eps, const void *cos,
                                   const void *sin, int cs_dtype, int dtype, rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  const char *name = "rk_qk_norm_rope_dev";
  RK_TRY(ensure(name));
  if (s < 0 || n_q_heads < 0 || n_kv_heads < 0 || s * (n_q_heads + n_kv_heads) > INT32_MAX)
    return fail(RK_E_SHAPE, name, "negative shape, or s·(q + k heads) of 2^31 or more");
  if (head_dim <= 0 || head_dim % 2 != 0 || head_dim > 4096)
    return fail(RK_E_SHAPE, name, "the head dim must be even and in [2, 4096]");
  if (row_stride < (int64_t)(n_q_heads + n_kv_heads) * head_dim)
    return fail(RK_E_SHAPE, name, "row_stride is shorter than the q and k heads");
  if (!float_dtype(dtype) || !float_dtype(cs_dtype)) return fail(RK_E_SHAPE, name, "unknown dtype");
  if (cs_dtype != dtype && cs_dtype != RK_DTYPE_F32)
    return fail(RK_E_UNSUPPORTED, name, "cos/sin must have the element type of qkv or be f32");
  if ((q_norm_w == nullptr) != (k_norm_w == nullptr))
    return fail(RK_E_SHAPE, name, "give both norm weights or neither");
  if (s == 0 || n_q_heads + n_kv_heads == 0) return RK_OK;
  if (!qkv || !cos || !sin) return fail(RK_E_SHAPE, name, "null buffer");
  if (rk_qk_norm_rope_cv(qkv, row_stride, (int)head_dim, dtype, q_norm_w, k_norm_w, cos, sin,
                         cs_dtype) == 0)
    return fail(RK_E_UNSUPPORTED, name,
                "head_dim / row_stride / buffer alignment allow no vector width (head_dim over 64 values per lane?)");
  HIP_TRY(rk_launch_qk_norm_rope(qkv, row_stride, (int)s, n_q_heads, n_kv_heads, (int)head_dim,
                                 q_norm_w, k_norm_w, (float)eps, cos, sin, cs_dtype, dtype,
                                 pick(stream)), name);
  return RK_OK;
}
extern "C" int rk_attention_qkv_dev(void *qkv, int64_t s, int64_t row_stride, int n_head,
                                    int n_kv_heads, int head_dim, const void *q_norm_w,
                                    const void *k_norm_w, double eps, const void *cos,
                                    const void *sin, int cs_dtype, float scale, float softcap,
                                    int mask_mode, int64_t window, int64_t q0, int64_t k0,
                                    void *out, int64_t out_stride, rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  const char *name = "rk_attention_qkv_dev";
  RK_TRY(ensure(name));
  int mode = mask_mode;
  RK_TRY(attn_check(s, s, n_head, n_kv_heads, head_dim, &mode, window, name));
  if (s * (n_head + n_kv_heads) > INT32_MAX)
    return fail(RK_E_SHAPE, name, "s·(q + k heads) of 2^31 or more");
  const int64_t width = (int64_t)(n_head + 2 * n_kv_heads) * head_dim;
  if (row_stride < width || out_stride < (int64_t)n_head * head_dim)
    return fail(RK_E_SHAPE, name, "a row stride is shorter than its heads");
  if ((row_stride | out_stride) % 8 != 0 || (((uintptr_t)qkv | (uintptr_t)out) & 15) != 0)
    return fail(RK_E_SHAPE, name, "row strides must be multiples of 8 values, buffers 16-byte aligned");
  if (cs_dtype != RK_DTYPE_F16 && cs_dtype != RK_DTYPE_F32)
    return fail(RK_E_UNSUPPORTED, name, "cos/sin must be fp16 or f32");
  if ((q_norm_w == nullptr) != (k_norm_w == nullptr))
    return fail(RK_E_SHAPE, name, "give both norm weights or neither");
  if (head_dim % 2 != 0) return fail(RK_E_SHAPE, name, "the head dim must be even");
  if (s == 0) return RK_OK;
  if (!qkv || !cos || !sin || !out) return fail(RK_E_SHAPE, name, "null buffer");
  if (rk_qk_norm_rope_cv(qkv, row_stride, head_dim, RK_DTYPE_F16, q_norm_w, k_norm_w, cos, sin,
                         cs_dtype) == 0)
    return fail(RK_E_UNSUPPORTED, name, "head_dim / row_stride / buffer alignment allow no vector width");
  hipStream_t st = pick(stream);
  CallScope cs(st);
  const int dvp = rk_attn_dv_pad(head_dim);
  const int64_t n_kv_pad = round_up_i(s, rk_attn_kv_tile());
  void *vt;
  RK_TRY(scratch(cs, "attn_vt", (size_t)n_kv_heads * dvp * n_kv_pad * 2, &vt));
  HIP_TRY(rk_launch_qk_norm_rope(qkv, row_stride, (int)s, n_head, n_kv_heads, head_dim, q_norm_w,
                                 k_norm_w, (float)eps, cos, sin, cs_dtype, RK_DTYPE_F16, st, vt,
                                 (int)n_kv_pad, dvp), name);
  RK_TRY(attn_run(qkv, (const uint16_t *)qkv + (int64_t)n_head * head_dim, vt, out, s, s, n_kv_pad,
                  n_head, n_kv_heads, head_dim, scale, softcap, mode, window, q0, k0, false, st,
                  name, &cs, row_stride, row_stride, out_stride));
  g_eng->calls++;
  return RK_OK;
}
extern "C" int rk_rms_norm_quantize_dev(const void *x, const void *w, int w_dtype, int64_t rows,
                                        int64_t d, double eps, int dtype, int8_t *q,
                                        float *q_scale, rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  const char *name = "rk_rms_norm_quantize_dev";
  RK_TRY(ensure(name));
  RK_TRY(rms_check(x, q, rows, d, dtype, name));
  if (w && !float_dtype(w_dtype)) return fail(RK_E_SHAPE, name, "unknown weight dtype");
  if (rows > 0 && !q_scale) return fail(RK_E_SHAPE, name, "null scale buffer");
  if (!rk_rms_quant_fits(x, w, w_dtype, q, (int)d, dtype))
    return fail(RK_E_UNSUPPORTED, name,
                "needs d a multiple of 16 bytes of x and at most 8 KB per row, the weight in x's "
                "type, 16-byte aligned x and w (use rk_rms_norm_dev + rk_quantize_rows_dev)");
  HIP_TRY(rk_launch_rms_quant(x, w, q, q_scale, rows, (int)d, (float)eps, dtype, pick(stream)),
          name);
  return RK_OK;
}
extern "C" int rk_rms_norm(const float *x, const float *w, float *out, int64_t rows, int64_t d,
                           double eps) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (rows > 0 && !w) return fail(RK_E_SHAPE, "rk_rms_norm", "null weight");
  return rms_host(x, w, out, rows, d, eps, "rk_rms_norm");
}
extern "C" int rk_rms_norm_noscale(const float *x, float *out, int64_t rows, int64_t d,
                                   double eps) {
  std::lock_guard<std::mutex> lk(g_mu);
  return rms_host(x, nullptr, out, rows, d, eps, "rk_rms_norm_noscale");
}
extern "C" int rk_rope(const float *x, const float *cos, const float *sin, float *out, int64_t b,
                       int64_t s, int64_t h, int64_t d) {
  std::lock_guard<std::mutex> lk(g_mu);
  const char *name = "rk_rope";
  RK_TRY(ensure(name));
  RK_TRY(rope_check(x, cos, sin, out, b, s, h, d, RK_DTYPE_F32, RK_DTYPE_F32, name));
  const size_t n = (size_t)(b * s * h * d), nt = (size_t)(s * (d / 2));
  if (n == 0) return RK_OK;
  hipStream_t st = g_eng->stream;
  CallScope cs(st);
  void *buf = nullptr;
  RK_TRY(scratch(cs, "rope", (n + 2 * nt) * 4, &buf));
  float *dx = (float *)buf, *dc = dx + n, *ds = dc + nt;
  auto compute = [&](int64_t, int64_t) {
    HIP_TRY(rk_launch_rope(dx, dc, ds, RK_DTYPE_F32, dx, (int)(b * s * h), (int)s, (int)h, (int)(d / 2),
                           RK_DTYPE_F32, st),
            name);
    return RK_OK;
  };
  return staged(cs, {{x, nullptr, dx, 0, n * 4}, {cos, nullptr, dc, 0, nt * 4}, {sin, nullptr, ds, 0, nt * 4}},
                {{nullptr, out, dx, 0, n * 4}}, 1, 1, compute, name);
}

extern "C" int rk_memcpy_dtod(void *dst, const void *src, size_t bytes, rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_memcpy_dtod"));
  HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice,
                         stream ? (hipStream_t)stream : g_eng->stream),
          "rk_memcpy_dtod");
  return RK_OK;
}
extern "C" int rk_cast_dev(const void *x, int x_dtype, void *y, int y_dtype, int64_t n,
                           rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  const char *op = "rk_cast_dev";
  RK_TRY(ensure(op));
  if (n < 0) return fail(RK_E_SHAPE, op, "negative element count");
  if (x_dtype < RK_DTYPE_F32 || x_dtype > RK_DTYPE_BF16 || y_dtype < RK_DTYPE_F32 ||
      y_dtype > RK_DTYPE_BF16)
    return fail(RK_E_SHAPE, op, "unknown dtype");
  if (n > 0 && (!x || !y)) return fail(RK_E_SHAPE, op, "null buffer");
  HIP_TRY(rk_launch_cast(x, x_dtype, y, y_dtype, n, pick(stream)), op);
  return RK_OK;
}
extern "C" int rk_memset_dev(void *dst, int value, size_t bytes) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_memset_dev"));
  HIP_TRY(hipMemset(dst, value, bytes), "rk_memset_dev");
  return RK_OK;
}
extern "C" int rk_stream_get(rk_stream *stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_stream_get"));
  *stream = (rk_stream)g_eng->stream;
  return RK_OK;
}
extern "C" int rk_stream_create(rk_stream *stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_stream_create"));
  if (!stream) return fail(RK_E_SHAPE, "rk_stream_create", "null output");
  hipStream_t st = nullptr;
  HIP_TRY(hipStreamCreateWithFlags(&st, hipStreamNonBlocking), "rk_stream_create");
  g_eng->own_streams.insert(st);
  *stream = (rk_stream)st;
  return RK_OK;
}
extern "C" int rk_stream_destroy(rk_stream stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_stream_destroy"));
  hipStream_t st = (hipStream_t)stream;
  if (!stream || st == g_eng->stream || !g_eng->own_streams.count(st))
    return fail(RK_E_SHAPE, "rk_stream_destroy", "not a stream made by rk_stream_create");
  // The stream's work completes first: buffers and MoE plans last used there
  // then need no further fence.
  HIP_TRY(hipStreamSynchronize(st), "rk_stream_destroy");
  for (auto &kv : g_eng->scratch)
    if (kv.second.ev_stream == st) kv.second.pending = kv.second.recorded = false;
  HIP_TRY(hipStreamDestroy(st), "rk_stream_destroy");
  g_eng->own_streams.erase(st);
  return RK_OK;
}
extern "C" int rk_stream_sync(rk_stream stream) {
  RK_TRY(ensure("rk_stream_sync"));
  HIP_TRY(hipStreamSynchronize(stream ? (hipStream_t)stream : g_eng->stream), "rk_stream_sync");
  return RK_OK;
}
extern "C" int rk_event_create(void **event) {
  RK_TRY(ensure("rk_event_create"));
  HIP_TRY(hipEventCreate((hipEvent_t *)event), "rk_event_create");
  return RK_OK;
}
extern "C" int rk_event_destroy(void *event) {
  HIP_TRY(hipEventDestroy((hipEvent_t)event), "rk_event_destroy");
  return RK_OK;
}
extern "C" int rk_event_record(void *event, rk_stream stream) {
  RK_TRY(ensure("rk_event_record"));
  HIP_TRY(hipEventRecord((hipEvent_t)event, stream ? (hipStream_t)stream : g_eng->stream),
          "rk_event_record");
  return RK_OK;
}
extern "C" int rk_event_elapsed_ms(void *start, void *stop, float *ms) {
  HIP_TRY(hipEventSynchronize((hipEvent_t)stop), "rk_event_elapsed_ms");
  HIP_TRY(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop), "rk_event_elapsed_ms");
  return RK_OK;
}
extern "C" int rk_device_info(char *name, size_t name_len, int *cus, int *clock_khz) {
  std::lock_guard<std::mutex> lk(g_mu);
  RK_TRY(ensure("rk_device_info"));
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, g_eng->device), "rk_device_info");
  if (name && name_len) {
    std::snprintf(name, name_len, "%s (%s)", prop.name, prop.gcnArchName);
  }
  if (cus) *cus = prop.multiProcessorCount;
  if (clock_khz) *clock_khz = prop.clockRate;
  return RK_OK;
}
