// Pinned host staging: a ring of page-locked slots per direction, a small
// memcpy thread pool and three streams (see stage.hpp).
#include "stage.hpp"

#include <algorithm>
#include <cstring>

namespace rkstage {

// ---------------------------------------------------------------- CopyPool --
CopyPool::CopyPool(int threads) : n_(std::max(1, threads)) {
  for (int i = 1; i < n_; ++i) th_.emplace_back(&CopyPool::worker, this, i);
}

CopyPool::~CopyPool() {
  {
    std::lock_guard<std::mutex> lk(mu_);
    stop_.store(true);
  }
  cv_.notify_all();
  for (auto &t : th_) t.join();
}

// Slice idx of parts of the current copy, in 64-byte multiples.
void CopyPool::slice(int idx, int parts) {
  const size_t per = (bytes_ / parts + 63) & ~(size_t)63;
  const size_t b = per * idx;
  if (b >= bytes_) return;
  std::memcpy(dst_ + b, src_ + b, std::min(bytes_, b + per) - b);
}

void CopyPool::worker(int idx) {
  uint64_t seen = 0;
  for (;;) {
    uint64_t g;
    for (;;) {
      g = gen_.load(std::memory_order_acquire);
      if (g != seen || stop_.load()) break;
      if (!active_.load(std::memory_order_relaxed)) {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return gen_.load() != seen || stop_.load() || active_.load(); });
      } else {
        __builtin_ia32_pause();
      }
    }
    if (stop_.load()) return;
    seen = g;
    slice(idx, n_);
    left_.fetch_sub(1, std::memory_order_acq_rel);
  }
}

void CopyPool::copy(void *dst, const void *src, size_t bytes) {
  if (n_ == 1 || bytes < ((size_t)512 << 10)) {
    std::memcpy(dst, src, bytes);
    return;
  }
  dst_ = (char *)dst;
  src_ = (const char *)src;
  bytes_ = bytes;
  left_.store(n_ - 1, std::memory_order_relaxed);
  gen_.fetch_add(1, std::memory_order_acq_rel);  // publishes the three fields above
  if (!active_.load()) {
    std::lock_guard<std::mutex> lk(mu_);
    cv_.notify_all();
  }
  slice(0, n_);
  // Every worker finishes its slice of this copy before the next one starts.
  while (left_.load(std::memory_order_acquire) != 0) __builtin_ia32_pause();
}

void CopyPool::begin() {
  {
    std::lock_guard<std::mutex> lk(mu_);
    active_.store(true);
  }
  cv_.notify_all();
}

void CopyPool::end() { active_.store(false); }

// --------------------------------------------------------------- HostStage --
#define ST_TRY(expr)                  \
  do {                                \
    hipError_t e_ = (expr);           \
    if (e_ != hipSuccess) return e_;  \
  } while (0)

HostStage::~HostStage() { delete pool_; }

hipError_t HostStage::setup(int device) {
  (void)device;
  if (ready_) return hipSuccess;
  ST_TRY(hipStreamCreateWithFlags(&in_st_, hipStreamNonBlocking));
  ST_TRY(hipStreamCreateWithFlags(&out_st_, hipStreamNonBlocking));
  ST_TRY(hipEventCreateWithFlags(&ev_start_, hipEventDisableTiming));
  for (int j = 0; j < kMaxChunks; ++j) {
    ST_TRY(hipEventCreateWithFlags(&ev_in_[j], hipEventDisableTiming));
    ST_TRY(hipEventCreate(&ev_k0_[j]));
    ST_TRY(hipEventCreate(&ev_done_[j]));
  }
  for (Slot *ring : {in_, out_})
    for (int i = 0; i < kSlots; ++i) ST_TRY(hipEventCreateWithFlags(&ring[i].ev, hipEventDisableTiming));
  const unsigned hw = std::thread::hardware_concurrency();
  pool_ = new CopyPool((int)std::min(8u, std::max(1u, hw / 2)));
  ready_ = true;
  return hipSuccess;
}

hipError_t HostStage::alloc_slots() {
  for (Slot *ring : {in_, out_})
    for (int i = 0; i < kSlots; ++i)
      if (!ring[i].p) ST_TRY(hipHostMalloc(&ring[i].p, kSlotBytes, hipHostMallocDefault));
  return hipSuccess;
}

size_t HostStage::pinned_bytes() const {
  size_t b = 0;
  for (const Slot *ring : {in_, out_})
    for (int i = 0; i < kSlots; ++i) b += ring[i].p ? kSlotBytes : 0;
  return b;
}

// Waits for the slot's DMA; an output slot's contents then go to their host
// destination.
hipError_t HostStage::wait_slot(Slot &s, bool drain) {
  if (!s.busy) return hipSuccess;
  ST_TRY(hipEventSynchronize(s.ev));
  if (drain && s.drain_to) pool_->copy(s.drain_to, s.p, s.len);
  s.busy = false;
  s.drain_to = nullptr;
  return hipSuccess;
}

hipError_t HostStage::put(const char *src, char *dev, size_t len) {
  Slot &s = in_[in_next_];
  in_next_ = (in_next_ + 1) % kSlots;
  ST_TRY(wait_slot(s, false));
  pool_->copy(s.p, src, len);
  ST_TRY(hipMemcpyAsync(dev, s.p, len, hipMemcpyHostToDevice, in_st_));
  ST_TRY(hipEventRecord(s.ev, in_st_));
  s.busy = true;
  return hipSuccess;
}

hipError_t HostStage::get(char *dst, const char *dev, size_t len) {
  Slot &s = out_[out_next_];
  out_next_ = (out_next_ + 1) % kSlots;
  ST_TRY(wait_slot(s, true));
  ST_TRY(hipMemcpyAsync(s.p, dev, len, hipMemcpyDeviceToHost, out_st_));
  ST_TRY(hipEventRecord(s.ev, out_st_));
  s.busy = true;
  s.drain_to = dst;
  s.len = len;
  return hipSuccess;
}

hipError_t HostStage::drain_all() {
  for (int i = 0; i < kSlots; ++i) ST_TRY(wait_slot(out_[(out_next_ + i) % kSlots], true));
  for (int i = 0; i < kSlots; ++i) ST_TRY(wait_slot(in_[i], false));
  return hipSuccess;
}

hipError_t HostStage::run(hipStream_t st, const std::vector<Xfer> &ins,
                          const std::vector<Xfer> &outs, int64_t rows, int64_t chunk_rows,
                          const Compute &compute, bool *compute_ok, float *kernel_ms) {
  *compute_ok = true;
  *kernel_ms = 0.f;
  if (rows < 1 || chunk_rows < 1 || (rows + chunk_rows - 1) / chunk_rows > kMaxChunks)
    return hipErrorInvalidValue;
  ST_TRY(alloc_slots());
  pool_->begin();
  int chunks_run = 0;
  auto body = [&]() -> hipError_t {
    auto put_all = [&](const void *src, void *dev, size_t n) -> hipError_t {
      for (size_t off = 0; off < n; off += kSlotBytes)
        ST_TRY(put((const char *)src + off, (char *)dev + off, std::min(kSlotBytes, n - off)));
      return hipSuccess;
    };
    auto get_all = [&](void *dst, const void *dev, size_t n) -> hipError_t {
      for (size_t off = 0; off < n; off += kSlotBytes)
        ST_TRY(get((char *)dst + off, (const char *)dev + off, std::min(kSlotBytes, n - off)));
      return hipSuccess;
    };
    // Uploads overwrite device buffers that earlier kernels on st may still read.
    ST_TRY(hipEventRecord(ev_start_, st));
    ST_TRY(hipStreamWaitEvent(in_st_, ev_start_, 0));
    for (const Xfer &x : ins)
      if (!x.row_bytes) ST_TRY(put_all(x.host_src, x.dev, x.bytes));
    const int64_t nchunks = (rows + chunk_rows - 1) / chunk_rows;
    for (int64_t j = 0; j < nchunks; ++j) {
      const int64_t r0 = j * chunk_rows, r1 = std::min(rows, r0 + chunk_rows);
      for (const Xfer &x : ins)
        if (x.row_bytes)
          ST_TRY(put_all((const char *)x.host_src + r0 * x.row_bytes, (char *)x.dev + r0 * x.row_bytes,
                         (size_t)(r1 - r0) * x.row_bytes));
      ST_TRY(hipEventRecord(ev_in_[j], in_st_));
      ST_TRY(hipStreamWaitEvent(st, ev_in_[j], 0));
      ST_TRY(hipEventRecord(ev_k0_[j], st));
      if (!compute(r0, r1)) {
        *compute_ok = false;
        return hipSuccess;
      }
      ST_TRY(hipEventRecord(ev_done_[j], st));
      ++chunks_run;
      ST_TRY(hipStreamWaitEvent(out_st_, ev_done_[j], 0));
      // The downloads of chunk j start when its kernels end; queueing them
      // drains the slots of chunk j-1, whose DMA ran during this upload.
      for (const Xfer &x : outs)
        if (x.row_bytes)
          ST_TRY(get_all((char *)x.host_dst + r0 * x.row_bytes, (const char *)x.dev + r0 * x.row_bytes,
                         (size_t)(r1 - r0) * x.row_bytes));
    }
    for (const Xfer &x : outs)
      if (!x.row_bytes) ST_TRY(get_all(x.host_dst, x.dev, x.bytes));
    return drain_all();
  };
  hipError_t err = body();
  pool_->end();
  // Nothing the call enqueued may still run when it returns: its slots, the
  // caller's buffers and the scratch are reused by the next call.
  hipError_t e1 = hipStreamSynchronize(in_st_);
  hipError_t e2 = hipStreamSynchronize(st);
  hipError_t e3 = hipStreamSynchronize(out_st_);
  for (Slot *ring : {in_, out_})
    for (int i = 0; i < kSlots; ++i) {
      ring[i].busy = false;
      ring[i].drain_to = nullptr;
    }
  if (err == hipSuccess) err = e1 != hipSuccess ? e1 : (e2 != hipSuccess ? e2 : e3);
  if (err == hipSuccess)
    for (int j = 0; j < chunks_run; ++j) {
      float ms = 0.f;
      if (hipEventElapsedTime(&ms, ev_k0_[j], ev_done_[j]) == hipSuccess) *kernel_ms += ms;
    }
  return err;
}

hipError_t HostStage::release() {
  if (!ready_) return hipSuccess;
  ST_TRY(hipStreamSynchronize(in_st_));
  ST_TRY(hipStreamSynchronize(out_st_));
  for (Slot *ring : {in_, out_})
    for (int i = 0; i < kSlots; ++i)
      if (ring[i].p) {
        ST_TRY(hipHostFree(ring[i].p));
        ring[i].p = nullptr;
        ring[i].busy = false;
      }
  return hipSuccess;
}

}  // namespace rkstage
