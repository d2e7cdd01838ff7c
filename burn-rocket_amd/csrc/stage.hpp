// Pinned host staging for the host-buffer entry points (rk_matmul, rk_attention, ...).
//
// The reference hands every op host tensors (`into_data`, ext.rs:759-779), so
// each host-buffer call crosses PCIe twice. Copies from pageable memory run at
// the runtime's bounce-buffer rate (17-28 GB/s measured on MI355X hosts);
// copies from page-locked memory run at the link rate (57 GB/s each way, 48 GB/s
// each way when both directions run). HostStage moves data through a ring of
// page-locked slots allocated with hipHostMalloc: a pool of CPU threads copies
// between the caller's pageable buffer and a slot while the DMA engines move
// other slots, and row-separable ops run chunk by chunk so that the upload of
// chunk j+1, the kernels of chunk j and the download of chunk j-1 overlap on
// three streams (uploads, kernels, downloads; all at the default priority).
#pragma once
#include <hip/hip_runtime.h>

#include <atomic>
#include <condition_variable>
#include <cstddef>
#include <cstdint>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

namespace rkstage {

// memcpy split over a few threads. The workers spin while a session is open
// (a host-buffer call is in flight) and sleep on a condition variable
// otherwise.
class CopyPool {
 public:
  explicit CopyPool(int threads);
  ~CopyPool();
  CopyPool(const CopyPool &) = delete;
  CopyPool &operator=(const CopyPool &) = delete;
  void copy(void *dst, const void *src, size_t bytes);
  void begin();
  void end();
  int threads() const { return n_; }

 private:
  void worker(int idx);
  void slice(int idx, int parts);
  int n_;  // slices per copy, the calling thread included
  std::vector<std::thread> th_;
  std::mutex mu_;
  std::condition_variable cv_;
  std::atomic<uint64_t> gen_{0};
  std::atomic<int> left_{0};
  std::atomic<bool> active_{false}, stop_{false};
  char *dst_ = nullptr;
  const char *src_ = nullptr;
  size_t bytes_ = 0;
};

// One transfer of a staged call. Row-sliced transfers move `row_bytes` per
// row of the chunk being processed (host and device offsets r0·row_bytes);
// whole transfers (row_bytes == 0) move `bytes` once, inputs before the first
// chunk and outputs after the last.
struct Xfer {
  const void *host_src = nullptr;  // inputs
  void *host_dst = nullptr;        // outputs
  void *dev = nullptr;
  size_t row_bytes = 0;
  size_t bytes = 0;
};

class HostStage {
 public:
  // compute(r0, r1) enqueues the kernels of rows [r0, r1) on the kernel stream
  // and returns false on failure (the caller keeps the reason).
  using Compute = std::function<bool(int64_t r0, int64_t r1)>;

  ~HostStage();
  // Streams, events, slots and copy threads; idempotent.
  hipError_t setup(int device);
  // Runs the inputs, `rows` rows in chunks of `chunk_rows` through compute,
  // and the outputs; returns when every output is in host memory. `st` is the
  // kernel stream. *compute_ok is false when compute failed (nothing more was
  // enqueued after it; the work already enqueued is waited for).
  hipError_t run(hipStream_t st, const std::vector<Xfer> &ins, const std::vector<Xfer> &outs,
                 int64_t rows, int64_t chunk_rows, const Compute &compute, bool *compute_ok,
                 float *kernel_ms);
  size_t pinned_bytes() const;
  // Frees the page-locked slots (they are allocated again on the next call).
  hipError_t release();

  static constexpr size_t kSlotBytes = 4u << 20;
  static constexpr int kSlots = 4;  // per direction
  static constexpr int kMaxChunks = 16;

 private:
  struct Slot {
    void *p = nullptr;
    hipEvent_t ev = nullptr;
    bool busy = false;     // a DMA from / into it is enqueued
    void *drain_to = nullptr;  // output slot: host destination of its contents
    size_t len = 0;
  };
  hipError_t alloc_slots();
  hipError_t wait_slot(Slot &s, bool drain);
  hipError_t put(const char *src, char *dev, size_t len);   // one input piece
  hipError_t get(char *dst, const char *dev, size_t len);   // one output piece
  hipError_t drain_all();

  bool ready_ = false;
  hipStream_t in_st_ = nullptr, out_st_ = nullptr;
  hipEvent_t ev_start_ = nullptr;
  hipEvent_t ev_in_[kMaxChunks] = {}, ev_done_[kMaxChunks] = {}, ev_k0_[kMaxChunks] = {};
  Slot in_[kSlots], out_[kSlots];
  int in_next_ = 0, out_next_ = 0;
  CopyPool *pool_ = nullptr;
};

}  // namespace rkstage
