// hostcopy.cpp — pinned staging ring and host copy threads for run() I/O.
#include "hostcopy.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <condition_variable>
#include <cstring>
#include <deque>
#include <mutex>
#include <thread>

namespace rgnpu {

namespace {

// Countdown shared by the pieces of one parallel_memcpy.
struct Latch {
  std::mutex m;
  std::condition_variable cv;
  int left = 0;
  void done() {
    std::lock_guard<std::mutex> lk(m);
    if (--left == 0) cv.notify_all();
  }
  void wait() {
    std::unique_lock<std::mutex> lk(m);
    cv.wait(lk, [&] { return left == 0; });
  }
};

// Process-wide memcpy threads.  Created on first use and never destroyed
// (they sleep on the queue until the process ends), so no program handle
// owns them and concurrent runs on any handle share them.
class CopyThreads {
 public:
  static CopyThreads& get() {
    static CopyThreads* inst = new CopyThreads();
    return *inst;
  }
  int threads() const { return n_; }
  void push(char* d, const char* s, size_t n, Latch* l) {
    {
      std::lock_guard<std::mutex> lk(mu_);
      q_.push_back(Task{d, s, n, l});
    }
    cv_.notify_one();
  }

 private:
  struct Task {
    char* d;
    const char* s;
    size_t n;
    Latch* l;
  };
  CopyThreads() {
    // Four pieces per copy outrun one DMA direction (about 25 GB/s per
    // thread against about 57 GB/s per direction on MI355X hosts); eight
    // threads leave room for several runs copying at once.
    const unsigned hw = std::thread::hardware_concurrency();
    n_ = (int)std::min(8u, hw > 1 ? hw / 2 : 1u);
    for (int i = 0; i < n_; i++) std::thread([this] { loop(); }).detach();
  }
  void loop() {
    for (;;) {
      Task t;
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return !q_.empty(); });
        t = q_.front();
        q_.pop_front();
      }
      std::memcpy(t.d, t.s, t.n);
      t.l->done();
    }
  }
  std::mutex mu_;
  std::condition_variable cv_;
  std::deque<Task> q_;
  int n_ = 0;
};

constexpr size_t kPieceAlign = size_t(64) << 10;
constexpr int kPieces = 4;

}  // namespace

void parallel_memcpy(void* dst, const void* src, size_t n) {
  CopyThreads& ct = CopyThreads::get();
  const int pieces = std::min(kPieces, ct.threads() + 1);
  if (n < 2 * kPieceAlign || pieces <= 1) {
    std::memcpy(dst, src, n);
    return;
  }
  const size_t per = (n / pieces + kPieceAlign - 1) / kPieceAlign * kPieceAlign;
  char* d = static_cast<char*>(dst);
  const char* s = static_cast<const char*>(src);
  Latch latch;
  int pushed = 0;
  for (size_t off = per; off < n; off += per) pushed++;
  latch.left = pushed;
  for (size_t off = per; off < n; off += per) ct.push(d + off, s + off, std::min(per, n - off), &latch);
  std::memcpy(d, s, std::min(per, n));  // the caller's own piece
  if (pushed) latch.wait();
}

Staging::~Staging() {
  for (auto& e : ev)
    if (e) (void)hipEventDestroy(e);
  if (pinned) (void)hipHostFree(pinned);
}

hipError_t Staging::ensure() {
  if (pinned) return hipSuccess;
  for (auto& e : ev) {
    if (e) continue;
    hipError_t r = hipEventCreateWithFlags(&e, hipEventDisableTiming);
    if (r != hipSuccess) return r;
  }
  return hipHostMalloc(reinterpret_cast<void**>(&pinned), kSlots * kSlotBytes, hipHostMallocDefault);
}

static size_t chunk_bytes(size_t n) {
  const size_t q = (n / 4 + kPieceAlign - 1) / kPieceAlign * kPieceAlign;
  return std::min(Staging::kSlotBytes, std::max(kStageMinBytes, q));
}

#define RG_TRY(expr)                 \
  do {                               \
    hipError_t e_ = (expr);          \
    if (e_ != hipSuccess) return e_; \
  } while (0)

hipError_t copy_to_device(Staging& st, void* dst_dev, const void* src_host, size_t n, hipStream_t s) {
  if (n < kStageMinBytes) return hipMemcpyAsync(dst_dev, src_host, n, hipMemcpyHostToDevice, s);
  RG_TRY(st.ensure());
  const size_t C = chunk_bytes(n);
  const size_t chunks = (n + C - 1) / C;
  for (size_t i = 0; i < chunks; i++) {
    const int r = (int)(i % Staging::kSlots);
    char* slot = st.pinned + (size_t)r * Staging::kSlotBytes;
    const size_t m = std::min(C, n - i * C);
    // the slot's previous DMA (chunk i - kSlots) must have read it
    if (i >= (size_t)Staging::kSlots) RG_TRY(hipEventSynchronize(st.ev[r]));
    parallel_memcpy(slot, static_cast<const char*>(src_host) + i * C, m);
    RG_TRY(hipMemcpyAsync(static_cast<char*>(dst_dev) + i * C, slot, m, hipMemcpyHostToDevice, s));
    RG_TRY(hipEventRecord(st.ev[r], s));
  }
  return hipSuccess;
}

hipError_t copy_to_host(Staging& st, void* dst_host, const void* src_dev, size_t n, hipStream_t s) {
  if (n < kStageMinBytes) {
    RG_TRY(hipMemcpyAsync(dst_host, src_dev, n, hipMemcpyDeviceToHost, s));
    return hipStreamSynchronize(s);
  }
  RG_TRY(st.ensure());
  const size_t C = chunk_bytes(n);
  const size_t chunks = (n + C - 1) / C;
  auto issue = [&](size_t i) -> hipError_t {
    const int r = (int)(i % Staging::kSlots);
    // stream order puts this DMA after every earlier use of the slot on s;
    // the host finished reading the slot's previous chunk before issuing it
    RG_TRY(hipMemcpyAsync(st.pinned + (size_t)r * Staging::kSlotBytes, static_cast<const char*>(src_dev) + i * C,
                          std::min(C, n - i * C), hipMemcpyDeviceToHost, s));
    return hipEventRecord(st.ev[r], s);
  };
  for (size_t i = 0; i < std::min(chunks, (size_t)Staging::kSlots); i++) RG_TRY(issue(i));
  for (size_t j = 0; j < chunks; j++) {
    const int r = (int)(j % Staging::kSlots);
    RG_TRY(hipEventSynchronize(st.ev[r]));
    parallel_memcpy(static_cast<char*>(dst_host) + j * C, st.pinned + (size_t)r * Staging::kSlotBytes,
                    std::min(C, n - j * C));
    if (j + Staging::kSlots < chunks) RG_TRY(issue(j + Staging::kSlots));
  }
  return hipSuccess;
}

}  // namespace rgnpu
