// Pageable host memory <-> device through pinned staging.
//
// On the MI355X box a pageable hipMemcpy moves ~27 GB/s host to device and
// ~16 GB/s device to host (the runtime stages it with one thread), while
// pinned memory moves ~57 GB/s each way and four threads copy pageable memory
// at ~77 GB/s.  A transfer is therefore cut into chunks that rotate through
// kStageSlots pinned slots: helper threads fill (or drain) one slot while the
// DMA engine moves the others.  Transfers below kStageMin go straight through
// hipMemcpyAsync.
#include "hostcopy.h"

#include <algorithm>
#include <condition_variable>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

#include <unistd.h>

#include "common.h"

namespace nship {
namespace {

constexpr size_t kStageChunk = size_t(16) << 20;  // bytes per pinned slot
constexpr size_t kStageMin = size_t(2) << 20;    // smaller transfers are not staged
constexpr size_t kPoolMin = size_t(1) << 20;     // smaller host copies run on the calling thread

// Process-wide helper threads for the host side of the staged copies.  One
// copy at a time (callers on several models serialise on call_mu); the
// calling thread takes part 0 and the helpers parts 1..n.  The pool lives
// until the process ends (never destroyed, so no join at exit); a child
// process forked after it started copies on its calling thread alone, as
// the helpers exist only in the parent.
class CopyPool {
 public:
  static CopyPool& get() {
    static CopyPool* pool = new CopyPool();
    return *pool;
  }
  void copy(void* dst, const void* src, size_t n) {
    if (n < kPoolMin || th_.empty() || getpid() != pid_) {
      std::memcpy(dst, src, n);
      return;
    }
    std::lock_guard<std::mutex> call(call_mu_);
    {
      std::lock_guard<std::mutex> lk(mu_);
      job_ = Job{static_cast<char*>(dst), static_cast<const char*>(src), n, (int)th_.size() + 1};
      pending_ = (int)th_.size();
      gen_++;
    }
    work_cv_.notify_all();
    run(job_, 0);
    std::unique_lock<std::mutex> lk(mu_);
    done_cv_.wait(lk, [&] { return pending_ == 0; });
  }

 private:
  struct Job {
    char* dst = nullptr;
    const char* src = nullptr;
    size_t n = 0;
    int parts = 1;
  };
  // Helper threads that cannot be created (a process or thread limit) are
  // simply fewer helpers: copies split over the threads that exist, down to
  // the calling thread alone, so no exception leaves the C ABI.
  CopyPool() {
    const unsigned hw = std::thread::hardware_concurrency();
    const int helpers = hw > 1 ? (int)std::min(4u, hw - 1) : 0;
    for (int i = 0; i < helpers; i++) {
      try {
        th_.emplace_back([this, i] { worker(i + 1); });
      } catch (const std::exception&) {
        break;
      }
    }
  }
  // part p of the job: 64-byte aligned pieces of ceil(n / parts)
  static void run(const Job& j, int p) {
    const size_t per = ((j.n + j.parts - 1) / j.parts + 63) & ~size_t(63);
    const size_t b = std::min(j.n, per * p), e = std::min(j.n, b + per);
    if (e > b) std::memcpy(j.dst + b, j.src + b, e - b);
  }
  void worker(int part) {
    unsigned long seen = 0;
    for (;;) {
      Job j;
      {
        std::unique_lock<std::mutex> lk(mu_);
        work_cv_.wait(lk, [&] { return gen_ != seen; });
        seen = gen_;
        j = job_;
      }
      run(j, part);
      {
        std::lock_guard<std::mutex> lk(mu_);
        if (--pending_ == 0) done_cv_.notify_one();
      }
    }
  }
  std::vector<std::thread> th_;
  std::mutex call_mu_, mu_;
  std::condition_variable work_cv_, done_cv_;
  Job job_;
  unsigned long gen_ = 0;
  int pending_ = 0;
  const pid_t pid_ = getpid();
};

// All slots or none: a failure part way frees what it allocated, so the
// next call tries again from scratch.
int stage_init(HostStage& st, hipStream_t s) {
  if (st.slot[kStageSlots - 1]) return 0;
  hipError_t e = hipSuccess;
  for (int k = 0; k < kStageSlots && e == hipSuccess; k++) {
    e = hipHostMalloc(reinterpret_cast<void**>(&st.slot[k]), kStageChunk, hipHostMallocDefault);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&st.ev[k], hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(st.ev[k], s);  // a slot starts free
  }
  if (e != hipSuccess) {
    stage_free(st);
    set_error(std::string("host staging buffers: ") + hipGetErrorString(e));
    return -1;
  }
  return 0;
}

}  // namespace

int stage_h2d(HostStage& st, void* dev, const void* host, size_t bytes, hipStream_t s) {
  if (bytes < kStageMin) {
    NSH_CHECK(hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, s));
    return 0;
  }
  if (stage_init(st, s) != 0) return -1;
  const char* h = static_cast<const char*>(host);
  char* d = static_cast<char*>(dev);
  for (size_t off = 0, i = 0; off < bytes; off += kStageChunk, i++) {
    const int k = (int)(i % kStageSlots);
    const size_t len = std::min(kStageChunk, bytes - off);
    NSH_CHECK(hipEventSynchronize(st.ev[k]));  // this slot's previous DMA has finished
    CopyPool::get().copy(st.slot[k], h + off, len);
    NSH_CHECK(hipMemcpyAsync(d + off, st.slot[k], len, hipMemcpyHostToDevice, s));
    NSH_CHECK(hipEventRecord(st.ev[k], s));
  }
  return 0;
}

int stage_d2h(HostStage& st, void* host, const void* dev, size_t bytes, hipStream_t s) {
  if (bytes < kStageMin) {
    NSH_CHECK(hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, s));
    NSH_CHECK(hipStreamSynchronize(s));
    return 0;
  }
  if (stage_init(st, s) != 0) return -1;
  char* h = static_cast<char*>(host);
  const char* d = static_cast<const char*>(dev);
  const size_t n = (bytes + kStageChunk - 1) / kStageChunk;
  auto issue = [&](size_t i) -> int {
    const int k = (int)(i % kStageSlots);
    const size_t off = i * kStageChunk, len = std::min(kStageChunk, bytes - off);
    NSH_CHECK(hipStreamWaitEvent(s, st.ev[k], 0));  // the slot's last DMA may be on another stream
    NSH_CHECK(hipMemcpyAsync(st.slot[k], d + off, len, hipMemcpyDeviceToHost, s));
    NSH_CHECK(hipEventRecord(st.ev[k], s));
    return 0;
  };
  for (size_t i = 0; i < std::min<size_t>(kStageSlots, n); i++)
    if (issue(i) != 0) return -1;
  for (size_t i = 0; i < n; i++) {
    const int k = (int)(i % kStageSlots);
    const size_t off = i * kStageChunk, len = std::min(kStageChunk, bytes - off);
    NSH_CHECK(hipEventSynchronize(st.ev[k]));
    CopyPool::get().copy(h + off, st.slot[k], len);
    if (i + kStageSlots < n && issue(i + kStageSlots) != 0) return -1;
  }
  return 0;
}

void stage_free(HostStage& st) {
  for (int k = 0; k < kStageSlots; k++) {
    if (st.ev[k]) {
      hipEventSynchronize(st.ev[k]);
      hipEventDestroy(st.ev[k]);
    }
    if (st.slot[k]) hipHostFree(st.slot[k]);
    st.ev[k] = nullptr;
    st.slot[k] = nullptr;
  }
}

}  // namespace nship
