// expert_stream.hip -- routed experts read from the packed layer file on
// demand, for models whose experts exceed HBM (the reference's expert
// streaming: parallel pread of the K selected experts per token,
// infer.m:1478-1602, N_PREAD_CHUNKS at 1502; the layer files of
// repack_experts.c, expert e at e * expert_size).
//
// Each streamed layer keeps an LRU cache of n_cache expert blobs in HBM.
// plan() does one token's cache bookkeeping; the caller then launches the
// shared expert and the hits at once, and read() reads the misses with a
// pool of host threads: every thread preads 4 MB chunks into its own two
// pinned buffers and queues each chunk's host-to-device copy on its own
// stream, behind an event, so file reads overlap PCIe copies.  As the last
// chunk of a miss is queued, the calling thread makes the compute stream
// wait for that miss's copies and launches its kernels: expert k computes
// while the others are still read (the reference encodes each expert as its
// last chunk lands, infer.m:1577-1601, and runs the shared expert alongside,
// 1886-1894).  The blobs stay in the packed layout; the expert kernels read
// it as they read caller blobs.
#include <errno.h>
#include <string.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <mutex>
#include <thread>

#include "../../include/fdm.h"
#include "fdm_internal.h"

namespace fdm {

namespace {

constexpr size_t kStreamChunk = 4u << 20;

// Pinned staging and copy streams shared by every streamed layer, grown to
// the largest n_threads a layer asks for.  One fetch at a time uses it.
struct ReadPool {
  struct Worker {
    hipStream_t s = nullptr;
    void* buf[2] = {};
    hipEvent_t ev[2] = {};
  };
  std::vector<Worker> w;
  int device = -1;
  std::mutex mu;  // held by a fetch's reads and by init

  hipError_t init(int n, int dev) {
    std::lock_guard<std::mutex> lock(mu);
    device = dev;
    while (w.size() < (size_t)n) {
      Worker k;  // kept only when complete
      hipError_t e = hipStreamCreateWithFlags(&k.s, hipStreamNonBlocking);
      for (int b = 0; b < 2 && e == hipSuccess; ++b) {
        e = hipHostMalloc(&k.buf[b], kStreamChunk, hipHostMallocDefault);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&k.ev[b], hipEventDisableTiming);
      }
      if (e != hipSuccess) {
        free_worker(k);
        return e;
      }
      w.push_back(k);
    }
    return hipSuccess;
  }
  static void free_worker(Worker& k) {
    if (k.s) (void)hipStreamSynchronize(k.s);
    for (int b = 0; b < 2; ++b) {
      if (k.ev[b]) (void)hipEventDestroy(k.ev[b]);
      if (k.buf[b]) (void)hipHostFree(k.buf[b]);
    }
    if (k.s) (void)hipStreamDestroy(k.s);
  }
  void release() {
    std::lock_guard<std::mutex> lock(mu);
    for (Worker& k : w) free_worker(k);
    w.clear();
  }
};

ReadPool g_pool;

}  // namespace

ExpertStream::~ExpertStream() {
  if (fd_ >= 0) close(fd_);
  for (hipEvent_t ev : chunk_ev_) (void)hipEventDestroy(ev);
  if (cache_) (void)hipFree(cache_);
}

int ExpertStream::open(const char* path, size_t expert_size, int n_experts, int n_cache, int n_threads,
                       int device, std::string* err) {
  es_ = expert_size;
  n_experts_ = n_experts;
  n_cache_ = n_cache;
  n_threads_ = n_threads;
  fd_ = ::open(path, O_RDONLY | O_CLOEXEC);
  if (fd_ < 0) {
    *err = std::string("cannot open ") + path + ": " + strerror(errno);
    return FDM_E_IO;
  }
  struct stat st;
  if (fstat(fd_, &st) != 0 || (uint64_t)st.st_size < (uint64_t)n_experts * es_) {
    *err = std::string(path) + " is shorter than n_experts x expert_size";
    return FDM_E_FORMAT;
  }
  if (hipMalloc(&cache_, (size_t)n_cache * es_) != hipSuccess) {
    *err = "cannot allocate the expert cache";
    return FDM_E_NOMEM;
  }
  if (g_pool.init(std::max(n_threads, 1), device) != hipSuccess) {
    *err = "cannot allocate the pinned read buffers";
    return FDM_E_NOMEM;
  }
  slot_of_.assign(n_experts, -1);
  expert_in_.assign(n_cache, -1);
  last_use_.assign(n_cache, 0);
  return FDM_OK;
}

int ExpertStream::plan(const int* ids, int K, int* slots, bool* miss, std::string* err) {
  plan_.clear();
  if (K > n_cache_) {
    *err = "K exceeds the expert cache";
    return FDM_E_INVAL;
  }
  ++tick_;
  std::vector<char> held(n_cache_, 0);  // slots this token uses
  for (int k = 0; k < K; ++k) {
    const int e = ids[k];
    if (e < 0 || e >= n_experts_) {
      *err = "routed expert id out of range";
      return FDM_E_INVAL;
    }
    miss[k] = false;
    if (slot_of_[e] >= 0) {
      slots[k] = slot_of_[e];
      if (!held[slots[k]]) ++hits_;
      held[slots[k]] = 1;
      last_use_[slots[k]] = tick_;
    } else {
      slots[k] = -1;
    }
  }
  for (int k = 0; k < K; ++k) {
    if (slots[k] >= 0) continue;
    const int e = ids[k];
    if (slot_of_[e] >= 0) {  // a repeated id of this token, placed just now
      slots[k] = slot_of_[e];
      miss[k] = true;
      for (Miss& m : plan_)
        if (m.expert == e) m.ks.push_back(k);
      continue;
    }
    int v = -1;  // least recently used slot that this token does not hold
    for (int c = 0; c < n_cache_; ++c)
      if (!held[c] && (v < 0 || last_use_[c] < last_use_[v])) v = c;
    if (expert_in_[v] >= 0) slot_of_[expert_in_[v]] = -1;
    expert_in_[v] = e;
    slot_of_[e] = v;
    last_use_[v] = tick_;
    held[v] = 1;
    slots[k] = v;
    miss[k] = true;
    plan_.push_back(Miss{e, v, {k}});
    ++misses_;
  }
  return FDM_OK;
}

int ExpertStream::read(hipStream_t compute, const std::function<int(int)>& ready, std::string* err) {
  if (plan_.empty()) return FDM_OK;
  const size_t per = (es_ + kStreamChunk - 1) / kStreamChunk;
  const size_t n_jobs = plan_.size() * per;
  while (chunk_ev_.size() < n_jobs) {
    hipEvent_t ev;
    if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
      *err = "cannot create the copy events";
      return FDM_E_HIP;
    }
    chunk_ev_.push_back(ev);
  }
  std::atomic<size_t> next{0};
  std::atomic<int> rc{FDM_OK};
  std::atomic<int> io_errno{0};
  // the chunk copies queued so far, handed to this thread
  std::mutex qmu;
  std::condition_variable qcv;
  std::vector<size_t> queued;
  int running = 0;
  std::lock_guard<std::mutex> pool_lock(g_pool.mu);
  auto work = [&](int t) {
    if (hipSetDevice(g_pool.device) != hipSuccess) {
      rc = FDM_E_HIP;
    } else {
      ReadPool::Worker& wk = g_pool.w[t];
      bool used[2] = {false, false};
      for (int j = 0;; ++j) {
        const size_t i = next.fetch_add(1);
        if (i >= n_jobs || rc.load() != FDM_OK) break;
        const Miss& m = plan_[i / per];
        const size_t off = (i % per) * kStreamChunk;
        const size_t len = std::min(kStreamChunk, es_ - off);
        const int b = j & 1;
        if (used[b] && hipEventSynchronize(wk.ev[b]) != hipSuccess) {
          rc = FDM_E_HIP;
          break;
        }
        uint8_t* dst = static_cast<uint8_t*>(wk.buf[b]);
        size_t got = 0;
        const off_t at = (off_t)((uint64_t)m.expert * es_ + off);
        while (got < len) {
          const ssize_t r = pread(fd_, dst + got, len - got, at + (off_t)got);
          if (r < 0 && errno == EINTR) continue;
          if (r <= 0) {
            io_errno = r < 0 ? errno : EIO;
            rc = FDM_E_IO;
            break;
          }
          got += (size_t)r;
        }
        if (rc.load() != FDM_OK) break;
        if (hipMemcpyAsync(cache_ + (size_t)m.slot * es_ + off, dst, len, hipMemcpyHostToDevice, wk.s) !=
                hipSuccess ||
            hipEventRecord(wk.ev[b], wk.s) != hipSuccess || hipEventRecord(chunk_ev_[i], wk.s) != hipSuccess) {
          rc = FDM_E_HIP;
          break;
        }
        used[b] = true;
        {
          std::lock_guard<std::mutex> lk(qmu);
          queued.push_back(i);
        }
        qcv.notify_one();
      }
      // the pinned buffers are free for the next call once their copies landed
      if (hipStreamSynchronize(wk.s) != hipSuccess) rc = FDM_E_HIP;
    }
    std::lock_guard<std::mutex> lk(qmu);
    --running;
    qcv.notify_one();
  };
  const int n_thr = (int)std::min<size_t>(std::min<size_t>((size_t)std::max(n_threads_, 1), g_pool.w.size()), n_jobs);
  running = n_thr;
  std::vector<std::thread> th;
  for (int t = 0; t < n_thr; ++t) th.emplace_back(work, t);
  // this thread: each miss's kernels behind its chunk copies, as they queue
  std::vector<size_t> issued(plan_.size(), 0);
  std::vector<char> launched(plan_.size(), 0);
  int launch_rc = FDM_OK;
  auto launch = [&](size_t mi, bool wait) {
    if (wait)
      for (size_t c = 0; c < per; ++c)
        if (hipStreamWaitEvent(compute, chunk_ev_[mi * per + c], 0) != hipSuccess) launch_rc = FDM_E_HIP;
    for (int k : plan_[mi].ks)
      if (int r = ready(k)) launch_rc = r;
    launched[mi] = 1;
  };
  for (;;) {
    std::vector<size_t> got;
    bool done;
    {
      std::unique_lock<std::mutex> lk(qmu);
      qcv.wait(lk, [&] { return !queued.empty() || running == 0; });
      got.swap(queued);
      done = running == 0;
    }
    for (size_t i : got)
      if (++issued[i / per] == per) launch(i / per, true);
    if (done) break;
  }
  for (auto& x : th) x.join();
  if (rc.load() != FDM_OK) {
    for (size_t mi = 0; mi < plan_.size(); ++mi) {
      if (launched[mi]) {
        bytes_ += es_;
        continue;
      }
      slot_of_[plan_[mi].expert] = -1;  // not a valid cache entry
      expert_in_[plan_[mi].slot] = -1;
      launch(mi, false);
    }
    *err = rc.load() == FDM_E_IO ? std::string("reading the layer file: ") + strerror(io_errno.load())
                                 : std::string("copying experts to the device");
    return rc.load();
  }
  bytes_ += (uint64_t)plan_.size() * es_;
  if (launch_rc != FDM_OK) *err = "launching the expert kernels";
  return launch_rc;
}

void release_stream_pool() { g_pool.release(); }

}  // namespace fdm
