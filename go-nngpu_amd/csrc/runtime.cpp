// runtime.cpp — process-wide HIP context, caching device allocator, pinned staging
// ring for pageable host copies, and GPUPtr handle registry.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <condition_variable>
#include <mutex>
#include <thread>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "common.h"

namespace gn {

// ------------------------------------------------------------------ errors
int set_error(CError *err, int code, const char *fmt, ...) {
  if (err) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    err->message = strdup(buf);
  }
  return code;
}

int hip_error(CError *err, int code, const char *what, hipError_t e) {
  return set_error(err, code, "%s: %s", what, hipGetErrorString(e));
}

// ------------------------------------------------------------------ context
static Context g_ctx;
static std::once_flag g_ctx_once;
static int g_ctx_status = 0;
static char g_ctx_msg[256];

static void init_context() {
  hipError_t e = hipGetDevice(&g_ctx.device);
  if (e != hipSuccess) {
    snprintf(g_ctx_msg, sizeof(g_ctx_msg), "no HIP device: %s", hipGetErrorString(e));
    g_ctx_status = -1;
    return;
  }
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, g_ctx.device);
  if (e != hipSuccess) {
    snprintf(g_ctx_msg, sizeof(g_ctx_msg), "hipGetDeviceProperties: %s", hipGetErrorString(e));
    g_ctx_status = -1;
    return;
  }
  g_ctx.num_cus = prop.multiProcessorCount;
  g_ctx.lds_per_block = prop.sharedMemPerBlock;
  snprintf(g_ctx.arch, sizeof(g_ctx.arch), "%s", prop.gcnArchName);
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    snprintf(g_ctx_msg, sizeof(g_ctx_msg), "device is %s; this library is built for gfx950 only", prop.gcnArchName);
    g_ctx_status = -1;
    return;
  }
  // Default-priority, non-blocking stream (never a non-default priority).
  e = hipStreamCreateWithFlags(&g_ctx.stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    snprintf(g_ctx_msg, sizeof(g_ctx_msg), "hipStreamCreate: %s", hipGetErrorString(e));
    g_ctx_status = -1;
    return;
  }
  // Device address of the allocation-free entry point's scratch array, looked up at set-up
  // so that its calls do no lookup. A failure here affects only that entry point, which
  // repeats the lookup and reports the error itself.
  CError scratch_err{nullptr};
  if (noalloc_scratch_setup(&scratch_err) != 0) free(scratch_err.message);
}

Context *context(CError *err) {
  std::call_once(g_ctx_once, init_context);
  if (g_ctx_status != 0) {
    set_error(err, -1, "%s", g_ctx_msg);
    return nullptr;
  }
  return &g_ctx;
}

hipStream_t resolve_stream(void *stream) {
  return stream ? reinterpret_cast<hipStream_t>(stream) : g_ctx.stream;
}

// ------------------------------------------------------------------ allocator
// Size-binned caching allocator with stream-ordered release. A freed block is not reused
// at once: dev_free_on records an event on the stream the block was last used on, and the
// block waits in `pending` until that event has completed. Work enqueued before the free
// therefore never sees the block handed to a new owner, without the device-wide
// synchronisation a plain free would need.
namespace {
struct PendingBlock {
  void *ptr;
  hipEvent_t ev;
};
struct Pool {
  std::mutex mu;
  std::unordered_map<size_t, std::vector<void *>> free_lists;  // rounded size -> ready blocks
  std::unordered_map<size_t, std::vector<PendingBlock>> pending;  // rounded size -> blocks in flight
  std::unordered_map<void *, size_t> live;                     // block -> rounded size
  std::vector<hipEvent_t> spare_events;
  long cur = 0, peak = 0;
  long fail_after = -1;  // fault injection: GONNGPU_FAIL_ALLOC_AFTER
  long n_calls = 0;
  bool env_read = false;
};
Pool &pool() {
  static Pool *p = new Pool();  // leaked on purpose: outlives static destructors
  return *p;
}

size_t round_size(size_t b) {
  if (b == 0) b = 1;
  if (b <= (1u << 20)) {
    size_t r = 256;
    while (r < b) r <<= 1;
    return r;
  }
  const size_t g = 2u << 20;
  return (b + g - 1) / g * g;
}

// Moves pending blocks of size r whose event has completed to the free list.
void reclaim_locked(Pool &p, size_t r) {
  auto it = p.pending.find(r);
  if (it == p.pending.end()) return;
  auto &v = it->second;
  for (size_t i = 0; i < v.size();) {
    if (hipEventQuery(v[i].ev) == hipSuccess) {
      p.free_lists[r].push_back(v[i].ptr);
      p.spare_events.push_back(v[i].ev);
      v[i] = v.back();
      v.pop_back();
    } else {
      (void)hipGetLastError();  // hipErrorNotReady is not an error here
      ++i;
    }
  }
}

// Returns every cached block to the driver (after the work still using pending ones).
void release_cached_locked(Pool &p) {
  for (auto &kv : p.pending)
    for (PendingBlock &b : kv.second) {
      (void)hipEventSynchronize(b.ev);
      p.free_lists[kv.first].push_back(b.ptr);
      p.spare_events.push_back(b.ev);
    }
  p.pending.clear();
  for (auto &kv : p.free_lists)
    for (void *q : kv.second) (void)hipFree(q);
  p.free_lists.clear();
}
}  // namespace

void *dev_alloc(size_t bytes, CError *err) {
  if (!context(err)) return nullptr;
  Pool &p = pool();
  std::lock_guard<std::mutex> lk(p.mu);
  if (!p.env_read) {
    const char *f = getenv("GONNGPU_FAIL_ALLOC_AFTER");
    if (f && *f) p.fail_after = atol(f);
    p.env_read = true;
  }
  if (p.fail_after >= 0 && p.n_calls++ >= p.fail_after) {
    set_error(err, -3, "device allocation of %zu bytes failed (injected by GONNGPU_FAIL_ALLOC_AFTER)", bytes);
    return nullptr;
  }
  size_t r = round_size(bytes);
  void *ptr = nullptr;
  auto it = p.free_lists.find(r);
  if (it == p.free_lists.end() || it->second.empty()) {
    reclaim_locked(p, r);
    it = p.free_lists.find(r);
  }
  if (it != p.free_lists.end() && !it->second.empty()) {
    ptr = it->second.back();
    it->second.pop_back();
  } else {
    hipError_t e = hipMalloc(&ptr, r);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      release_cached_locked(p);
      e = hipMalloc(&ptr, r);
    }
    if (e != hipSuccess) {
      (void)hipGetLastError();
      set_error(err, -3, "hipMalloc(%zu): %s", r, hipGetErrorString(e));
      return nullptr;
    }
  }
  p.live[ptr] = r;
  p.cur += (long)r;
  if (p.cur > p.peak) p.peak = p.cur;
  return ptr;
}

void dev_free_on(void *ptr, hipStream_t s) {
  if (!ptr) return;
  Pool &p = pool();
  std::lock_guard<std::mutex> lk(p.mu);
  auto it = p.live.find(ptr);
  if (it == p.live.end()) return;  // not ours: ignore
  size_t r = it->second;
  p.live.erase(it);
  p.cur -= (long)r;
  hipEvent_t ev = nullptr;
  if (!p.spare_events.empty()) {
    ev = p.spare_events.back();
    p.spare_events.pop_back();
  } else if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
    (void)hipGetLastError();
    ev = nullptr;
  }
  if (ev && hipEventRecord(ev, s) == hipSuccess) {
    p.pending[r].push_back(PendingBlock{ptr, ev});
    return;
  }
  // No event: wait for the stream instead, then the block is free at once.
  (void)hipGetLastError();
  if (ev) p.spare_events.push_back(ev);
  (void)hipStreamSynchronize(s);
  p.free_lists[r].push_back(ptr);
}

void dev_free(void *ptr) { dev_free_on(ptr, g_ctx.stream); }

void memory_stats(long *cur, long *peak, long *n) {
  Pool &p = pool();
  std::lock_guard<std::mutex> lk(p.mu);
  if (cur) *cur = p.cur;
  if (peak) *peak = p.peak;
  if (n) *n = (long)p.live.size();
}

// ------------------------------------------------------------------ staging
namespace {
constexpr size_t kStageBytes = 32u << 20;  // two 32 MiB pinned buffers

// Host copies between pageable memory and the pinned staging buffers, split over the
// caller and kCopyWorkers persistent threads: one thread's memcpy runs at ~10-15 GB/s,
// below what a PCIe Gen5 link carries. Started on first use and never stopped (the
// threads wait on a condition variable between copies). Used under Staging::mu, so one
// copy runs at a time.
constexpr int kCopyWorkers = 4;
class CopyPool {
 public:
  void copy(void *dst, const void *src, size_t n) {
    if (n < (2u << 20)) {
      memcpy(dst, src, n);
      return;
    }
    start();
    constexpr size_t parts = kCopyWorkers + 1;
    const size_t slice = ((n + parts - 1) / parts + 63) & ~size_t(63);
    {
      std::lock_guard<std::mutex> lk(mu_);
      dst_ = static_cast<char *>(dst);
      src_ = static_cast<const char *>(src);
      n_ = n;
      slice_ = slice;
      pending_ = kCopyWorkers;
      ++gen_;
    }
    cv_.notify_all();
    memcpy(dst, src, std::min(slice, n));  // slice 0 on the calling thread
    std::unique_lock<std::mutex> lk(mu_);
    done_.wait(lk, [&] { return pending_ == 0; });
  }

 private:
  void start() {
    if (started_) return;
    started_ = true;
    for (int w = 0; w < kCopyWorkers; ++w) std::thread([this, w] { worker(w + 1); }).detach();
  }
  void worker(int part) {
    uint64_t seen = 0;
    for (;;) {
      char *dst;
      const char *src;
      size_t n, slice;
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return gen_ != seen; });
        seen = gen_;
        dst = dst_;
        src = src_;
        n = n_;
        slice = slice_;
      }
      const size_t off = (size_t)part * slice;
      if (off < n) memcpy(dst + off, src + off, std::min(slice, n - off));
      std::lock_guard<std::mutex> lk(mu_);
      if (--pending_ == 0) done_.notify_one();
    }
  }
  std::mutex mu_;
  std::condition_variable cv_, done_;
  char *dst_ = nullptr;
  const char *src_ = nullptr;
  size_t n_ = 0, slice_ = 0;
  int pending_ = 0;
  uint64_t gen_ = 0;
  bool started_ = false;
};
CopyPool &copy_pool() {
  static CopyPool *p = new CopyPool();
  return *p;
}
struct Staging {
  std::mutex mu;
  void *buf[2] = {nullptr, nullptr};
  hipEvent_t ev[2] = {nullptr, nullptr};
  bool ready = false;
};
Staging &staging() {
  static Staging *s = new Staging();
  return *s;
}
int staging_init(Staging &st, CError *err) {
  if (st.ready) return 0;
  for (int i = 0; i < 2; ++i) {
    hipError_t e = hipHostMalloc(&st.buf[i], kStageBytes, hipHostMallocDefault);
    if (e != hipSuccess) return hip_error(err, -4, "hipHostMalloc(staging)", e);
    e = hipEventCreateWithFlags(&st.ev[i], hipEventDisableTiming);
    if (e != hipSuccess) return hip_error(err, -4, "hipEventCreate(staging)", e);
  }
  st.ready = true;
  return 0;
}
}  // namespace

int upload(void *dst_dev, const void *src_host, size_t bytes, hipStream_t s, CError *err) {
  if (bytes == 0) return 0;
  Staging &st = staging();
  std::lock_guard<std::mutex> lk(st.mu);
  if (int rc = staging_init(st, err)) return rc;
  size_t off = 0;
  int b = 0;
  bool used[2] = {false, false};
  while (off < bytes) {
    size_t n = bytes - off < kStageBytes ? bytes - off : kStageBytes;
    if (used[b]) {
      hipError_t e = hipEventSynchronize(st.ev[b]);
      if (e != hipSuccess) return hip_error(err, -4, "upload wait", e);
    }
    copy_pool().copy(st.buf[b], static_cast<const char *>(src_host) + off, n);
    hipError_t e = hipMemcpyAsync(static_cast<char *>(dst_dev) + off, st.buf[b], n, hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return hip_error(err, -4, "upload hipMemcpyAsync", e);
    e = hipEventRecord(st.ev[b], s);
    if (e != hipSuccess) return hip_error(err, -4, "upload hipEventRecord", e);
    used[b] = true;
    off += n;
    b ^= 1;
  }
  hipError_t e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_error(err, -4, "upload sync", e);
  return 0;
}

int download(void *dst_host, const void *src_dev, size_t bytes, hipStream_t s, CError *err) {
  if (bytes == 0) return 0;
  Staging &st = staging();
  std::lock_guard<std::mutex> lk(st.mu);
  if (int rc = staging_init(st, err)) return rc;
  // Pipeline: enqueue chunk i into buffer i%2, then drain chunk i-1 to the host.
  size_t nchunks = (bytes + kStageBytes - 1) / kStageBytes;
  for (size_t i = 0; i <= nchunks; ++i) {
    if (i < nchunks) {
      size_t off = i * kStageBytes;
      size_t n = bytes - off < kStageBytes ? bytes - off : kStageBytes;
      int b = (int)(i & 1);
      hipError_t e = hipMemcpyAsync(st.buf[b], static_cast<const char *>(src_dev) + off, n, hipMemcpyDeviceToHost, s);
      if (e != hipSuccess) return hip_error(err, -4, "download hipMemcpyAsync", e);
      e = hipEventRecord(st.ev[b], s);
      if (e != hipSuccess) return hip_error(err, -4, "download hipEventRecord", e);
    }
    if (i > 0) {
      size_t j = i - 1;
      size_t off = j * kStageBytes;
      size_t n = bytes - off < kStageBytes ? bytes - off : kStageBytes;
      int b = (int)(j & 1);
      hipError_t e = hipEventSynchronize(st.ev[b]);
      if (e != hipSuccess) return hip_error(err, -4, "download wait", e);
      copy_pool().copy(static_cast<char *>(dst_host) + off, st.buf[b], n);
    }
  }
  return 0;
}

// ------------------------------------------------------------------ handles
namespace {
std::mutex g_handles_mu;
std::unordered_set<Buffer *> &handles() {
  static auto *h = new std::unordered_set<Buffer *>();
  return *h;
}
}  // namespace

Buffer *as_buffer(GPUPtr p) {
  if (!p) return nullptr;
  std::lock_guard<std::mutex> lk(g_handles_mu);
  Buffer *b = static_cast<Buffer *>(p);
  if (!handles().count(b)) return nullptr;
  return b->magic == kBufferMagic ? b : nullptr;
}

Buffer *register_buffer(void *dptr, size_t bytes) {
  Buffer *b = new Buffer{kBufferMagic, dptr, bytes};
  std::lock_guard<std::mutex> lk(g_handles_mu);
  handles().insert(b);
  return b;
}

bool unregister_buffer(Buffer *b) {
  std::lock_guard<std::mutex> lk(g_handles_mu);
  if (!handles().erase(b)) return false;
  b->magic = 0;
  return true;
}

// ---------------------------------------------------------------- per-stream scratch
static std::mutex g_scratch_mu;
struct StreamScratch {
  void *ptr = nullptr;
  size_t bytes = 0;
};
static std::unordered_map<hipStream_t, StreamScratch> g_scratch;
// Scratch blocks above this size go back to the pool after the call that needed them (see
// stream_scratch_trim): the pool's cache can hand them out again or, when hipMalloc fails,
// return them to the driver, which it cannot do with a block a stream keeps.
constexpr size_t kScratchRetainBytes = (size_t)256 << 20;

void *stream_scratch(hipStream_t s, size_t bytes, std::unique_lock<std::mutex> &lk, CError *err) {
  lk = std::unique_lock<std::mutex>(g_scratch_mu);
  StreamScratch &w = g_scratch[s];
  if (w.bytes < bytes) {
    if (w.ptr) {
      dev_free_on(w.ptr, s);  // reused only after the kernels already enqueued on s
      w = StreamScratch{};
    }
    const size_t nb = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
    void *p = dev_alloc(nb, err);
    if (!p) return nullptr;
    w.ptr = p;
    w.bytes = nb;
  }
  return w.ptr;
}

void stream_scratch_trim(hipStream_t s, std::unique_lock<std::mutex> &lk) {
  if (!lk.owns_lock()) return;
  auto it = g_scratch.find(s);
  if (it == g_scratch.end() || it->second.bytes <= kScratchRetainBytes) return;
  dev_free_on(it->second.ptr, s);  // after the kernels just enqueued; then back in the pool's cache
  g_scratch.erase(it);
}

}  // namespace gn
