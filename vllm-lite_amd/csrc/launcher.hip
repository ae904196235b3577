// A submission thread for captured step graphs. The reference has no
// counterpart: its engine runs every step synchronously on the host
// (vllmlite/engine.py:99-181).
//
// hipGraphLaunch of a TinyLlama decode step's graph (~33 kernel and copy
// nodes) costs the calling host thread ~33 us. The engine has other work for
// that time (the previous step's outputs, the next schedule), so the launch,
// and the event record after it, run on a thread of their own: the caller
// stages the step, submits, and goes on. Submissions run in order on the
// launcher's one stream; a ticket names each. The thread spins for a while
// before it sleeps, so that a submission made while steps are flowing starts
// within microseconds instead of a futex wake-up later.
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <deque>
#include <mutex>
#include <thread>

#include "vl_common.h"

namespace {

struct Item {
  hipGraphExec_t exec;
  hipEvent_t event;
  uint64_t ticket;
};

struct Launcher {
  int device = 0;
  hipStream_t stream = nullptr;
  std::thread th;
  std::mutex mu;
  std::condition_variable cv_work, cv_done;
  std::deque<Item> q;            // under mu
  uint64_t next_ticket = 1;      // under mu
  int status = 0;                // the first failure (a hipError_t), under mu
  bool stop = false;             // under mu
  std::atomic<uint64_t> queued{0};     // tickets handed out
  std::atomic<uint64_t> completed{0};  // the last ticket whose calls have returned

  void run() {
    (void)hipSetDevice(device);
    for (;;) {
      // spin up to ~200 us for the next submission before sleeping
      const auto t0 = std::chrono::steady_clock::now();
      while (queued.load(std::memory_order_acquire) == completed.load(std::memory_order_relaxed) &&
             std::chrono::steady_clock::now() - t0 < std::chrono::microseconds(200))
        std::this_thread::yield();
      Item it;
      {
        std::unique_lock<std::mutex> lk(mu);
        cv_work.wait(lk, [&] { return stop || !q.empty(); });
        if (q.empty()) return;  // stopped with nothing left to launch
        it = q.front();
        q.pop_front();
      }
      hipError_t e = hipSuccess;
      if (it.exec) e = hipGraphLaunch(it.exec, stream);
      if (e == hipSuccess && it.event) e = hipEventRecord(it.event, stream);
      {
        std::lock_guard<std::mutex> lk(mu);
        if (e != hipSuccess && status == 0) status = (int)e;
        completed.store(it.ticket, std::memory_order_release);
      }
      cv_done.notify_all();
    }
  }
};

}  // namespace

extern "C" int vl_launcher_create(int device, void* stream, void** out) {
  VL_CHECK_ARG(out && stream, "null pointer");
  Launcher* l = new Launcher;
  l->device = device;
  l->stream = (hipStream_t)stream;
  l->th = std::thread([l] { l->run(); });
  *out = l;
  return VL_OK;
}

extern "C" int vl_launcher_submit(void* launcher, void* graph_exec, void* event,
                                  uint64_t* ticket) {
  VL_CHECK_ARG(launcher && ticket, "null pointer");
  Launcher* l = static_cast<Launcher*>(launcher);
  {
    std::lock_guard<std::mutex> lk(l->mu);
    VL_CHECK_ARG(!l->stop, "launcher stopped");
    *ticket = l->next_ticket++;
    l->q.push_back(Item{(hipGraphExec_t)graph_exec, (hipEvent_t)event, *ticket});
    l->queued.store(*ticket, std::memory_order_release);
  }
  l->cv_work.notify_one();
  return VL_OK;
}

extern "C" int vl_launcher_wait(void* launcher, uint64_t ticket) {
  VL_CHECK_ARG(launcher, "null pointer");
  Launcher* l = static_cast<Launcher*>(launcher);
  if (l->completed.load(std::memory_order_acquire) < ticket) {
    std::unique_lock<std::mutex> lk(l->mu);
    VL_CHECK_ARG(ticket < l->next_ticket, "ticket %llu was never issued",
                 (unsigned long long)ticket);
    l->cv_done.wait(lk, [&] { return l->completed.load(std::memory_order_acquire) >= ticket; });
  }
  std::lock_guard<std::mutex> lk(l->mu);
  if (l->status) {
    vl_set_error("a graph launch or event record on the launcher thread failed: %s",
                 hipGetErrorString((hipError_t)l->status));
    return l->status;
  }
  return VL_OK;
}

extern "C" int vl_host_wait_nonneg(const int32_t* values, int64_t n, int64_t timeout_us) {
  VL_CHECK_ARG(n >= 0 && (values || n == 0), "bad arguments");
  const volatile int32_t* v = values;
  const auto t0 = std::chrono::steady_clock::now();
  int64_t i = 0;
  for (;;) {
    while (i < n && v[i] >= 0) ++i;
    if (i == n) return VL_OK;
    if (std::chrono::steady_clock::now() - t0 > std::chrono::microseconds(timeout_us)) {
      vl_set_error("value %lld of %lld still negative after %lld us", (long long)i,
                   (long long)n, (long long)timeout_us);
      return VL_EINVAL;
    }
    __builtin_ia32_pause();
  }
}

extern "C" int vl_launcher_destroy(void* launcher) {
  if (!launcher) return VL_OK;
  Launcher* l = static_cast<Launcher*>(launcher);
  {
    std::lock_guard<std::mutex> lk(l->mu);
    l->stop = true;  // the queue still drains: every submission is launched
  }
  l->cv_work.notify_one();
  l->th.join();
  delete l;
  return VL_OK;
}
