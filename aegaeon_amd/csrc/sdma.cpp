// DMA-engine copies issued by the library, for STAGED host transfers.
//
// STAGED moves each chunk between device staging and the host pool with
// copies. hipMemcpyAsync leaves the choice between an SDMA engine and a
// blit kernel on the stream's queue to the HIP runtime. A blit kernel holds
// CUs for the whole copy (under rocprof's kernel trace the runtime ran
// these copies as 256-workgroup blit kernels, and a GEMM beside them lost
// half its rate). Here each chunk's copies go straight to ROCr's
// hsa_amd_memory_async_copy, which runs host<->device copies on the
// agent's SDMA engines. The engines are the runtime's own choice: ROCr's
// header warns that fixing engines with hsa_amd_memory_async_copy_on_engine
// while other code uses hsa_amd_memory_async_copy "can result in resource
// conflicts", and hipMemcpyAsync is such other code.
//
// Ordering with the caller's HIP stream, without any device-side wait and
// without any HIP call on the library's threads:
//   * a lane per (device, direction, stream) runs that stream's jobs (one
//     per staged chunk) in submission order on a library thread;
//   * where a job's copies may start (after the gather kernel, or after the
//     scatter that last used the staging buffer) the stream runs a one-wave
//     kernel that stores the job's number into the job's own start slot, a
//     pinned host word; the lane's thread polls the slot (at most 60 s),
//     issues the copies, waits for their completion signals, then stores
//     the job's number into the lane's done word, also pinned;
//   * the stream waits for the done word with a host function
//     (hipLaunchHostFunc) before the scatter kernel, before reusing a
//     staging buffer, and before the call's last operation. The command
//     processor holds the stream meanwhile; no wave waits on a CU.
// A host function waits only for jobs its own stream released earlier, so
// host functions of different streams, which may run on one runtime
// thread, never wait for each other. Every wait ends within 60 s; a late
// one sets a flag that the next call reports.
//
// The HSA runtime is the one the HIP runtime in this process already
// loaded (found among the loaded objects); the library does not link
// another copy.

#include <hip/hip_runtime.h>
#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>

#include "aegkv.h"
#include "errors.h"
#include "sdma.h"

#include <dlfcn.h>
#include <link.h>

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdio>
#include <cstring>
#include <deque>
#include <map>
#include <mutex>
#include <set>
#include <string>
#include <thread>
#include <tuple>
#include <vector>

namespace aegkv_sdma {
namespace {

#define fail aegkv_set_error

struct Api {
  decltype(&hsa_init) init = nullptr;
  decltype(&hsa_system_get_info) system_get_info = nullptr;
  decltype(&hsa_iterate_agents) iterate_agents = nullptr;
  decltype(&hsa_agent_get_info) agent_get_info = nullptr;
  decltype(&hsa_signal_create) signal_create = nullptr;
  decltype(&hsa_signal_destroy) signal_destroy = nullptr;
  decltype(&hsa_signal_wait_scacquire) signal_wait = nullptr;
  decltype(&hsa_amd_memory_async_copy) async_copy = nullptr;
  uint64_t ticks_per_s = 0;  // unit of the signal waits' timeout hint
};

// Path of the HSA runtime loaded in this process.
int find_hsa(dl_phdr_info* info, size_t, void* data) {
  if (info->dlpi_name && std::strstr(info->dlpi_name, "libhsa-runtime64")) {
    *static_cast<std::string*>(data) = info->dlpi_name;
    return 1;
  }
  return 0;
}

template <typename F>
bool bind(void* lib, const char* name, F* out) {
  *out = reinterpret_cast<F>(dlsym(lib, name));
  return *out != nullptr;
}

std::mutex g_api_mu;
Api* g_api = nullptr;

int load_api(Api** out) {
  std::lock_guard<std::mutex> lk(g_api_mu);
  if (g_api) {
    *out = g_api;
    return 0;
  }
  std::string path;
  dl_iterate_phdr(find_hsa, &path);
  if (path.empty()) return fail(AEGKV_EINVAL, "no HSA runtime is loaded in this process");
  void* lib = dlopen(path.c_str(), RTLD_NOW | RTLD_NOLOAD);
  if (!lib) return fail(AEGKV_EINVAL, "cannot open the loaded HSA runtime %s", path.c_str());
  Api a;
  if (!bind(lib, "hsa_init", &a.init) || !bind(lib, "hsa_iterate_agents", &a.iterate_agents) ||
      !bind(lib, "hsa_system_get_info", &a.system_get_info) ||
      !bind(lib, "hsa_agent_get_info", &a.agent_get_info) ||
      !bind(lib, "hsa_signal_create", &a.signal_create) ||
      !bind(lib, "hsa_signal_destroy", &a.signal_destroy) ||
      !bind(lib, "hsa_signal_wait_scacquire", &a.signal_wait) ||
      !bind(lib, "hsa_amd_memory_async_copy", &a.async_copy))
    return fail(AEGKV_EINVAL, "the HSA runtime %s lacks the calls STAGED needs", path.c_str());
  if (a.init() != HSA_STATUS_SUCCESS) return fail(AEGKV_EINVAL, "hsa_init failed");
  if (a.system_get_info(HSA_SYSTEM_INFO_TIMESTAMP_FREQUENCY, &a.ticks_per_s) !=
          HSA_STATUS_SUCCESS || a.ticks_per_s == 0)
    return fail(AEGKV_EINVAL, "no HSA timestamp frequency");
  g_api = new Api(a);  // lives until the process ends
  *out = g_api;
  return 0;
}

struct Agents {
  uint32_t bdfid = 0, domain = 0;
  hsa_agent_t gpu{0};
  bool found = false;
  std::vector<hsa_agent_t> cpus;
  Api* api = nullptr;
};

hsa_status_t visit_agent(hsa_agent_t agent, void* data) {
  auto* s = static_cast<Agents*>(data);
  hsa_device_type_t type;
  if (s->api->agent_get_info(agent, HSA_AGENT_INFO_DEVICE, &type) != HSA_STATUS_SUCCESS)
    return HSA_STATUS_SUCCESS;
  if (type == HSA_DEVICE_TYPE_CPU) {
    s->cpus.push_back(agent);
  } else if (type == HSA_DEVICE_TYPE_GPU && !s->found) {
    uint32_t bdfid = 0, domain = 0;
    s->api->agent_get_info(agent, static_cast<hsa_agent_info_t>(HSA_AMD_AGENT_INFO_BDFID), &bdfid);
    s->api->agent_get_info(agent, static_cast<hsa_agent_info_t>(HSA_AMD_AGENT_INFO_DOMAIN),
                           &domain);
    if (bdfid == s->bdfid && domain == s->domain) {
      s->gpu = agent;
      s->found = true;
    }
  }
  return HSA_STATUS_SUCCESS;
}

struct Copy {
  void* dst;
  const void* src;
  size_t len;
};

struct Job {
  uint64_t seq;              // start slot value, then done-word value
  std::vector<Copy> copies;
};

// Longest a lane polls a job's start slot, and longest it waits for the
// job's copies, before it records a failure (the stream's own wait for the
// done word has the same budget).
constexpr auto kHostWait = std::chrono::seconds(60);

// Start slots per lane: a job's slot is reused kStartSlots jobs later, and
// submit() keeps fewer than that many jobs unfinished.
constexpr uint64_t kStartSlots = 1024;

enum Stage : int { IDLE = 0, WAIT_START = 1, COPYING = 2, FAILED = 3 };

// One direction of one stream: its pinned words and worker thread.
// The thread calls the HSA runtime only.
struct Lane {
  int dir = 0, device = -1;
  Api* api = nullptr;
  hsa_agent_t dst_agent{0}, src_agent{0};
  uint64_t* done = nullptr;  // pinned: number of the newest finished job
  uint64_t* slots = nullptr; // pinned: kStartSlots start slots, job seq at seq % kStartSlots
  std::mutex mu;
  std::condition_variable cv;       // a job was queued
  std::condition_variable cv_space; // a job finished
  std::deque<Job> jobs;
  std::set<uint64_t> abandoned;     // jobs whose copies are skipped
  uint64_t submitted = 0, finished = 0;
  std::string error;                // first failure, reported by the next call
  std::atomic<int> stage{IDLE};
  std::atomic<uint64_t> current{0};
  std::atomic<int64_t> pending{0};  // copies of the current job not yet complete
  std::atomic<bool> broken{false};  // copies were left pending: no more jobs run

  void run() {
    for (;;) {
      Job job;
      {
        std::unique_lock<std::mutex> lk(mu);
        cv.wait(lk, [&] { return !jobs.empty(); });
        job = std::move(jobs.front());
        jobs.pop_front();
      }
      current.store(job.seq);
      std::string err = execute(job);
      {
        std::lock_guard<std::mutex> lk(mu);
        abandoned.erase(job.seq);
        if (!err.empty() && error.empty()) error = err;
        finished = job.seq;
      }
      stage.store(err.empty() ? IDLE : FAILED);
      // release the stream even after a failure; the error is reported
      __atomic_store_n(done, job.seq, __ATOMIC_RELEASE);
      cv_space.notify_all();
    }
  }

  bool wait_start(uint64_t seq) {
    const uint64_t* slot = slots + seq % kStartSlots;
    const auto t0 = std::chrono::steady_clock::now();
    for (int spins = 0; __atomic_load_n(slot, __ATOMIC_ACQUIRE) < seq; ++spins) {
      if (spins < 4096) {
        std::this_thread::yield();
        continue;
      }
      if (std::chrono::steady_clock::now() - t0 > kHostWait) return false;
      std::this_thread::sleep_for(std::chrono::microseconds(20));
    }
    return true;
  }

  std::string execute(Job& job) {
    char msg[160];
    stage.store(WAIT_START);
    if (!wait_start(job.seq)) {
      std::snprintf(msg, sizeof msg, "job %llu: its start slot was not set within %lld s",
                    static_cast<unsigned long long>(job.seq),
                    static_cast<long long>(kHostWait.count()));
      return msg;
    }
    {
      std::lock_guard<std::mutex> lk(mu);
      if (abandoned.count(job.seq)) return "";
    }
    if (job.copies.empty() || broken.load()) return "";
    stage.store(COPYING);
    // One completion signal per job: each copy lowers it by one.
    const int64_t total = static_cast<int64_t>(job.copies.size());
    hsa_signal_t sig{0};
    if (api->signal_create(total, 0, nullptr, &sig) != HSA_STATUS_SUCCESS)
      return "hsa_signal_create failed";
    std::string err;
    int64_t issued = 0;
    for (const Copy& c : job.copies) {
      if (api->async_copy(c.dst, dst_agent, c.src, src_agent, c.len, 0, nullptr, sig) !=
          HSA_STATUS_SUCCESS) {
        err = "hsa_amd_memory_async_copy failed";
        break;
      }
      ++issued;
    }
    // Wait for the issued copies. Blocked waits with a 2 ms hint, so that a
    // completion whose interrupt is missed is still seen within 2 ms.
    const hsa_signal_value_t target = total - issued;
    const uint64_t hint = api->ticks_per_s / 500;
    const auto t0 = std::chrono::steady_clock::now();
    hsa_signal_value_t v;
    for (;;) {
      v = api->signal_wait(sig, HSA_SIGNAL_CONDITION_LT, target + 1, hint,
                           HSA_WAIT_STATE_BLOCKED);
      pending.store(v - target);
      if (v <= target) break;
      if (std::chrono::steady_clock::now() - t0 > kHostWait) {
        // the engines may still write: keep the signal, fail the lane
        broken.store(true);
        std::snprintf(msg, sizeof msg, "job %llu: %lld of %lld copies still pending after %lld s",
                      static_cast<unsigned long long>(job.seq), static_cast<long long>(v - target),
                      static_cast<long long>(total), static_cast<long long>(kHostWait.count()));
        return msg;
      }
    }
    if (v < 0 && err.empty()) err = "a DMA copy reported an error";
    api->signal_destroy(sig);
    pending.store(0);
    return err;
  }
};

// A device's HSA agents.
struct DeviceInfo {
  Api* api = nullptr;
  hsa_agent_t gpu{0}, cpu{0};
};

std::mutex g_dev_mu;
std::map<int, DeviceInfo*> g_dev;                                   // lives until exit
std::map<std::tuple<int, int, uintptr_t>, Lane*> g_lanes;           // lives until exit

// Under g_dev_mu.
int device_info(int dev, DeviceInfo** out) {
  auto it = g_dev.find(dev);
  if (it != g_dev.end()) {
    *out = it->second;
    return 0;
  }
  Api* api = nullptr;
  int rc = load_api(&api);
  if (rc) return rc;
  int bus = 0, slot = 0, domain = 0;
  if (hipDeviceGetAttribute(&bus, hipDeviceAttributePciBusId, dev) != hipSuccess ||
      hipDeviceGetAttribute(&slot, hipDeviceAttributePciDeviceId, dev) != hipSuccess ||
      hipDeviceGetAttribute(&domain, hipDeviceAttributePciDomainID, dev) != hipSuccess)
    return fail(AEGKV_EINVAL, "device %d has no PCI address", dev);
  Agents ag;
  ag.api = api;
  ag.bdfid = (static_cast<uint32_t>(bus) << 8) | (static_cast<uint32_t>(slot) << 3);
  ag.domain = static_cast<uint32_t>(domain);
  api->iterate_agents(visit_agent, &ag);
  if (!ag.found || ag.cpus.empty())
    return fail(AEGKV_EINVAL, "no HSA agents for device %d (PCI %x:%x)", dev, bus, slot);
  hsa_agent_t cpu = ag.cpus.front();
  hsa_agent_t near_cpu{0};
  if (api->agent_get_info(ag.gpu, static_cast<hsa_agent_info_t>(HSA_AMD_AGENT_INFO_NEAREST_CPU),
                          &near_cpu) == HSA_STATUS_SUCCESS && near_cpu.handle)
    cpu = near_cpu;
  auto* d = new DeviceInfo();
  d->api = api;
  d->gpu = ag.gpu;
  d->cpu = cpu;
  g_dev[dev] = d;
  *out = d;
  return 0;
}

// Under g_dev_mu.
int make_lane(int dev, int dir, DeviceInfo* d, Lane** out) {
  void* p = nullptr;
  const size_t words = 8 + kStartSlots;  // done word on its own 64 B line, then the slots
  if (hipHostMalloc(&p, words * sizeof(uint64_t),
                    hipHostMallocMapped | hipHostMallocPortable | hipHostMallocCoherent) !=
      hipSuccess) {
    (void)hipGetLastError();
    return fail(AEGKV_EINVAL, "cannot allocate the SDMA lane words");
  }
  std::memset(p, 0, words * sizeof(uint64_t));
  auto* l = new Lane();  // lives until the process ends (its thread never stops)
  l->dir = dir;
  l->device = dev;
  l->api = d->api;
  l->dst_agent = dir == DIR_TO_HOST ? d->cpu : d->gpu;
  l->src_agent = dir == DIR_TO_HOST ? d->gpu : d->cpu;
  l->done = static_cast<uint64_t*>(p);
  l->slots = l->done + 8;
  std::thread([l] { l->run(); }).detach();
  *out = l;
  return 0;
}

// Host-function wait: the stream goes on once the lane's done word reaches
// the value, or after the wait budget (then the flag is set).
struct HostWait {
  const uint64_t* done;
  uint64_t value;
  uint64_t* timed_out;
  const Lane* lane;
};

std::mutex g_late_mu;
std::string g_late;  // what the last wait that ran out of time waited for

void host_wait(void* data) {
  HostWait* w = static_cast<HostWait*>(data);
  const auto t0 = std::chrono::steady_clock::now();
  for (int spins = 0; __atomic_load_n(w->done, __ATOMIC_ACQUIRE) < w->value; ++spins) {
    if (spins < 4096) {
      std::this_thread::yield();
      continue;
    }
    const auto waited = std::chrono::steady_clock::now() - t0;
    if (waited > kHostWait) {
      char buf[200];
      std::snprintf(buf, sizeof buf,
                    "a %s wait for job %llu gave up after %.1f s with the done word at %llu",
                    w->lane->dir == DIR_TO_HOST ? "to-host" : "to-device",
                    static_cast<unsigned long long>(w->value),
                    std::chrono::duration<double>(waited).count(),
                    static_cast<unsigned long long>(__atomic_load_n(w->done, __ATOMIC_ACQUIRE)));
      {
        std::lock_guard<std::mutex> lk(g_late_mu);
        g_late = buf;
      }
      __atomic_store_n(w->timed_out, uint64_t(1), __ATOMIC_RELEASE);
      break;
    }
    std::this_thread::sleep_for(std::chrono::microseconds(20));
  }
  delete w;
}

const char* stage_name(int s) {
  switch (s) {
    case IDLE: return "idle";
    case WAIT_START: return "waiting for the start slot";
    case COPYING: return "waiting for copies";
    default: return "failed";
  }
}

}  // namespace

int lane_for(int device, int dir, hipStream_t stream, LaneRef* out) {
  Lane* l = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_dev_mu);
    const auto key = std::make_tuple(device, dir, reinterpret_cast<uintptr_t>(stream));
    auto it = g_lanes.find(key);
    if (it != g_lanes.end()) {
      l = it->second;
    } else {
      DeviceInfo* d = nullptr;
      int rc = device_info(device, &d);
      if (!rc) rc = make_lane(device, dir, d, &l);
      if (rc) return rc;
      g_lanes[key] = l;
    }
  }
  {
    std::lock_guard<std::mutex> lk(l->mu);
    if (l->broken.load())
      return fail(AEGKV_EINVAL, "SDMA copies of device %d were left pending: %s", device,
                  l->error.empty() ? "(reported before)" : l->error.c_str());
    if (!l->error.empty()) {
      std::string e;
      e.swap(l->error);
      return fail(AEGKV_EINVAL, "an earlier SDMA transfer failed: %s", e.c_str());
    }
  }
  out->lane = l;
  out->slots = l->slots;
  out->slot_count = kStartSlots;
  return 0;
}

int submit(const LaneRef& ref, const CopyList& copies, uint64_t* seq) {
  Lane& l = *static_cast<Lane*>(ref.lane);
  Job job;
  job.copies.reserve(copies.size());
  for (const CopyRun& c : copies) job.copies.push_back({c.dst, c.src, c.len});
  {
    std::unique_lock<std::mutex> lk(l.mu);
    // Every queued job's start store is already enqueued on the lane's
    // stream, so the lane finishes them without help from this thread.
    if (!l.cv_space.wait_for(lk, kHostWait + std::chrono::seconds(5),
                             [&] { return l.submitted - l.finished < kStartSlots - 1; }))
      return fail(AEGKV_EINVAL, "SDMA lane of device %d made no progress for %lld s", l.device,
                  static_cast<long long>(kHostWait.count()));
    job.seq = ++l.submitted;
    *seq = job.seq;
    l.jobs.push_back(std::move(job));
  }
  l.cv.notify_one();
  return 0;
}

void abandon(const LaneRef& ref, uint64_t seq) {
  Lane& l = *static_cast<Lane*>(ref.lane);
  {
    std::lock_guard<std::mutex> lk(l.mu);
    if (seq <= l.finished) return;
    l.abandoned.insert(seq);
  }
  __atomic_store_n(l.slots + seq % kStartSlots, seq, __ATOMIC_RELEASE);
}

hipError_t enqueue_wait(const LaneRef& ref, uint64_t seq, uint64_t* timed_out,
                        hipStream_t stream) {
  const Lane* l = static_cast<const Lane*>(ref.lane);
  auto* w = new HostWait{l->done, seq, timed_out, l};
  hipError_t e = hipLaunchHostFunc(stream, host_wait, w);
  if (e != hipSuccess) delete w;
  return e;
}

std::string describe(int device) {
  std::vector<Lane*> lanes;
  {
    std::lock_guard<std::mutex> lk(g_dev_mu);
    for (const auto& kv : g_lanes)
      if (std::get<0>(kv.first) == device) lanes.push_back(kv.second);
  }
  std::string out;
  {
    std::lock_guard<std::mutex> lk(g_late_mu);
    if (!g_late.empty()) out = g_late + "; ";
  }
  if (lanes.empty()) return out + "no SDMA lanes";
  for (Lane* lp : lanes) {
    Lane& l = *lp;
    uint64_t submitted, finished;
    std::string error;
    {
      std::lock_guard<std::mutex> lk(l.mu);
      submitted = l.submitted;
      finished = l.finished;
      error = l.error;
    }
    char buf[256];
    std::snprintf(buf, sizeof buf,
                  "%s%s lane%s: %s (job %llu; jobs submitted %llu, finished %llu; done word %llu; "
                  "%lld copies pending)",
                  out.empty() ? "" : "; ", l.dir == DIR_TO_HOST ? "to-host" : "to-device",
                  l.broken.load() ? " (broken)" : "",
                  stage_name(l.stage.load()), static_cast<unsigned long long>(l.current.load()),
                  static_cast<unsigned long long>(submitted),
                  static_cast<unsigned long long>(finished),
                  static_cast<unsigned long long>(__atomic_load_n(l.done, __ATOMIC_ACQUIRE)),
                  static_cast<long long>(l.pending.load()));
    out += buf;
    if (!error.empty()) out += " error: " + error;
  }
  return out;
}

}  // namespace aegkv_sdma
