// Error reporting and per-(device, stream) scratch memory.
#include <hip/hip_runtime.h>

#include <cstring>
#include <map>
#include <vector>
#include <mutex>
#include <string>
#include <utility>

#include "common.h"

namespace dr {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

static std::mutex g_mu;
static std::map<std::pair<int, hipStream_t>, Scratch*> g_scratch;
static thread_local int g_scratch_fail = DR_ERR_HIP;

int scratch_fail() { return g_scratch_fail; }

uint64_t stream_capture_id(hipStream_t stream) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  unsigned long long id = 0;
  if (hipStreamGetCaptureInfo(stream, &st, &id) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return st == hipStreamCaptureStatusActive ? (uint64_t)id | (1ull << 63) : 0;
}

static void capture_refused(const char* what) {
  g_scratch_fail = DR_ERR_CAPTURE;
  set_error(std::string(what) +
            " while the stream is being captured into a HIP graph: run the same call once on "
            "this stream before capturing (or size the rasterizer with dr_rasterize_reserve)");
}

Scratch* scratch_for(hipStream_t stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    set_error("hipGetDevice failed");
    g_scratch_fail = DR_ERR_HIP;
    return nullptr;
  }
  const uint64_t cap = stream_capture_id(stream);
  std::lock_guard<std::mutex> lk(g_mu);
  auto key = std::make_pair(dev, stream);
  auto it = g_scratch.find(key);
  if (it != g_scratch.end()) {
    it->second->cur_capture = cap;
    if (cap) it->second->captured = true;
    return it->second;
  }
  if (cap) {  // the pinned counters below would be allocated
    capture_refused("the library's first call on a stream allocates its scratch");
    return nullptr;
  }
  g_scratch_fail = DR_ERR_HIP;
  Scratch* sc = new Scratch();
  if (hipHostMalloc((void**)&sc->pinned_total, 2 * sizeof(int64_t), hipHostMallocDefault) != hipSuccess ||
      hipHostGetDevicePointer((void**)&sc->pinned_total_dev, sc->pinned_total, 0) != hipSuccess ||
      hipHostMalloc((void**)&sc->wave_stats, 2 * Scratch::kWaveStatsMax * sizeof(int64_t),
                    hipHostMallocDefault) != hipSuccess ||
      hipHostGetDevicePointer((void**)&sc->wave_stats_dev, sc->wave_stats, 0) != hipSuccess ||
      hipEventCreateWithFlags(&sc->total_event, hipEventDisableTiming) != hipSuccess) {
    set_error("scratch: pinned counter / event allocation failed");
    if (sc->pinned_total) (void)hipHostFree(sc->pinned_total);
    if (sc->wave_stats) (void)hipHostFree(sc->wave_stats);
    delete sc;
    return nullptr;
  }
  sc->pinned_total[0] = sc->pinned_total[1] = 0;
  g_scratch[key] = sc;
  return sc;
}

void* scratch_get(Scratch* sc, hipStream_t stream, int s, size_t bytes) {
  if (bytes == 0) bytes = 256;
  if (sc->cap[s] >= bytes) return sc->ptr[s];
  if (sc->cur_capture) {
    capture_refused(("scratch slot " + std::to_string(s) + " would grow to " +
                     std::to_string(bytes) + " bytes").c_str());
    return nullptr;
  }
  g_scratch_fail = DR_ERR_MEMORY;
  // Grow: the old buffer may still be read by queued work on this stream,
  // or by a graph captured on it (then it is kept until dr_release_scratch).
  if (sc->ptr[s]) {
    if (sc->captured) {
      sc->retired.push_back(sc->ptr[s]);
    } else {
      if (hipStreamSynchronize(stream) != hipSuccess) {
        set_error("scratch: stream synchronize failed");
        return nullptr;
      }
      (void)hipFree(sc->ptr[s]);
    }
    sc->ptr[s] = nullptr;
    sc->cap[s] = 0;
  }
  size_t want = bytes + bytes / 4;
  want = (want + 4095) & ~(size_t)4095;
  void* p = nullptr;
  if (hipMalloc(&p, want) != hipSuccess) {
    (void)hipGetLastError();
    set_error("scratch: hipMalloc of " + std::to_string(want) + " bytes failed");
    return nullptr;
  }
  sc->ptr[s] = p;
  sc->cap[s] = want;
  return p;
}

int64_t* stage_acquire(Scratch* sc, size_t n, int& slot) {
  if (sc->cur_capture) {  // a replay would copy whatever the buffer then holds
    capture_refused("range mode stages its ranges through host memory");
    return nullptr;
  }
  g_scratch_fail = DR_ERR_HIP;
  slot = sc->stage_next;
  sc->stage_next = (sc->stage_next + 1) % Scratch::kStageRing;
  if (sc->stage_pending[slot]) {
    if (hipEventSynchronize(sc->stage_event[slot]) != hipSuccess) {
      set_error("range staging: event synchronize failed");
      return nullptr;
    }
    sc->stage_pending[slot] = false;
  }
  if (!sc->stage_event[slot] &&
      hipEventCreateWithFlags(&sc->stage_event[slot], hipEventDisableTiming) != hipSuccess) {
    set_error("range staging: event creation failed");
    return nullptr;
  }
  if (sc->stage_cap[slot] < n) {
    // Pinned allocations may wait for the device: grow this buffer and every
    // idle one that is also too small now, so that later calls of the same
    // size allocate nothing (a buffer a queued copy may still read keeps
    // its size until it is acquired).
    const size_t want = n + n / 4 + 64;
    for (int r = 0; r < Scratch::kStageRing; ++r)  // copies that have run free their buffers
      if (sc->stage_pending[r] && hipEventQuery(sc->stage_event[r]) == hipSuccess)
        sc->stage_pending[r] = false;
    (void)hipGetLastError();  // hipErrorNotReady of the queries
    for (int r = 0; r < Scratch::kStageRing; ++r) {
      if (r != slot && (sc->stage_pending[r] || sc->stage_cap[r] >= n)) continue;
      if (sc->stage[r]) (void)hipHostFree(sc->stage[r]);
      sc->stage[r] = nullptr;
      sc->stage_cap[r] = 0;
      if (hipHostMalloc((void**)&sc->stage[r], want * sizeof(int64_t), hipHostMallocDefault) !=
          hipSuccess) {
        (void)hipGetLastError();
        if (r != slot) continue;  // only the acquired buffer must exist now
        set_error("range staging: pinned allocation failed");
        return nullptr;
      }
      sc->stage_cap[r] = want;
    }
  }
  return sc->stage[slot];
}

int stage_release(Scratch* sc, int slot, hipStream_t stream) {
  if (hipEventRecord(sc->stage_event[slot], stream) != hipSuccess) {
    set_error("range staging: event record failed");
    return DR_ERR_HIP;
  }
  sc->stage_pending[slot] = true;
  return DR_OK;
}

int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cu = 0;
    if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cu <= 0)
      cu = 256;
    cached[dev] = cu;
  }
  return cached[dev];
}

// ---- kernel timing -------------------------------------------------------

bool g_prof_enabled = false;
static std::string g_prof_only;  // empty: time every kernel

struct ProfRec {
  const char* name;
  hipEvent_t a, b;
};

static std::mutex g_prof_mu;
static std::vector<ProfRec> g_prof;
static std::vector<hipEvent_t> g_prof_pool;

static hipEvent_t prof_event() {
  if (!g_prof_pool.empty()) {
    hipEvent_t e = g_prof_pool.back();
    g_prof_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

ProfScope::ProfScope(const char* n, hipStream_t s) : name(n), stream(s) {
  if (!g_prof_enabled) return;
  if (!g_prof_only.empty() && g_prof_only != n) return;
  std::lock_guard<std::mutex> lk(g_prof_mu);
  start = prof_event();
  if (start) (void)hipEventRecord(start, stream);
}

ProfScope::~ProfScope() {
  if (!start) return;
  std::lock_guard<std::mutex> lk(g_prof_mu);
  hipEvent_t end = prof_event();
  if (!end) return;
  (void)hipEventRecord(end, stream);
  g_prof.push_back({name, start, end});
}

}  // namespace dr

extern "C" {

int dr_profile_enable(int on) {
  dr::g_prof_enabled = on != 0;
  return DR_OK;
}

int dr_profile_select(const char* kernel) {
  std::lock_guard<std::mutex> lk(dr::g_prof_mu);
  dr::g_prof_only = kernel ? kernel : "";
  return DR_OK;
}

int dr_profile_reset(void) {
  std::lock_guard<std::mutex> lk(dr::g_prof_mu);
  for (auto& r : dr::g_prof) {
    (void)hipEventSynchronize(r.b);
    dr::g_prof_pool.push_back(r.a);
    dr::g_prof_pool.push_back(r.b);
  }
  dr::g_prof.clear();
  // events for the next 1,024 timed launches are created here, outside the
  // measured loop (hipEventCreate costs tens of microseconds, as much as a
  // small workload's whole step)
  while (dr::g_prof_pool.size() < 2048) {
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) break;
    dr::g_prof_pool.push_back(e);
  }
  return DR_OK;
}

int dr_profile_report(char* buf, int len) {
  std::lock_guard<std::mutex> lk(dr::g_prof_mu);
  std::map<std::string, std::pair<long, double>> agg;
  for (auto& r : dr::g_prof) {
    float ms = 0.0f;
    if (hipEventSynchronize(r.b) != hipSuccess) return -1;
    if (hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess) return -1;
    auto& e = agg[r.name];
    e.first += 1;
    e.second += ms;
  }
  std::string out;
  for (auto& kv : agg)
    out += kv.first + " " + std::to_string(kv.second.first) + " " +
           std::to_string(kv.second.second) + "\n";
  if (buf && len > 0) {
    size_t n = out.size() < (size_t)(len - 1) ? out.size() : (size_t)(len - 1);
    memcpy(buf, out.data(), n);
    buf[n] = 0;
  }
  return (int)out.size();
}

int dr_abi_version(void) { return DR_ABI_VERSION; }

const char* dr_get_last_error(void) { return dr::g_last_error.c_str(); }

int dr_release_scratch(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return DR_ERR_HIP;
  std::lock_guard<std::mutex> lk(dr::g_mu);
  for (auto it = dr::g_scratch.begin(); it != dr::g_scratch.end();) {
    if (it->first.first != dev) {
      ++it;
      continue;
    }
    dr::Scratch* sc = it->second;
    (void)hipStreamSynchronize(it->first.second);
    for (int s = 0; s < dr::SLOT_COUNT; ++s)
      if (sc->ptr[s]) (void)hipFree(sc->ptr[s]);
    for (void* p : sc->retired) (void)hipFree(p);
    if (sc->pinned_total) (void)hipHostFree(sc->pinned_total);
    if (sc->wave_stats) (void)hipHostFree(sc->wave_stats);
    if (sc->total_event) (void)hipEventDestroy(sc->total_event);
    for (int r = 0; r < dr::Scratch::kStageRing; ++r) {
      if (sc->stage_event[r]) (void)hipEventDestroy(sc->stage_event[r]);
      if (sc->stage[r]) (void)hipHostFree(sc->stage[r]);
    }
    delete sc;
    it = dr::g_scratch.erase(it);
  }
  return DR_OK;
}

}  // extern "C"
