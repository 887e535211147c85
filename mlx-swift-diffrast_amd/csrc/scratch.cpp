// Error reporting and per-(device, stream) scratch memory.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <string>
#include <utility>

#include "common.h"

namespace dr {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

static std::mutex g_mu;
static std::map<std::pair<int, hipStream_t>, Scratch*> g_scratch;

Scratch* scratch_for(hipStream_t stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    set_error("hipGetDevice failed");
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_mu);
  auto key = std::make_pair(dev, stream);
  auto it = g_scratch.find(key);
  if (it != g_scratch.end()) return it->second;
  Scratch* sc = new Scratch();
  if (hipHostMalloc((void**)&sc->pinned_total, sizeof(int64_t), hipHostMallocDefault) != hipSuccess ||
      hipEventCreateWithFlags(&sc->total_event, hipEventDisableTiming) != hipSuccess) {
    set_error("scratch: pinned counter / event allocation failed");
    delete sc;
    return nullptr;
  }
  *sc->pinned_total = 0;
  g_scratch[key] = sc;
  return sc;
}

void* scratch_get(Scratch* sc, hipStream_t stream, int s, size_t bytes) {
  if (bytes == 0) bytes = 256;
  if (sc->cap[s] >= bytes) return sc->ptr[s];
  // Grow: the old buffer may still be read by queued work on this stream.
  if (sc->ptr[s]) {
    if (hipStreamSynchronize(stream) != hipSuccess) {
      set_error("scratch: stream synchronize failed");
      return nullptr;
    }
    (void)hipFree(sc->ptr[s]);
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

}  // namespace dr

extern "C" {

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
    if (sc->pinned_total) (void)hipHostFree(sc->pinned_total);
    if (sc->total_event) (void)hipEventDestroy(sc->total_event);
    delete sc;
    it = dr::g_scratch.erase(it);
  }
  return DR_OK;
}

}  // extern "C"
