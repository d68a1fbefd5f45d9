#include "sdma_engines.h"

#include <hip/hip_runtime_api.h>

#include <string>

namespace kvx {
namespace {

struct AgentSearch {
  uint32_t domain = 0;
  uint32_t bus = 0;
  uint32_t dev = 0;
  hsa_agent_t gpu{};
  hsa_agent_t cpu{};
  bool gpu_found = false;
  bool cpu_found = false;
};

hsa_status_t VisitAgent(hsa_agent_t agent, void* data) {
  AgentSearch* s = static_cast<AgentSearch*>(data);
  hsa_device_type_t type;
  if (hsa_agent_get_info(agent, HSA_AGENT_INFO_DEVICE, &type) != HSA_STATUS_SUCCESS) {
    return HSA_STATUS_SUCCESS;
  }
  if (type == HSA_DEVICE_TYPE_CPU && !s->cpu_found) {
    s->cpu = agent;
    s->cpu_found = true;
  } else if (type == HSA_DEVICE_TYPE_GPU && !s->gpu_found) {
    // Location ID: bus << 8 | device << 3 | function.
    uint32_t bdf = 0, domain = 0;
    if (hsa_agent_get_info(agent, static_cast<hsa_agent_info_t>(HSA_AMD_AGENT_INFO_BDFID),
                           &bdf) == HSA_STATUS_SUCCESS &&
        hsa_agent_get_info(agent, static_cast<hsa_agent_info_t>(HSA_AMD_AGENT_INFO_DOMAIN),
                           &domain) == HSA_STATUS_SUCCESS &&
        domain == s->domain && (bdf >> 8) == s->bus && ((bdf >> 3) & 0x1f) == s->dev) {
      s->gpu = agent;
      s->gpu_found = true;
    }
  }
  return HSA_STATUS_SUCCESS;
}

Status HsaStatus(hsa_status_t st, const char* what) {
  if (st == HSA_STATUS_SUCCESS) return OkStatus();
  const char* msg = nullptr;
  hsa_status_string(st, &msg);
  return InternalError(std::string(what) + ": " + (msg != nullptr ? msg : "HSA error"));
}

// Lowest set bit of `mask` (0 if none).
uint32_t LowestBit(uint32_t mask) { return mask & (~mask + 1); }

}  // namespace

StatusOr<std::unique_ptr<SdmaEngines>> SdmaEngines::Create(int device) {
  int domain = 0, bus = 0, dev = 0;
  if (hipDeviceGetAttribute(&domain, hipDeviceAttributePciDomainId, device) != hipSuccess ||
      hipDeviceGetAttribute(&bus, hipDeviceAttributePciBusId, device) != hipSuccess ||
      hipDeviceGetAttribute(&dev, hipDeviceAttributePciDeviceId, device) != hipSuccess) {
    return FailedPreconditionError("PCI location of the device unknown");
  }
  // The HIP runtime has initialised ROCr already; this takes a reference,
  // which the object gives back.
  KVX_RETURN_IF_ERROR(HsaStatus(hsa_init(), "hsa_init"));
  std::unique_ptr<SdmaEngines> e(new SdmaEngines());
  e->hsa_ref_ = true;
  AgentSearch s;
  s.domain = static_cast<uint32_t>(domain);
  s.bus = static_cast<uint32_t>(bus);
  s.dev = static_cast<uint32_t>(dev);
  KVX_RETURN_IF_ERROR(HsaStatus(hsa_iterate_agents(VisitAgent, &s), "hsa_iterate_agents"));
  if (!s.gpu_found || !s.cpu_found) {
    return NotFoundError("no ROCr agent at the device's PCI location");
  }
  e->gpu_ = s.gpu;
  // The host side of the copies: the CPU agent nearest the device when ROCr
  // names one (the first CPU agent otherwise).
  hsa_agent_t nearest{};
  e->cpu_ = hsa_agent_get_info(s.gpu, static_cast<hsa_agent_info_t>(HSA_AMD_AGENT_INFO_NEAREST_CPU),
                               &nearest) == HSA_STATUS_SUCCESS && nearest.handle != 0
                ? nearest
                : s.cpu;
  uint32_t avail_h2d = 0, avail_d2h = 0, pref_h2d = 0, pref_d2h = 0;
  KVX_RETURN_IF_ERROR(HsaStatus(hsa_amd_memory_copy_engine_status(e->gpu_, e->cpu_, &avail_h2d),
                                "copy engine status (host to device)"));
  KVX_RETURN_IF_ERROR(HsaStatus(hsa_amd_memory_copy_engine_status(e->cpu_, e->gpu_, &avail_d2h),
                                "copy engine status (device to host)"));
  // Preferences are hints (0: none); an engine must be available.
  (void)hsa_amd_memory_get_preferred_copy_engine(e->gpu_, e->cpu_, &pref_h2d);
  (void)hsa_amd_memory_get_preferred_copy_engine(e->cpu_, e->gpu_, &pref_d2h);
  const uint32_t h2d = LowestBit((pref_h2d & avail_h2d) != 0 ? (pref_h2d & avail_h2d) : avail_h2d);
  uint32_t d2h = LowestBit(pref_d2h & avail_d2h & ~h2d);
  if (d2h == 0) d2h = LowestBit(avail_d2h & ~h2d);
  if (d2h == 0) d2h = LowestBit(avail_d2h);  // one engine: both directions share it
  if (h2d == 0 || d2h == 0) return UnavailableError("no SDMA engine for host copies");
  e->h2d_engine_ = h2d;
  e->d2h_engine_ = d2h;
  return e;
}

SdmaEngines::~SdmaEngines() {
  if (hsa_ref_) (void)hsa_shut_down();
}

Status SdmaEngines::Start(bool d2h, void* dst, const void* src, size_t bytes,
                          hsa_signal_t done) const {
  hsa_signal_store_screlease(done, 1);
  const hsa_status_t st = hsa_amd_memory_async_copy_on_engine(
      dst, d2h ? cpu_ : gpu_, src, d2h ? gpu_ : cpu_, bytes, 0, nullptr, done,
      static_cast<hsa_amd_sdma_engine_id_t>(d2h ? d2h_engine_ : h2d_engine_),
      /*force_copy_on_sdma=*/true);
  // A copy that was not started never lowers the signal: leave it as a
  // finished one, so that waits on it return.
  if (st != HSA_STATUS_SUCCESS) hsa_signal_store_screlease(done, 0);
  return HsaStatus(st, "SDMA copy");
}

Status SdmaEngines::Wait(hsa_signal_t done) {
  hsa_signal_value_t v;
  do {
    v = hsa_signal_wait_scacquire(done, HSA_SIGNAL_CONDITION_LT, 1, UINT64_MAX,
                                  HSA_WAIT_STATE_BLOCKED);
  } while (v >= 1);
  if (v < 0) return InternalError("SDMA copy failed");
  return OkStatus();
}

StatusOr<hsa_signal_t> SdmaEngines::NewSignal() {
  hsa_signal_t s{};
  KVX_RETURN_IF_ERROR(HsaStatus(hsa_signal_create(0, 0, nullptr, &s), "hsa_signal_create"));
  return s;
}

void SdmaEngines::DestroySignal(hsa_signal_t s) {
  if (s.handle != 0) (void)hsa_signal_destroy(s);
}

}  // namespace kvx
