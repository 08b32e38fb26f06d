// Library-level entry points: version, status text, workspace error word.
#include <mutex>
#include <unordered_map>

#include "common.h"
#include "lookback.h"

namespace tssm {
uint32_t next_epoch(const void* workspace) {
  static std::mutex mu;
  static std::unordered_map<const void*, uint32_t> epochs;
  std::lock_guard<std::mutex> lock(mu);
  uint32_t& e = epochs[workspace];
  if (++e == 0) e = 1;
  return e;
}
}  // namespace tssm

extern "C" int tssm_abi_version(void) { return 1; }

extern "C" const char* tssm_strerror(int status) {
  switch (status) {
    case TSSM_OK: return "ok";
    case TSSM_ERR_NULL: return "a required pointer is NULL";
    case TSSM_ERR_SHAPE: return "invalid or inconsistent sizes";
    case TSSM_ERR_STRIDE: return "invalid stride";
    case TSSM_ERR_DTYPE: return "unsupported dtype";
    case TSSM_ERR_WORKSPACE: return "workspace missing or too small";
    case TSSM_ERR_UNSUPPORTED: return "unsupported configuration";
    case TSSM_ERR_ALIGN: return "pointer or stride not aligned for vector access";
    case TSSM_ERR_SCRATCH:
      return "problem needs more look-back words than the fixed scratch of the "
             "no-allocation entry point holds (TSSM_NOALLOC_SCRATCH_BYTES)";
    default: break;
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "unknown tssm status";
}

extern "C" int tssm_workspace_error(const void* workspace, int clear, int* error_out) {
  TSSM_CHECK(error_out, TSSM_ERR_NULL);
  if (workspace == nullptr) return tssm::noalloc_scratch_error(clear, error_out);
  const auto* hdr = reinterpret_cast<const tssm::WsHeader*>(workspace);
  uint32_t e = 0;
  hipError_t st = hipMemcpy(&e, &hdr->error, sizeof(e), hipMemcpyDeviceToHost);
  if (st != hipSuccess) return (int)st;
  *error_out = (int)e;
  if (clear && e) {
    const uint32_t z = 0;
    st = hipMemcpy(const_cast<uint32_t*>(&hdr->error), &z, sizeof(z), hipMemcpyHostToDevice);
    if (st != hipSuccess) return (int)st;
  }
  return TSSM_OK;
}

extern "C" int tssm_workspace_attach_host_flag(void* workspace, int* host_flag) {
  void* hdr = workspace;
  if (hdr == nullptr) {
    const int rc = tssm::noalloc_scratch_header(&hdr);
    if (rc != TSSM_OK) return rc;
  }
  uint64_t addr = 0;
  if (host_flag != nullptr) {
    void* dev = nullptr;
    const hipError_t st = hipHostGetDevicePointer(&dev, host_flag, 0);
    if (st != hipSuccess) return (int)st;
    addr = (uint64_t)(uintptr_t)dev;
  }
  auto* h = reinterpret_cast<tssm::WsHeader*>(hdr);
  return (int)hipMemcpy(&h->host_flag, &addr, sizeof(addr), hipMemcpyHostToDevice);
}
