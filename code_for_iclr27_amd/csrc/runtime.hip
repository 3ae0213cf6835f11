// Error state, ABI version and host-memory registration (module lazy_recall._host,
// csrc/host.cpp:5-13 in the reference).
#include "lr_common.hpp"

namespace lr {
namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& message) { g_last_error = message; }
void clear_error() { g_last_error.clear(); }

int check_launch(const char* what) {
  const hipError_t status = hipGetLastError();
  if (status != hipSuccess) {
    set_error(std::string(what) + " launch failed: " + hipGetErrorString(status));
    return LR_ERR_HIP;
  }
  return LR_OK;
}

}  // namespace lr

extern "C" const char* lr_last_error(void) { return lr::g_last_error.c_str(); }

extern "C" int lr_abi_version(void) { return 1; }

extern "C" int lr_register_host(uint64_t address, uint64_t bytes) {
  lr::clear_error();
  LR_REQUIRE(address != 0 && bytes != 0, "hipHostRegister failed: empty range");
  const hipError_t status =
      hipHostRegister(reinterpret_cast<void*>(address), bytes, hipHostRegisterDefault);
  if (status != hipSuccess) {
    (void)hipGetLastError();  // do not leave a sticky error for the caller's next HIP call
    lr::set_error(std::string("hipHostRegister failed: ") + hipGetErrorString(status));
    return LR_ERR_HIP;
  }
  return LR_OK;
}

extern "C" int lr_unregister_host(uint64_t address) {
  lr::clear_error();
  LR_REQUIRE(address != 0, "hipHostUnregister failed: null address");
  const hipError_t status = hipHostUnregister(reinterpret_cast<void*>(address));
  if (status != hipSuccess) {
    (void)hipGetLastError();
    lr::set_error(std::string("hipHostUnregister failed: ") + hipGetErrorString(status));
    return LR_ERR_HIP;
  }
  return LR_OK;
}
