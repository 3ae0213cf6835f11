// Error state, ABI version, host-memory registration (module lazy_recall._host,
// csrc/host.cpp:5-13 in the reference) and the fused step's metadata staging.
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

// Pinned host memory that kernels read directly: fine-grained (coherent), so a kernel launched
// after the host wrote it reads the written words.
extern "C" int lr_staging_alloc(size_t bytes, void** host) {
  lr::clear_error();
  LR_REQUIRE(bytes > 0 && host != nullptr, "Invalid staging size");
  *host = nullptr;
  const hipError_t status = hipHostMalloc(host, bytes, hipHostMallocCoherent | hipHostMallocMapped);
  if (status != hipSuccess) {
    (void)hipGetLastError();
    *host = nullptr;
    lr::set_error(std::string("hipHostMalloc failed: ") + hipGetErrorString(status));
    return LR_ERR_HIP;
  }
  return LR_OK;
}

extern "C" int lr_staging_free(void* host) {
  lr::clear_error();
  if (host == nullptr) return LR_OK;
  const hipError_t status = hipHostFree(host);
  if (status != hipSuccess) {
    (void)hipGetLastError();
    lr::set_error(std::string("hipHostFree failed: ") + hipGetErrorString(status));
    return LR_ERR_HIP;
  }
  return LR_OK;
}

namespace lr {
namespace {
// One word per thread: every load is in flight at once (a host-memory read costs one bus round
// trip), then every store.
__global__ __launch_bounds__(256) void copy_words_kernel(const int64_t* __restrict__ source,
                                                         int64_t* __restrict__ destination,
                                                         int64_t words) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < words) destination[i] = source[i];
}

// Device-to-device copy of 16-byte granules with nontemporal loads and stores, four granules
// per thread in flight, one pass (no grid-stride loop): the form of the all-layer row kernels,
// on a plain copy.
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
constexpr int kStreamUnroll = 4;
__global__ __launch_bounds__(256) void stream_copy_kernel(const u32x4* __restrict__ source,
                                                          u32x4* __restrict__ destination,
                                                          int64_t granules) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * 256 * kStreamUnroll + threadIdx.x;
  u32x4 v[kStreamUnroll];
#pragma unroll
  for (int u = 0; u < kStreamUnroll; ++u) {
    const int64_t i = base + static_cast<int64_t>(u) * 256;
    if (i < granules) v[u] = __builtin_nontemporal_load(source + i);
  }
#pragma unroll
  for (int u = 0; u < kStreamUnroll; ++u) {
    const int64_t i = base + static_cast<int64_t>(u) * 256;
    if (i < granules) __builtin_nontemporal_store(v[u], destination + i);
  }
}
}  // namespace
}  // namespace lr

extern "C" int lr_copy_words(const int64_t* source, int64_t* destination, int64_t words,
                             void* stream) {
  lr::clear_error();
  LR_REQUIRE(words >= 0 && words < (int64_t{1} << 31), "Invalid word count");
  if (words == 0) return LR_OK;
  LR_REQUIRE(source != nullptr && destination != nullptr, "Expected non-null buffers");
  const unsigned blocks = static_cast<unsigned>((words + 255) / 256);
  lr::copy_words_kernel<<<blocks, 256, 0, lr::as_stream(stream)>>>(source, destination, words);
  return lr::check_launch("copy_words");
}

extern "C" int lr_stream_copy(const void* source, void* destination, int64_t bytes, void* stream) {
  lr::clear_error();
  LR_REQUIRE(bytes >= 0 && bytes % 16 == 0, "Copy size must be a multiple of 16 bytes");
  if (bytes == 0) return LR_OK;
  LR_REQUIRE(source != nullptr && destination != nullptr, "Expected non-null buffers");
  LR_REQUIRE((reinterpret_cast<uintptr_t>(source) & 15) == 0 &&
                 (reinterpret_cast<uintptr_t>(destination) & 15) == 0,
             "Copy buffers must be 16-byte aligned");
  const int64_t granules = bytes / 16;
  const int64_t blocks = (granules + 256 * lr::kStreamUnroll - 1) / (256 * lr::kStreamUnroll);
  LR_REQUIRE(blocks < (int64_t{1} << 31), "Copy too large");
  lr::stream_copy_kernel<<<static_cast<unsigned>(blocks), 256, 0, lr::as_stream(stream)>>>(
      static_cast<const lr::u32x4*>(source), static_cast<lr::u32x4*>(destination), granules);
  return lr::check_launch("stream_copy");
}
