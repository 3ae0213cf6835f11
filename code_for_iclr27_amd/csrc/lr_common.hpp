// Internal helpers shared by the HIP translation units of liblazyrecall_hip.so.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/lazyrecall.h"

namespace lr {

// Per-thread last error text, exposed through lr_last_error().
void set_error(const std::string& message);
void clear_error();

// Returns LR_ERR_HIP and records the message if the last launch failed.
int check_launch(const char* what);

inline hipStream_t as_stream(void* stream) { return reinterpret_cast<hipStream_t>(stream); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Launches never exceed this many blocks in x; kernels grid-stride beyond it.
constexpr int64_t kMaxGridX = 1 << 30;

// Sliding-max pool of every segment (temporal.hip), arguments checked by the caller. With
// `clear` given, the launch also zeroes clear[0, clear_words) before any later launch on the
// stream starts.
int launch_pool(const float* scores, int64_t total, const int64_t* bounds, int64_t segments,
                int64_t max_count, int64_t width, float* out, uint32_t* clear, int clear_words,
                hipStream_t stream);

}  // namespace lr

#define LR_REQUIRE(cond, message)      \
  do {                                 \
    if (!(cond)) {                     \
      ::lr::set_error(message);        \
      return LR_ERR_INVALID;           \
    }                                  \
  } while (0)

#define LR_HIP_TRY(expr)                                                        \
  do {                                                                          \
    hipError_t status_ = (expr);                                                \
    if (status_ != hipSuccess) {                                                \
      ::lr::set_error(std::string(#expr) + ": " + hipGetErrorString(status_));  \
      return LR_ERR_HIP;                                                        \
    }                                                                           \
  } while (0)

namespace lr {

// Copy granule chosen per call: the widest of 16/8/4/2/1 bytes that divides the row size
// and the alignment of every base pointer involved.
inline int granule_for(int64_t row_bytes, std::initializer_list<const void*> pointers) {
  int g = 16;
  while (g > 1) {
    bool ok = (row_bytes % g) == 0;
    for (const void* p : pointers) ok = ok && (reinterpret_cast<uintptr_t>(p) % g) == 0;
    if (ok) break;
    g >>= 1;
  }
  return g;
}

template <int G>
struct Granule;
template <>
struct Granule<16> { using type = uint4; };
template <>
struct Granule<8> { using type = uint2; };
template <>
struct Granule<4> { using type = uint32_t; };
template <>
struct Granule<2> { using type = uint16_t; };
template <>
struct Granule<1> { using type = uint8_t; };

// Dispatches a functor templated on the copy granule.
template <typename F>
int dispatch_granule(int granule, F&& f) {
  switch (granule) {
    case 16: return f.template operator()<16>();
    case 8: return f.template operator()<8>();
    case 4: return f.template operator()<4>();
    case 2: return f.template operator()<2>();
    default: return f.template operator()<1>();
  }
}

inline bool valid_elem_bytes(int e) { return e == 2 || e == 4 || e == 8; }

// MI355X dispatches consecutive workgroups of a grid round-robin over its 8 XCDs, each with its
// own L2. This permutation of blockIdx.x gives XCD x (the blocks with blockIdx.x % 8 == x) one
// contiguous range of logical block ids, in dispatch order, so workgroups that share inputs
// (the tiles of one segment) share one L2. It is a bijection for any grid size, so results do
// not depend on the dispatch policy.
__device__ __forceinline__ unsigned xcd_local_block(unsigned block, unsigned blocks) {
  constexpr unsigned kXcds = 8;
  const unsigned xcd = block % kXcds, k = block / kXcds;
  const unsigned per = blocks / kXcds, extra = blocks % kXcds;
  return xcd * per + (xcd < extra ? xcd : extra) + k;
}

}  // namespace lr
