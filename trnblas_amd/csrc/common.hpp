// Shared helpers of the gfx950 op library: error reporting, MFMA vector types,
// XCD-aware block remapping.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <string>

#include "../../include/trnblas_hip.h"

namespace trnblas {

// Thread-local last-error message (trnblas_hip_last_error).
void set_error(const char* fmt, ...);
void clear_error();

#define TRNBLAS_CHECK_ARG(cond, ...)           \
  do {                                         \
    if (!(cond)) {                             \
      ::trnblas::set_error(__VA_ARGS__);       \
      return TRNBLAS_E_ARG;                    \
    }                                          \
  } while (0)

// After a launch: map hipGetLastError to TRNBLAS_E_LAUNCH.
int check_launch(const char* what);

// Compute units of the current device, queried once per device (256 if the
// query fails).
int device_cus();

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// MI355X: 256 CUs in 8 XCDs. Workgroups are handed to the XCDs round-robin
// (workgroup b runs on XCD b % 8), and each XCD has its own L2. This maps the
// launch order to a tile order in which each XCD works on one contiguous
// range of tiles, so tiles that share operand panels share an L2.
constexpr int kNumXcd = 8;

__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  const int q = nblocks / kNumXcd, r = nblocks % kNumXcd;
  const int x = bid % kNumXcd, i = bid / kNumXcd;
  return x * q + (x < r ? x : r) + i;
}

// Grouped tile order: `group` consecutive tile rows are walked column by
// column, so a band of A panels stays hot while B panels stream.
__device__ __forceinline__ void grouped_tile(int t, int ntm, int ntn, int group, int& tm,
                                             int& tn) {
  const int per_group = group * ntn;
  const int g = t / per_group;
  const int first = g * group;
  const int gs = (ntm - first) < group ? (ntm - first) : group;
  const int r = t - g * per_group;
  tm = first + r % gs;
  tn = r / gs;
}

// One 16-byte-per-lane LDS DMA (buffer_load_dwordx4 ... lds) issued by
// inline asm, so the compiler does not see it: it then places no wait for it
// before LDS reads of the other stage, and the kernel waits for it itself
// (`s_waitcnt vmcnt` before the barrier that publishes the stage). Lane l's
// 16 bytes at voff + soff of the resource land at lds + 16 l.
// The resource spans nrec bytes from base: a lane whose voff (the range
// check does not include soff) is at or past nrec reads zeros.
__device__ __forceinline__ void lds_dma16_asm(const void* base, const void* lds, uint32_t voff,
                                              int soff, int nrec = 0x7ffffff0) {
  const uint64_t b = (uint64_t)base;
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  r[1] = __builtin_amdgcn_readfirstlane((int)((uint32_t)(b >> 32) & 0xffffu));
  r[2] = __builtin_amdgcn_readfirstlane(nrec);
  r[3] = 0x00020000;
  const int m = __builtin_amdgcn_readfirstlane(
      (int)(uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)lds);
  // m0 (the LDS address of the DMA) is saved and restored around the load,
  // so the statement leaves every register the compiler may use as it was
  int saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %2, %3, %4 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(m), "v"(voff), "s"(r), "s"(soff)
      : "memory");
}

}  // namespace trnblas
