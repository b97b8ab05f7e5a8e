// Shared device and host helpers of the gfx950 KV-cache data path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/pkv.h"

namespace pkv {

constexpr int kWave = 64;  // CDNA wavefront width

// ---------------------------------------------------------------------------------------------
// bfloat16 <-> float32. bfloat16 is the upper half of a binary32, so widening is a shift and
// narrowing rounds the dropped 16 bits to nearest, ties to even. NaN becomes the canonical quiet
// NaN 0x7FC0 (what torch's float->bfloat16 conversion also produces).
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// ---------------------------------------------------------------------------------------------
// Sum over aligned groups of LPT lanes (LPT in {1, 2, 4, 8}) with DPP lane permutes, leaving the
// group's sum in every lane of the group. quad_perm [1,0,3,2] swaps neighbours, [2,3,0,1] swaps
// lane pairs inside a quad, and row_half_mirror reverses each 8-lane half row, which after the
// two quad steps exchanges the two quads of an 8-lane group. All lanes must be active.
// ---------------------------------------------------------------------------------------------
template <int LPT>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(LPT == 1 || LPT == 2 || LPT == 4 || LPT == 8, "group of 1, 2, 4 or 8 lanes");
  if constexpr (LPT >= 2) {
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));
  }
  if constexpr (LPT >= 4) {
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));
  }
  if constexpr (LPT >= 8) {
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false));
  }
  return x;
}

// 2^x on the hardware exponential unit (v_exp_f32). exp2(-inf) = 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------------------------

// Makes `device` current for the lifetime of the object and restores the caller's device.
class DeviceGuard {
 public:
  explicit DeviceGuard(int device) {
    ok_ = hipGetDevice(&previous_) == hipSuccess;
    if (ok_ && previous_ != device) {
      ok_ = hipSetDevice(device) == hipSuccess;
      changed_ = ok_;
    }
  }
  ~DeviceGuard() {
    if (changed_) (void)hipSetDevice(previous_);
  }
  bool ok() const { return ok_; }

 private:
  int previous_ = 0;
  bool ok_ = false;
  bool changed_ = false;
};

inline int check_launch() { return hipGetLastError() == hipSuccess ? PKV_OK : PKV_EHIP; }

inline int dtype_size(pkv_dtype t) { return t == PKV_F32 ? 4 : (t == PKV_BF16 ? 2 : 0); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace pkv
