// Greedy sampling on the device: the index of each logits row's maximum, with NumPy's argmax
// rules (ties resolve to the lowest index; a NaN beats every number and the first NaN wins), so
// only one int32 per row crosses PCIe instead of the whole vocabulary row.
#include <math.h>

#include "pkv_common.h"

namespace pkv {
namespace {

constexpr int kArgmaxThreads = 256;
constexpr int kArgmaxWaves = kArgmaxThreads / kWave;

// A candidate (value, index); index -1 marks "no element seen".
struct Best {
  float value;
  int64_t index;
};

// True when candidate a is argmax-preferred over candidate b.
__device__ __forceinline__ bool beats(const Best& a, const Best& b) {
  if (a.index < 0) return false;
  if (b.index < 0) return true;
  const bool an = isnan(a.value);
  const bool bn = isnan(b.value);
  if (an != bn) return an;
  if (!an && a.value != b.value) return a.value > b.value;
  return a.index < b.index;  // equal values (or both NaN): the lower index
}

__device__ __forceinline__ Best shfl_xor_best(const Best& b, int mask) {
  Best o;
  o.value = __shfl_xor(b.value, mask);
  o.index = __shfl_xor(b.index, mask);
  return o;
}

// One workgroup per row. Thread t scans elements t, t + 256, ... (in increasing order, so within
// a thread a later element only wins by being strictly greater, or by being the first NaN).
template <bool kVec4>
__global__ __launch_bounds__(kArgmaxThreads) void greedy_kernel(int32_t* __restrict__ out,
                                                                const float* __restrict__ logits,
                                                                int64_t row_stride,
                                                                int64_t vocab) {
  const int64_t row = blockIdx.x;
  const float* x = logits + row * row_stride;
  Best best{0.f, -1};
  auto consider = [&](float v, int64_t i) {
    if (best.index < 0 || (isnan(v) && !isnan(best.value)) || v > best.value) best = Best{v, i};
  };
  if constexpr (kVec4) {
    const int64_t quads = vocab / 4;
    for (int64_t q = threadIdx.x; q < quads; q += kArgmaxThreads) {
      const float4 v = reinterpret_cast<const float4*>(x)[q];
      consider(v.x, 4 * q);
      consider(v.y, 4 * q + 1);
      consider(v.z, 4 * q + 2);
      consider(v.w, 4 * q + 3);
    }
    // The tail (vocab % 4 elements) comes after every quad, so it is merged, not scanned.
    for (int64_t i = quads * 4 + threadIdx.x; i < vocab; i += kArgmaxThreads) {
      const Best tail{x[i], i};
      if (beats(tail, best)) best = tail;
    }
  } else {
    for (int64_t i = threadIdx.x; i < vocab; i += kArgmaxThreads) consider(x[i], i);
  }
  // Merge within the wavefront, then across the wavefronts through LDS.
#pragma unroll
  for (int mask = kWave / 2; mask > 0; mask >>= 1) {
    const Best other = shfl_xor_best(best, mask);
    if (beats(other, best)) best = other;
  }
  __shared__ float s_value[kArgmaxWaves];
  __shared__ int64_t s_index[kArgmaxWaves];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  if (lane == 0) {
    s_value[wave] = best.value;
    s_index[wave] = best.index;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    Best total{s_value[0], s_index[0]};
    for (int w = 1; w < kArgmaxWaves; ++w) {
      const Best other{s_value[w], s_index[w]};
      if (beats(other, total)) total = other;
    }
    out[row] = static_cast<int32_t>(total.index);
  }
}

}  // namespace
}  // namespace pkv

extern "C" int pkv_greedy_tokens(int32_t* token_ids, const float* logits, int64_t row_stride,
                                 int64_t num_rows, int64_t vocab_size, int device,
                                 void* stream) {
  using namespace pkv;
  if (num_rows < 0 || vocab_size < 1 || vocab_size > 0x7fffffff || row_stride < vocab_size) {
    return PKV_EINVAL;
  }
  if (num_rows == 0) return PKV_OK;
  if (!token_ids || !logits) return PKV_EINVAL;
  if (num_rows > 0x7fffffff) return PKV_EUNSUPPORTED;
  DeviceGuard guard(device);
  if (!guard.ok()) return PKV_EHIP;
  const dim3 grid(static_cast<uint32_t>(num_rows));
  auto s = static_cast<hipStream_t>(stream);
  if (row_stride % 4 == 0 && aligned16(logits)) {
    hipLaunchKernelGGL((greedy_kernel<true>), grid, dim3(kArgmaxThreads), 0, s, token_ids, logits,
                       row_stride, vocab_size);
  } else {
    hipLaunchKernelGGL((greedy_kernel<false>), grid, dim3(kArgmaxThreads), 0, s, token_ids,
                       logits, row_stride, vocab_size);
  }
  return check_launch();
}
