// The elementwise and row-wise steps of the decoder's forward pass around the KV data path, each
// one launch instead of a chain of framework kernels: RMSNorm, optionally fused with the residual
// add that precedes it, the SwiGLU gate product, and the row gather of the embedding lookup and
// of the logits rows. The matrix products are rocBLAS/hipBLASLt GEMMs.
//
// Both follow the float32 expressions of the reference model (src/paged_kv_serving/engine/
// model.py:43-51) operation by operation. Products, quotients and square roots are IEEE float32
// operations on both sides (hipcc keeps float32 division and sqrtf correctly rounded by default),
// and the sum of squares is summed in another order (a wavefront tree here, pairwise blocks in
// NumPy). The exponential is the device's expf, which, like NumPy's float32 exp, is not correctly
// rounded, so silu agrees with the reference to a few units in the last place rather than bit for
// bit; the tests hold silu_mul to a relative 1e-6 (about 8 float32 ulp) of the reference's silu
// and rms_norm to 2e-6.
#include <math.h>

#include "pkv_common.h"

namespace pkv {
namespace {

constexpr int kNormThreads = 256;
constexpr int kNormRows = kNormThreads / kWave;  // one wavefront per row
constexpr int kGateThreads = 256;

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int mask = 32; mask > 0; mask >>= 1) x += __shfl_xor(x, mask);
  return x;
}

// Row r: h = hidden[r] (+ delta[r], written back to hidden[r] when delta is given), then
// out[r] = h / sqrt(mean(h * h) + eps) * weight. Lane l handles columns l, l + 64, ... and
// writes output column j only after the whole row's sum is known, so out may be hidden itself.
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(
    float* out, int64_t out_stride, float* hidden, int64_t hidden_stride,
    const float* __restrict__ delta, int64_t delta_stride, const float* __restrict__ weight,
    int64_t num_rows, int32_t dim, float eps) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kNormRows + threadIdx.x / kWave;
  if (row >= num_rows) return;
  const int lane = threadIdx.x & (kWave - 1);
  float* h = hidden + row * hidden_stride;
  float squares = 0.f;
  if (delta != nullptr) {
    const float* d = delta + row * delta_stride;
    for (int j = lane; j < dim; j += kWave) {
      const float v = h[j] + d[j];
      h[j] = v;
      squares += v * v;
    }
  } else {
    for (int j = lane; j < dim; j += kWave) {
      const float v = h[j];
      squares += v * v;
    }
  }
  const float mean = wave_sum(squares) / static_cast<float>(dim);
  const float scale = sqrtf(mean + eps);
  float* o = out + row * out_stride;
  for (int j = lane; j < dim; j += kWave) o[j] = (h[j] / scale) * weight[j];
}

// out[r, j] = silu(gate[r, j]) * up[r, j], silu(x) = x * (1 / (1 + exp(-clip(x, -60, 60)))).
__global__ __launch_bounds__(kGateThreads) void silu_mul_kernel(float* __restrict__ out,
                                                                int64_t out_stride,
                                                                const float* __restrict__ gate,
                                                                const float* __restrict__ up,
                                                                int64_t in_stride, int64_t num_rows,
                                                                int32_t width) {
  const int64_t total = num_rows * width;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * kGateThreads + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * kGateThreads) {
    const int64_t r = e / width;
    const int64_t j = e - r * width;
    const float g = gate[r * in_stride + j];
    const float u = up[r * in_stride + j];
    const float sigmoid = 1.f / (1.f + expf(-fminf(fmaxf(g, -60.f), 60.f)));
    out[r * out_stride + j] = (g * sigmoid) * u;
  }
}

// out[r] = src[index[r]] (float32 rows of `width`), or zeros when index[r] lies outside
// [0, src_rows). One wavefront per row; kVec: 16-byte accesses (both row starts aligned).
template <bool kVec>
__global__ __launch_bounds__(kNormThreads) void gather_rows_kernel(float* __restrict__ out, int64_t out_stride,
                                                                    const float* __restrict__ src,
                                                                    int64_t src_stride,
                                                                    const int64_t* __restrict__ index,
                                                                    int64_t num_rows, int32_t width,
                                                                    int64_t src_rows) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kNormRows + threadIdx.x / kWave;
  if (row >= num_rows) return;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t at = index[row];
  const bool ok = at >= 0 && at < src_rows;
  float* o = out + row * out_stride;
  const float* s = src + (ok ? at : 0) * src_stride;
  if constexpr (kVec) {
    for (int j = 4 * lane; j < width; j += 4 * kWave) {
      const float4 v = ok ? *reinterpret_cast<const float4*>(s + j) : make_float4(0.f, 0.f, 0.f, 0.f);
      *reinterpret_cast<float4*>(o + j) = v;
    }
  } else {
    for (int j = lane; j < width; j += kWave) o[j] = ok ? s[j] : 0.f;
  }
}

}  // namespace
}  // namespace pkv

extern "C" int pkv_gather_rows(float* out, int64_t out_stride, const float* src, int64_t src_stride,
                               int64_t src_rows, const int64_t* index, int64_t num_rows, int32_t width,
                               int device, void* stream) {
  using namespace pkv;
  if (num_rows < 0 || width < 1 || src_rows < 0 || out_stride < width || src_stride < width) return PKV_EINVAL;
  if (num_rows == 0) return PKV_OK;
  if (!out || !src || !index) return PKV_EINVAL;
  const int64_t blocks = (num_rows + kNormRows - 1) / kNormRows;
  if (blocks > 0x7fffffff) return PKV_EUNSUPPORTED;
  DeviceGuard guard(device);
  if (!guard.ok()) return PKV_EHIP;
  (void)hipGetLastError();
  const bool vec = width % 4 == 0 && out_stride % 4 == 0 && src_stride % 4 == 0 && aligned16(out) && aligned16(src);
  auto s = static_cast<hipStream_t>(stream);
  if (vec) {
    hipLaunchKernelGGL(gather_rows_kernel<true>, dim3(static_cast<uint32_t>(blocks)), dim3(kNormThreads), 0, s, out,
                       out_stride, src, src_stride, index, num_rows, width, src_rows);
  } else {
    hipLaunchKernelGGL(gather_rows_kernel<false>, dim3(static_cast<uint32_t>(blocks)), dim3(kNormThreads), 0, s, out,
                       out_stride, src, src_stride, index, num_rows, width, src_rows);
  }
  return check_launch();
}

extern "C" int pkv_rms_norm(float* out, int64_t out_stride, float* hidden, int64_t hidden_stride,
                            const float* delta, int64_t delta_stride, const float* weight,
                            int64_t num_rows, int32_t dim, float eps, int device, void* stream) {
  using namespace pkv;
  if (num_rows < 0 || dim < 1 || out_stride < dim || hidden_stride < dim ||
      (delta != nullptr && delta_stride < dim) || !(eps >= 0.f)) {
    return PKV_EINVAL;
  }
  if (num_rows == 0) return PKV_OK;
  if (!out || !hidden || !weight) return PKV_EINVAL;
  const int64_t blocks = (num_rows + kNormRows - 1) / kNormRows;
  if (blocks > 0x7fffffff) return PKV_EUNSUPPORTED;
  DeviceGuard guard(device);
  if (!guard.ok()) return PKV_EHIP;
  (void)hipGetLastError();
  hipLaunchKernelGGL(rms_norm_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kNormThreads), 0,
                     static_cast<hipStream_t>(stream), out, out_stride, hidden, hidden_stride, delta,
                     delta_stride, weight, num_rows, dim, eps);
  return check_launch();
}

extern "C" int pkv_silu_mul(float* out, int64_t out_stride, const float* gate, const float* up,
                            int64_t in_stride, int64_t num_rows, int32_t width, int device,
                            void* stream) {
  using namespace pkv;
  if (num_rows < 0 || width < 1 || out_stride < width || in_stride < width) return PKV_EINVAL;
  if (num_rows == 0) return PKV_OK;
  if (!out || !gate || !up) return PKV_EINVAL;
  const int64_t total = num_rows * width;
  const int64_t wanted = (total + kGateThreads - 1) / kGateThreads;
  const uint32_t blocks = static_cast<uint32_t>(wanted < 65536 ? wanted : 65536);
  DeviceGuard guard(device);
  if (!guard.ok()) return PKV_EHIP;
  (void)hipGetLastError();
  hipLaunchKernelGGL(silu_mul_kernel, dim3(blocks), dim3(kGateThreads), 0, static_cast<hipStream_t>(stream),
                     out, out_stride, gate, up, in_stride, num_rows, width);
  return check_launch();
}
