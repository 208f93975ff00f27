// Format kernels (affine quantize / dequantize) and the HBM stream
// calibrator.
#include "common.h"
#include "kernels.h"

namespace rmoe {

// One thread per 64-value group.  Arithmetic is plain IEEE fp32 (correctly
// rounded division, round-half-even rint), so the result is reproducible on
// the host bit for bit.
template <int BITS>
__global__ __launch_bounds__(256) void quantize_kernel(const float* __restrict__ w,
                                                       const int64_t groups,
                                                       uint32_t* __restrict__ wq,
                                                       uint16_t* __restrict__ s_out,
                                                       uint16_t* __restrict__ b_out) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= groups) return;
  const float* src = w + g * 64;
  float v[64];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float4 f = reinterpret_cast<const float4*>(src)[i];
    v[4 * i + 0] = f.x;
    v[4 * i + 1] = f.y;
    v[4 * i + 2] = f.z;
    v[4 * i + 3] = f.w;
  }
  float w_max = v[0], w_min = v[0];
#pragma unroll
  for (int i = 1; i < 64; ++i) {
    w_max = v[i] > w_max ? v[i] : w_max;
    w_min = v[i] < w_min ? v[i] : w_min;
  }
  const float n_bins = (float)((1 << BITS) - 1);
  const bool mask = fabsf(w_min) > fabsf(w_max);
  float scale = (w_max - w_min) / n_bins;
  scale = scale > 1e-7f ? scale : 1e-7f;
  scale = mask ? scale : -scale;
  const float edge = mask ? w_min : w_max;
  const float q0 = rintf(edge / scale);
  if (q0 != 0.0f) scale = edge / q0;
  const float bias = q0 == 0.0f ? 0.0f : edge;
  const uint32_t sb = f32_to_bf16(scale);
  const uint32_t bb = f32_to_bf16(bias);
  s_out[g] = (uint16_t)sb;
  b_out[g] = (uint16_t)bb;
  const float s = bf16_to_f32(sb);
  const float b = bf16_to_f32(bb);
  constexpr int VPW = 32 / BITS;
  uint32_t* dst = wq + g * (64 / VPW);
#pragma unroll
  for (int wi = 0; wi < 64 / VPW; ++wi) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < VPW; ++j) {
      float q = rintf((v[wi * VPW + j] - b) / s);
      q = q < 0.0f ? 0.0f : (q > n_bins ? n_bins : q);
      word |= ((uint32_t)q) << (BITS * j);
    }
    dst[wi] = word;
  }
}

hipError_t launch_quantize(const float* w, int64_t rows, int cols, int bits,
                           uint32_t* wq, uint16_t* s, uint16_t* b, hipStream_t st) {
  const int64_t groups = rows * (cols / 64);
  if (groups == 0) return hipSuccess;
  const unsigned blocks = (unsigned)((groups + 255) / 256);
  if (bits == 8)
    hipLaunchKernelGGL(quantize_kernel<8>, dim3(blocks), dim3(256), 0, st, w,
                       groups, wq, s, b);
  else
    hipLaunchKernelGGL(quantize_kernel<4>, dim3(blocks), dim3(256), 0, st, w,
                       groups, wq, s, b);
  return hipGetLastError();
}

// One thread per packed word: fl32(q * s + b) with q * s exact, i.e. a
// single rounding, and optionally bf16 (round-to-nearest-even) of it.
template <int BITS>
__global__ __launch_bounds__(256) void dequantize_kernel(const QW q, const int cols,
                                                         const int64_t row_begin,
                                                         const int64_t words,
                                                         float* __restrict__ out_f32,
                                                         uint16_t* __restrict__ out_bf16) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= words) return;
  constexpr int VPW = 32 / BITS;
  const int wpr = cols / VPW;
  const int64_t r = i / wpr;
  const int wi = (int)(i - r * wpr);
  const int64_t grow = row_begin + r;
  const uint32_t word = q.w[grow * wpr + wi];
  const int grp = (wi * VPW) >> 6;
  const float s = bf16_to_f32(q.s[grow * (cols >> 6) + grp]);
  const float b = bf16_to_f32(q.b[grow * (cols >> 6) + grp]);
  const int64_t base = r * cols + (int64_t)wi * VPW;
#pragma unroll
  for (int j = 0; j < VPW; ++j) {
    const float code = (float)((word >> (BITS * j)) & ((1u << BITS) - 1u));
    const float v = fmaf(code, s, b);
    if (out_f32) out_f32[base + j] = v;
    if (out_bf16) out_bf16[base + j] = (uint16_t)f32_to_bf16(v);
  }
}

hipError_t launch_dequantize(const QW& q, int cols, int bits, int64_t row_begin,
                             int64_t rows, float* out_f32, uint16_t* out_bf16,
                             hipStream_t st) {
  const int64_t words = rows * (cols / (32 / bits));
  if (words == 0) return hipSuccess;
  const unsigned blocks = (unsigned)((words + 255) / 256);
  if (bits == 8)
    hipLaunchKernelGGL(dequantize_kernel<8>, dim3(blocks), dim3(256), 0, st, q,
                       cols, row_begin, words, out_f32, out_bf16);
  else
    hipLaunchKernelGGL(dequantize_kernel<4>, dim3(blocks), dim3(256), 0, st, q,
                       cols, row_begin, words, out_f32, out_bf16);
  return hipGetLastError();
}

// Grid-stride read of 16-byte vectors, 4 loads in flight per lane; each
// workgroup folds what it read into partials[blockIdx.x].
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ buf,
                                                          const int64_t n,
                                                          uint32_t* __restrict__ partials) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 3 * stride < n; i += 4 * stride) {
    const u32x4 a = __builtin_nontemporal_load(buf + i);
    const u32x4 b = __builtin_nontemporal_load(buf + i + stride);
    const u32x4 c = __builtin_nontemporal_load(buf + i + 2 * stride);
    const u32x4 d = __builtin_nontemporal_load(buf + i + 3 * stride);
    acc += (a.x ^ a.y ^ a.z ^ a.w) + (b.x ^ b.y ^ b.z ^ b.w) +
           (c.x ^ c.y ^ c.z ^ c.w) + (d.x ^ d.y ^ d.z ^ d.w);
  }
  for (; i < n; i += stride) {
    const u32x4 a = __builtin_nontemporal_load(buf + i);
    acc += a.x ^ a.y ^ a.z ^ a.w;
  }
  __shared__ uint32_t red[4];
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) acc += __shfl_xor(acc, d, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) partials[blockIdx.x] = red[0] + red[1] + red[2] + red[3];
}

hipError_t launch_stream_read(const void* buf, size_t bytes, uint32_t* partials,
                              int blocks, hipStream_t st) {
  hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(256), 0, st,
                     reinterpret_cast<const u32x4*>(buf), (int64_t)(bytes / 16),
                     partials);
  return hipGetLastError();
}

}  // namespace rmoe
