// probe.hip -- on-box ceilings the roofline fractions are read against.
//
// The roofline denominators are MI355X's published peaks (8 TB/s HBM3E,
// 2516.6 TFLOP/s dense bf16 MFMA).  These two kernels measure what one part
// actually sustains, so a kernel's distance to its roofline splits into what
// is reachable and what is not:
//   - loom_hip_peak_hbm_read streams a buffer once with 16-byte non-temporal
//     loads, four in flight per thread, grid-stride over one workgroup of 512
//     threads per CU (the shape that read fastest, over both a 2 GiB buffer
//     and a single 134.7 MB pass, in a sweep of workgroup counts, sizes and
//     loads in flight);
//   - loom_hip_peak_mfma_bf16 runs independent v_mfma_f32_16x16x32_bf16
//     chains, eight per wave and two waves per SIMD, so the MFMA pipes never
//     wait on a result.
// Neither has a counterpart in the reference.
#include "common.h"

namespace {

__global__ void __launch_bounds__(512) hbm_read_kernel(const u32x4_t* __restrict__ p, size_t n16,
                                                       uint32_t* sink) {
  constexpr int UNR = 4;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (UNR - 1) * stride < n16; i += UNR * stride) {
    u32x4_t v[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
    for (int u = 0; u < UNR; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  for (; i < n16; i += stride) {
    const u32x4_t v = p[i];
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  // the result must look used; it is stored only in the (practically
  // impossible) case that the xor of the whole buffer matches
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

__global__ void __launch_bounds__(512) mfma_kernel(int iters, float* sink) {
  constexpr int CH = 8;   // independent accumulator chains per wave
  const u32x4_t a = u32x4_t{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u} ^ threadIdx.x;
  const u32x4_t b = u32x4_t{0x3c003c00u, 0x3c003c00u, 0x3c003c00u, 0x3c003c00u};
  f32x4_t acc[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) acc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < CH; ++c) acc[c] = mfma16(a, b, acc[c]);
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
  if (s == 1234.5f) sink[0] = s;
}

}  // namespace

extern "C" {

int loom_hip_peak_hbm_read(const void* buf, size_t bytes, void* sink, void* stream, char* err,
                           size_t errlen) {
  if (!buf || !sink || bytes < 16 || !aligned16(buf))
    return loom_fail(err, errlen, LOOM_EINVAL,
                     "peak_hbm_read: a 16-byte-aligned buffer of at least 16 bytes and a sink "
                     "are needed");
  int cus = stream_cus(static_cast<hipStream_t>(stream));   // CUs of the stream's device
  if (cus <= 0) cus = 256;
  hipLaunchKernelGGL(hbm_read_kernel, dim3((unsigned)cus), dim3(512), 0,
                     static_cast<hipStream_t>(stream), static_cast<const u32x4_t*>(buf),
                     bytes / 16, static_cast<uint32_t*>(sink));
  return loom_check_launch(err, errlen, "peak_hbm_read");
}

int loom_hip_peak_mfma_bf16(int64_t iters, void* sink, double* flop, void* stream, char* err,
                            size_t errlen) {
  if (iters <= 0 || iters > (1 << 30) || !sink)
    return loom_fail(err, errlen, LOOM_EINVAL, "peak_mfma_bf16: 1 <= iters <= 2^30 and a sink");
  int cus = stream_cus(static_cast<hipStream_t>(stream));
  if (cus <= 0) cus = 256;
  // one workgroup of eight waves per CU: two waves per SIMD
  if (flop) *flop = (double)cus * 8 * 8 * 16384.0 * (double)iters;
  hipLaunchKernelGGL(mfma_kernel, dim3((unsigned)cus), dim3(512), 0,
                     static_cast<hipStream_t>(stream), (int)iters, static_cast<float*>(sink));
  return loom_check_launch(err, errlen, "peak_mfma_bf16");
}

}  // extern "C"
