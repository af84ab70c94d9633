// Probes for bench.py --read-probe and --mfma-probe and the bench line's
// measured_peaks (built as libcohx_probe.so, not part of the step library):
// a plain streaming read, for the HBM rate this device reaches, and
// back-to-back f16 MFMAs, for its matrix-core rate.  Every launch here is in
// bounds by construction.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

// Streaming read: thread t of the grid sums float4s i = t, t + stride, ...
// below n and writes its sum (so no load is dead); every index is in bounds.
__global__ __launch_bounds__(256) void k_probe_read(const float4 *__restrict__ src, size_t n,
                                                    float *__restrict__ out) {
  const size_t stride = (size_t)gridDim.x * 256;
  float acc = 0.0f;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
    const float4 v = src[i];
    acc += (v.x + v.y) + (v.z + v.w);
  }
  out[(size_t)blockIdx.x * 256 + threadIdx.x] = acc;
}

typedef _Float16 probe_half8 __attribute__((ext_vector_type(8)));
typedef float probe_float4 __attribute__((ext_vector_type(4)));

// Matrix-core rate: each wave runs kAcc independent v_mfma_f32_16x16x32_f16
// accumulation chains for `iters` steps on register operands, then writes one
// float per lane (so nothing is dead).
template <int kAcc>
__global__ __launch_bounds__(256) void k_probe_mfma(int iters, float *__restrict__ out) {
  probe_half8 a, b;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    a[i] = (_Float16)(0.001f * (threadIdx.x % 7 + i));
    b[i] = (_Float16)(0.002f * (threadIdx.x % 5 + i));
  }
  probe_float4 acc[kAcc];
#pragma unroll
  for (int k = 0; k < kAcc; k++) acc[k] = probe_float4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int k = 0; k < kAcc; k++) acc[k] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[k], 0, 0, 0);
  }
  float t = 0.0f;
#pragma unroll
  for (int k = 0; k < kAcc; k++) t += acc[k][0] + acc[k][1] + acc[k][2] + acc[k][3];
  out[(size_t)blockIdx.x * 256 + threadIdx.x] = t;
}

}  // namespace

// Matrix-core rate: `blocks` workgroups of 4 waves, each wave 8 chains of
// `iters` 16x16x32 f16 MFMAs (16,384 flops each); returns 0 and the kernel's
// ms (one untimed launch first).
extern "C" int cohx_probe_mfma(int blocks, int iters, float *ms) {
  if (!ms || blocks <= 0 || blocks > 65536 || iters <= 0 || iters > 1 << 20) return 2;
  float *out = nullptr;
  if (hipMalloc(&out, (size_t)blocks * 256 * sizeof(float)) != hipSuccess) return 1;
  hipEvent_t a, b;
  (void)hipEventCreate(&a);
  (void)hipEventCreate(&b);
  hipLaunchKernelGGL(k_probe_mfma<8>, dim3(blocks), dim3(256), 0, 0, iters, out);
  (void)hipEventRecord(a, 0);
  hipLaunchKernelGGL(k_probe_mfma<8>, dim3(blocks), dim3(256), 0, 0, iters, out);
  (void)hipEventRecord(b, 0);
  (void)hipEventSynchronize(b);
  (void)hipEventElapsedTime(ms, a, b);
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  (void)hipFree(out);
  return hipGetLastError() != hipSuccess;
}

// Read bandwidth: `mib` MiB streamed `reps` times by a grid of `blocks`
// workgroups (after one untimed pass); returns 0 and the mean ms per pass.
extern "C" int cohx_probe_read(int mib, int blocks, int reps, float *ms) {
  if (!ms || mib <= 0 || mib > 8192 || blocks <= 0 || blocks > 65536 || reps <= 0 || reps > 1000) return 2;
  const size_t bytes = (size_t)mib << 20, n = bytes / 16;
  float4 *src = nullptr;
  float *out = nullptr;
  if (hipMalloc(&src, bytes) != hipSuccess) return 1;
  if (hipMalloc(&out, (size_t)blocks * 256 * sizeof(float)) != hipSuccess) {
    (void)hipFree(src);
    return 1;
  }
  (void)hipMemset(src, 0, bytes);
  hipEvent_t a, b;
  (void)hipEventCreate(&a);
  (void)hipEventCreate(&b);
  hipLaunchKernelGGL(k_probe_read, dim3(blocks), dim3(256), 0, 0, src, n, out);
  (void)hipEventRecord(a, 0);
  for (int r = 0; r < reps; r++) hipLaunchKernelGGL(k_probe_read, dim3(blocks), dim3(256), 0, 0, src, n, out);
  (void)hipEventRecord(b, 0);
  (void)hipEventSynchronize(b);
  float total = 0.0f;
  (void)hipEventElapsedTime(&total, a, b);
  *ms = total / reps;
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  (void)hipFree(src);
  (void)hipFree(out);
  return hipGetLastError() != hipSuccess;
}
