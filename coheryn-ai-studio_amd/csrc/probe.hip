// Probes for bench.py --valu-probe and --read-probe (built as
// libcohx_probe.so, not part of the step library): the exact attention
// pass's instruction pattern without memory traffic, to separate its VALU
// cost from its K/V stream, and a plain streaming read, for the HBM rate this
// device reaches.  Every launch here is in bounds by construction.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

// C independent f64 chains per thread; per step E elements: C products
// q*k in f32, their widenings, and the chain adds, in the attention pass's
// grouping (products, then widenings, then adds).
template <int C, int E>
__global__ __launch_bounds__(256) void k_probe_triples(const float *__restrict__ q, const float *__restrict__ kin,
                                                       double *__restrict__ out, int steps) {
  float k[E];
#pragma unroll
  for (int e = 0; e < E; e++) k[e] = kin[(threadIdx.x + e) % 256];
  double acc[C];
#pragma unroll
  for (int c = 0; c < C; c++) acc[c] = 0.0;
  for (int s = 0; s < steps; s++) {
#pragma unroll
    for (int e = 0; e < E; e++) {
      float pr[C];
#pragma unroll
      for (int c = 0; c < C; c++) pr[c] = q[((s % 32) * E + e) * 16 + c] * k[e];
      double w[C];
#pragma unroll
      for (int c = 0; c < C; c++) w[c] = (double)pr[c];
#pragma unroll
      for (int c = 0; c < C; c++) acc[c] += w[c];
    }
  }
  double t = 0;
#pragma unroll
  for (int c = 0; c < C; c++) t += acc[c];
  out[(size_t)blockIdx.x * 256 + threadIdx.x] = t;
}

template <int C, int E>
int time_triples(int blocks, int steps, float *ms_out) {
  float *q = nullptr, *k = nullptr;
  double *o = nullptr;
  if (hipMalloc(&q, 32 * E * 16 * sizeof(float)) != hipSuccess) return 1;
  if (hipMalloc(&k, 256 * sizeof(float)) != hipSuccess) return 1;
  if (hipMalloc(&o, (size_t)blocks * 256 * sizeof(double)) != hipSuccess) return 1;
  (void)hipMemset(q, 0, 32 * E * 16 * sizeof(float));
  (void)hipMemset(k, 0, 256 * sizeof(float));
  hipEvent_t a, b;
  (void)hipEventCreate(&a);
  (void)hipEventCreate(&b);
  hipLaunchKernelGGL((k_probe_triples<C, E>), dim3(blocks), dim3(256), 0, 0, q, k, o, steps);
  (void)hipDeviceSynchronize();
  (void)hipEventRecord(a, 0);
  hipLaunchKernelGGL((k_probe_triples<C, E>), dim3(blocks), dim3(256), 0, 0, q, k, o, steps);
  (void)hipEventRecord(b, 0);
  (void)hipEventSynchronize(b);
  (void)hipEventElapsedTime(ms_out, a, b);
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  (void)hipFree(q);
  (void)hipFree(k);
  (void)hipFree(o);
  return hipGetLastError() != hipSuccess;
}

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

}  // namespace

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

// Time `blocks` workgroups of 256 threads, each thread running `steps`
// steps of E elements x C chains; returns 0 and the kernel time in ms.
// (C, E) in {(7, 4), (4, 4), (3, 2), (14, 2), (7, 8)}.
extern "C" int cohx_probe_triples(int chains, int elements, int blocks, int steps, float *ms) {
  if (!ms || blocks <= 0 || blocks > 65536 || steps <= 0 || steps > 4096) return 2;
  if (chains == 7 && elements == 4) return time_triples<7, 4>(blocks, steps, ms);
  if (chains == 4 && elements == 4) return time_triples<4, 4>(blocks, steps, ms);
  if (chains == 3 && elements == 2) return time_triples<3, 2>(blocks, steps, ms);
  if (chains == 14 && elements == 2) return time_triples<14, 2>(blocks, steps, ms);
  if (chains == 7 && elements == 8) return time_triples<7, 8>(blocks, steps, ms);
  return 2;
}
