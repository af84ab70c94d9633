// Probes for bench.py --valu-probe and --read-probe (built as
// libcohx_probe.so, not part of the step library): the exact attention
// pass's instruction pattern without memory traffic, to separate its VALU
// cost from its K/V stream, and a plain streaming read, for the HBM rate this
// device reaches.  Every launch here is in bounds by construction.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

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

// K-stream probe: the exact scores pass's memory pattern without its
// arithmetic, over an owned pool and page table (every index in bounds by
// construction: tokens < kv[r] <= 64 * kMaxPagesProbe / 4, page entries <
// the pool's page count).  Thread = token; its 64 floats come as 16 float4
// loads of the element-quad-major page layout, rotated by page and head, and
// are summed into one float per token.
constexpr int kProbeRows = 128, kProbeHeads = 2, kMaxPagesProbe = 128;

__device__ __forceinline__ float probe_token(const float *__restrict__ kpool, const int32_t *__restrict__ pt,
                                             const int *__restrict__ kv, int r, int g, int t) {
  const int32_t phys = pt[r * kMaxPagesProbe + t / 16];
  const int rot = ((t / 16) * 5 + g * 3) & 15;
  const float *kq = kpool + ((size_t)phys * kProbeHeads + g) * 1024 + (t % 16) * 4;
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; j++) {
    const float4 v = *reinterpret_cast<const float4 *>(kq + ((j + rot) & 15) * 64);
    acc += (v.x + v.y) + (v.z + v.w);
  }
  return acc;
}

// One workgroup per (row, head, 256-token chunk, part): the launch shape of
// the scores pass (parts > 1 load the same rows again, as its head split does).
__global__ __launch_bounds__(256) void k_probe_kstream(const float *__restrict__ kpool, const int32_t *__restrict__ pt,
                                                       const int *__restrict__ kv, int parts, float *__restrict__ out) {
  const int r = blockIdx.x, g = blockIdx.y, c = (int)(gridDim.z / parts) - 1 - (int)(blockIdx.z / parts);
  const int t = c * 256 + threadIdx.x;
  if (c * 256 >= kv[r]) return;
  const float v = t < kv[r] ? probe_token(kpool, pt, kv, r, g, t) : 0.0f;
  out[((size_t)(r * kProbeHeads + g) * 2048 + (t & 2047)) * 2 + (blockIdx.z % parts)] = v;
}

// Both parts of an item in one workgroup of 512 threads (threads t and
// t + 256 load the same token's row, on the same CU).
__global__ __launch_bounds__(512) void k_probe_kstream_pair(const float *__restrict__ kpool,
                                                            const int32_t *__restrict__ pt,
                                                            const int *__restrict__ kv, float *__restrict__ out) {
  const int r = blockIdx.x, g = blockIdx.y, c = (int)gridDim.z - 1 - (int)blockIdx.z;
  const int t = c * 256 + threadIdx.x % 256, part = threadIdx.x / 256;
  if (c * 256 >= kv[r]) return;
  const float v = t < kv[r] ? probe_token(kpool, pt, kv, r, g, t) : 0.0f;
  out[((size_t)(r * kProbeHeads + g) * 2048 + (t & 2047)) * 2 + part] = v;
}

// Persistent form: `blocks` workgroups walk the live (row, head, chunk)
// items of a host-built list in order, item i by workgroup i % blocks.
__global__ __launch_bounds__(256) void k_probe_kstream_walk(const float *__restrict__ kpool,
                                                            const int32_t *__restrict__ pt,
                                                            const int *__restrict__ kv, const int4 *__restrict__ items,
                                                            int n_items, float *__restrict__ out) {
  for (int i = blockIdx.x; i < n_items; i += gridDim.x) {
    const int4 it = items[i];  // row, head, chunk
    const int t = it.z * 256 + threadIdx.x;
    const float v = t < kv[it.x] ? probe_token(kpool, pt, kv, it.x, it.y, t) : 0.0f;
    out[((size_t)(it.x * kProbeHeads + it.y) * 2048 + (t & 2047)) * 2] = v;
  }
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

// K-stream probe (see k_probe_kstream), over 24 layer pools in turn: mode 0
// one workgroup per item, mode 1
// the same with every item loaded by two workgroups, mode 2 `blocks`
// persistent workgroups over the item list.  128 rows with KV lengths from a
// fixed U[64, 2048] sequence, pages scattered over the pool.  Returns 0, the
// mean ms per launch and the bytes of K rows per launch.
extern "C" int cohx_probe_kstream(int mode, int blocks, int reps, float *ms, double *bytes) {
  if (!ms || !bytes || mode < 0 || mode > 3 || blocks <= 0 || blocks > 65536 || reps <= 0 || reps > 1000) return 2;
  int kvh[kProbeRows];
  uint32_t x = 12345u;
  int pages = 0;
  for (int r = 0; r < kProbeRows; r++) {
    x = x * 1664525u + 1013904223u;
    kvh[r] = 64 + (int)((x >> 8) % 1985u);  // 64 .. 2048
    pages += (kvh[r] + 15) / 16;
  }
  // page ids: row pages interleaved across rows (allocation order of a pool
  // filled lane by lane, step by step), then a fixed scramble
  int32_t *pth = new int32_t[kProbeRows * kMaxPagesProbe];
  for (int i = 0; i < kProbeRows * kMaxPagesProbe; i++) pth[i] = 0;
  int next = 0;
  for (int pg = 0; pg < kMaxPagesProbe; pg++)
    for (int r = 0; r < kProbeRows; r++)
      if (pg * 16 < kvh[r]) pth[r * kMaxPagesProbe + pg] = next++;
  double b = 0.0;
  for (int r = 0; r < kProbeRows; r++) b += (double)kvh[r] * kProbeHeads * 256.0;
  *bytes = b;
  std::vector<int4> itemsh;
  for (int c = 7; c >= 0; c--)
    for (int g = 0; g < kProbeHeads; g++)
      for (int r = 0; r < kProbeRows; r++)
        if (c * 256 < kvh[r]) itemsh.push_back(make_int4(r, g, c, 0));
  float *kpool = nullptr, *out = nullptr;
  int32_t *pt = nullptr;
  int *kv = nullptr;
  int4 *items = nullptr;
  // 24 layer pools, one per launch in turn, so no launch finds its rows in
  // the 256 MB last-level cache (as in a step, where 24 layers pass between
  // two reads of one layer's rows)
  constexpr int kLayers = 24;
  const size_t layer_floats = (size_t)pages * kProbeHeads * 1024;
  const size_t pool_floats = layer_floats * kLayers;
  const size_t out_floats = (size_t)kProbeRows * kProbeHeads * 2048 * 2;
  int rc = 0;
  if (hipMalloc(&kpool, pool_floats * 4) != hipSuccess || hipMalloc(&out, out_floats * 4) != hipSuccess ||
      hipMalloc(&pt, sizeof(int32_t) * kProbeRows * kMaxPagesProbe) != hipSuccess ||
      hipMalloc(&kv, sizeof(int) * kProbeRows) != hipSuccess ||
      hipMalloc(&items, sizeof(int4) * itemsh.size()) != hipSuccess)
    rc = 1;
  if (!rc) {
    (void)hipMemset(kpool, 0, pool_floats * 4);
    (void)hipMemcpy(pt, pth, sizeof(int32_t) * kProbeRows * kMaxPagesProbe, hipMemcpyHostToDevice);
    (void)hipMemcpy(kv, kvh, sizeof(int) * kProbeRows, hipMemcpyHostToDevice);
    (void)hipMemcpy(items, itemsh.data(), sizeof(int4) * itemsh.size(), hipMemcpyHostToDevice);
    const int parts = mode == 1 ? 2 : 1;
    int layer = 0;
    auto launch = [&]() {
      const float *lp = kpool + layer_floats * layer;
      layer = (layer + 1) % kLayers;
      if (mode == 2)
        hipLaunchKernelGGL(k_probe_kstream_walk, dim3(blocks), dim3(256), 0, 0, lp, pt, kv, items,
                           (int)itemsh.size(), out);
      else if (mode == 3)
        hipLaunchKernelGGL(k_probe_kstream_pair, dim3(kProbeRows, kProbeHeads, 8), dim3(512), 0, 0, lp, pt, kv,
                           out);
      else
        hipLaunchKernelGGL(k_probe_kstream, dim3(kProbeRows, kProbeHeads, 8 * parts), dim3(256), 0, 0, lp, pt,
                           kv, parts, out);
    };
    launch();
    hipEvent_t a, e;
    (void)hipEventCreate(&a);
    (void)hipEventCreate(&e);
    (void)hipEventRecord(a, 0);
    for (int i = 0; i < reps; i++) launch();
    (void)hipEventRecord(e, 0);
    (void)hipEventSynchronize(e);
    float total = 0.0f;
    (void)hipEventElapsedTime(&total, a, e);
    *ms = total / reps;
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(e);
    rc = hipGetLastError() != hipSuccess;
  }
  if (kpool) (void)hipFree(kpool);
  if (out) (void)hipFree(out);
  if (pt) (void)hipFree(pt);
  if (kv) (void)hipFree(kv);
  if (items) (void)hipFree(items);
  delete[] pth;
  return rc;
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
