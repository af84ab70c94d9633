// Library GEMMs (hipBLASLt) for the linears of a step in the packed-prefill
// regime: Y[M][N] (+)= X[M][K] . W[N][K]^T with binary16 (Qwen2 F16) or
// bfloat16 (Qwen3.5, whose f32 activations enter as a hi + lo pair of
// bfloat16 GEMMs) operands, exact products and f32 sums, the same contract as
// the regime's own matrix-core kernel (k_gemm_f16) and held to the same
// tolerance against the reference's sequential f64 dot (cpu.rs:31-48).  Only
// eager steps use it (never under graph capture, never from the
// allocation-free entry point).
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <tuple>

#include "kernels.h"

namespace cohx {

struct GemmLib {
  // per (operand type, N, K, ldo, accumulate, M rounded up to 256): the
  // matmul descriptor and the heuristic's algorithm; per exact M: the
  // operand layouts
  struct Plan {
    hipblasLtMatmulDesc_t op = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    bool ok = false;
  };
  struct Shape {
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    bool ok = false;
  };
  hipblasLtHandle_t h = nullptr;
  void *ws = nullptr;
  size_t ws_bytes = 0;
  std::map<std::tuple<int, int, int, int, bool, int>, Plan> plans;
  std::map<std::tuple<int, int, int, int, int>, Shape> shapes;  // (type, N, K, M, ldo)
};

namespace {

void release(GemmLib::Plan &p) {
  if (p.op) (void)hipblasLtMatmulDescDestroy(p.op);
  p = GemmLib::Plan();
}
void release(GemmLib::Shape &l) {
  if (l.a) (void)hipblasLtMatrixLayoutDestroy(l.a);
  if (l.b) (void)hipblasLtMatrixLayoutDestroy(l.b);
  if (l.c) (void)hipblasLtMatrixLayoutDestroy(l.c);
  l = GemmLib::Shape();
}

// Column-major view: C (N x M, ld ldo) = op_T(W as K x N) . (X as K x M).
bool make_shape(GemmLib::Shape &l, hipDataType t, int N, int K, int M, int ldo) {
  l.ok = !hipblasLtMatrixLayoutCreate(&l.a, t, K, N, K) && !hipblasLtMatrixLayoutCreate(&l.b, t, K, M, K) &&
         !hipblasLtMatrixLayoutCreate(&l.c, HIP_R_32F, N, M, ldo);
  return l.ok;
}

bool make_plan(GemmLib &lib, GemmLib::Plan &p, hipDataType t, int N, int K, int Mb, int ldo) {
  if (hipblasLtMatmulDescCreate(&p.op, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS) return false;
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  if (hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) ||
      hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)))
    return false;
  GemmLib::Shape l;
  if (!make_shape(l, t, N, K, Mb, ldo)) {
    release(l);
    return false;
  }
  hipblasLtMatmulPreference_t pref = nullptr;
  bool ok = !hipblasLtMatmulPreferenceCreate(&pref);
  size_t wsb = lib.ws_bytes;
  hipblasLtMatmulHeuristicResult_t res[1];
  int got = 0;
  ok = ok &&
       !hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb, sizeof(wsb)) &&
       !hipblasLtMatmulAlgoGetHeuristic(lib.h, p.op, l.a, l.b, l.c, l.c, pref, 1, res, &got) && got > 0;
  if (pref) (void)hipblasLtMatmulPreferenceDestroy(pref);
  release(l);
  if (!ok) return false;
  p.algo = res[0].algo;
  p.ok = true;
  return true;
}

}  // namespace

GemmLib *gemm_lib_create(void *workspace, size_t workspace_bytes) {
  GemmLib *lib = new GemmLib();
  if (hipblasLtCreate(&lib->h) != HIPBLAS_STATUS_SUCCESS) {
    delete lib;
    return nullptr;
  }
  lib->ws = workspace;
  lib->ws_bytes = workspace_bytes;
  return lib;
}

void gemm_lib_destroy(GemmLib *lib) {
  if (!lib) return;
  for (auto &kv : lib->plans) release(kv.second);
  for (auto &kv : lib->shapes) release(kv.second);
  if (lib->h) (void)hipblasLtDestroy(lib->h);
  delete lib;
}

namespace {

bool gemm_lib_run(GemmLib *lib, hipStream_t s, hipDataType t, const uint16_t *w, int N, int K, const uint16_t *x,
                  int M, float *out, int ldo, bool accumulate) {
  if (!lib || M <= 0) return false;
  const int Mb = (M + 255) / 256 * 256;
  const auto pkey = std::make_tuple((int)t, N, K, ldo, accumulate, Mb);
  auto pit = lib->plans.find(pkey);
  if (pit == lib->plans.end()) {
    GemmLib::Plan p;
    if (!make_plan(*lib, p, t, N, K, Mb, ldo)) release(p);
    pit = lib->plans.emplace(pkey, p).first;
  }
  if (!pit->second.ok) return false;
  const auto skey = std::make_tuple((int)t, N, K, M, ldo);
  auto sit = lib->shapes.find(skey);
  if (sit == lib->shapes.end()) {
    if (lib->shapes.size() >= 1024) {  // packed row counts vary step to step
      for (auto &kv : lib->shapes) release(kv.second);
      lib->shapes.clear();
    }
    GemmLib::Shape l;
    if (!make_shape(l, t, N, K, M, ldo)) release(l);
    sit = lib->shapes.emplace(skey, l).first;
  }
  const GemmLib::Shape &l = sit->second;
  if (!l.ok) return false;
  const GemmLib::Plan &p = pit->second;
  const float alpha = 1.0f, beta = accumulate ? 1.0f : 0.0f;
  return hipblasLtMatmul(lib->h, p.op, &alpha, w, l.a, x, l.b, &beta, out, l.c, out, l.c, &p.algo, lib->ws,
                         lib->ws_bytes, s) == HIPBLAS_STATUS_SUCCESS;
}

}  // namespace

bool gemm_lib_f16(GemmLib *lib, hipStream_t s, const uint16_t *w, int N, int K, const uint16_t *x, int M,
                  float *out, int ldo, bool accumulate) {
  return gemm_lib_run(lib, s, HIP_R_16F, w, N, K, x, M, out, ldo, accumulate);
}

bool gemm_lib_bf16(GemmLib *lib, hipStream_t s, const uint16_t *w, int N, int K, const uint16_t *x, int M,
                   float *out, int ldo, bool accumulate) {
  return gemm_lib_run(lib, s, HIP_R_16BF, w, N, K, x, M, out, ldo, accumulate);
}

}  // namespace cohx
