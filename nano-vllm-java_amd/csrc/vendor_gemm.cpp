// o_proj batches of more than a few rows on hipBLASLt (Linear.Row.forward -> Ops.linear,
// layers/Linear.java:296-335, tensor/Ops.java:84-124): y[rows, out] = x[rows, in] W^T + bias,
// in fp32 (HIPBLAS_COMPUTE_32F: fp32 products on the matrix cores) with the bias added in the
// GEMM's epilogue.  A plain GEMM is the vendor library's job: its stream-K 128 x 128 x 64 kernels
// run the 4096-row Qwen3 o_proj in 126 us against 145-164 us for this library's 128 x 128 tiles.
// Decode batches stay on the library's GEMV and 32 x 32-block kernels, which are faster there
// (up to 3x at 1-8 rows) once hipBLASLt's per-call host cost is counted.
//
// hipBLASLt is column-major: with W row-major [out, in] (column-major in x out, transposed) and
// x row-major [rows, in] (column-major in x rows), D = op(A) op(B) = W x^T is column-major
// out x rows, i.e. y row-major.  Each shape's descriptors and the heuristic's algorithm are
// built once and kept; the workspace grows to the largest an algorithm asks for.
#include <hipblaslt/hipblaslt.h>

#include <cstdio>

#include "nva_internal.h"

namespace nva {

namespace {

constexpr size_t kMaxWorkspace = 64ull << 20;  // offered to the heuristic
constexpr size_t kMaxShapes = 32;              // descriptor sets kept per context

struct Shape {
  int rows = 0, in = 0, out = 0;
  bool bias = false;
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  size_t workspace = 0;
  uint64_t last_use = 0;
};

void release(Shape &s) {
  if (s.c) (void)hipblasLtMatrixLayoutDestroy(s.c);
  if (s.b) (void)hipblasLtMatrixLayoutDestroy(s.b);
  if (s.a) (void)hipblasLtMatrixLayoutDestroy(s.a);
  if (s.desc) (void)hipblasLtMatmulDescDestroy(s.desc);
  s = Shape();
}

}  // namespace

struct VendorGemm {
  int device = 0;
  hipblasLtHandle_t handle = nullptr;
  std::vector<Shape> shapes;
  void *workspace = nullptr;
  size_t workspace_bytes = 0;
  uint64_t tick = 0;
};

VendorGemm *vendor_gemm_create(int device, std::string *err) {
  hipblasLtHandle_t h = nullptr;
  const hipblasStatus_t st = hipblasLtCreate(&h);
  if (st != HIPBLAS_STATUS_SUCCESS) {
    char buf[96];
    snprintf(buf, sizeof buf, "hipblasLtCreate failed (status %d)", (int)st);
    *err = buf;
    return nullptr;
  }
  VendorGemm *v = new VendorGemm();
  v->device = device;
  v->handle = h;
  return v;
}

void vendor_gemm_destroy(VendorGemm *v) {
  if (!v) return;
  for (Shape &s : v->shapes) release(s);
  if (v->workspace) (void)hipFree(v->workspace);
  if (v->handle) (void)hipblasLtDestroy(v->handle);
  delete v;
}

bool vendor_gemm_run(VendorGemm *v, const float *x, const float *w, const float *bias, float *y,
                     int rows, int in, int out, hipStream_t stream, std::string *err) {
  char buf[160];
  auto bad = [&](const char *what, int code) {
    snprintf(buf, sizeof buf, "hipBLASLt %s failed (status %d) for [%d, %d] x [%d, %d]^T", what,
             code, rows, in, out, in);
    *err = buf;
    return false;
  };
  const bool has_bias = bias != nullptr;
  Shape *sh = nullptr;
  for (Shape &s : v->shapes)
    if (s.rows == rows && s.in == in && s.out == out && s.bias == has_bias) sh = &s;
  if (!sh) {
    if (v->shapes.size() >= kMaxShapes) {  // drop the least recently used
      size_t lru = 0;
      for (size_t j = 1; j < v->shapes.size(); j++)
        if (v->shapes[j].last_use < v->shapes[lru].last_use) lru = j;
      release(v->shapes[lru]);
      v->shapes.erase(v->shapes.begin() + (long)lru);
    }
    Shape s;
    s.rows = rows;
    s.in = in;
    s.out = out;
    s.bias = has_bias;
    hipblasStatus_t st = hipblasLtMatmulDescCreate(&s.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
    if (st != HIPBLAS_STATUS_SUCCESS) return bad("descriptor", (int)st);
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    st = hipblasLtMatmulDescSetAttribute(s.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta);
    if (st == HIPBLAS_STATUS_SUCCESS)
      st = hipblasLtMatmulDescSetAttribute(s.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb);
    if (st == HIPBLAS_STATUS_SUCCESS && has_bias) {
      const hipblasLtEpilogue_t ep = HIPBLASLT_EPILOGUE_BIAS;
      const hipDataType bt = HIP_R_32F;
      st = hipblasLtMatmulDescSetAttribute(s.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &ep, sizeof ep);
      if (st == HIPBLAS_STATUS_SUCCESS)
        st = hipblasLtMatmulDescSetAttribute(s.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt,
                                             sizeof bt);
    }
    if (st == HIPBLAS_STATUS_SUCCESS)
      st = hipblasLtMatrixLayoutCreate(&s.a, HIP_R_32F, (uint64_t)in, (uint64_t)out, in);
    if (st == HIPBLAS_STATUS_SUCCESS)
      st = hipblasLtMatrixLayoutCreate(&s.b, HIP_R_32F, (uint64_t)in, (uint64_t)rows, in);
    if (st == HIPBLAS_STATUS_SUCCESS)
      st = hipblasLtMatrixLayoutCreate(&s.c, HIP_R_32F, (uint64_t)out, (uint64_t)rows, out);
    hipblasLtMatmulPreference_t pref = nullptr;
    if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatmulPreferenceCreate(&pref);
    if (st == HIPBLAS_STATUS_SUCCESS) {
      const uint64_t ws = kMaxWorkspace;
      st = hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                 &ws, sizeof ws);
    }
    hipblasLtMatmulHeuristicResult_t result{};
    int found = 0;
    if (st == HIPBLAS_STATUS_SUCCESS)
      st = hipblasLtMatmulAlgoGetHeuristic(v->handle, s.desc, s.a, s.b, s.c, s.c, pref, 1, &result,
                                           &found);
    if (pref) (void)hipblasLtMatmulPreferenceDestroy(pref);
    if (st != HIPBLAS_STATUS_SUCCESS || found < 1) {
      release(s);
      return bad("algorithm selection", st != HIPBLAS_STATUS_SUCCESS ? (int)st : -1);
    }
    s.algo = result.algo;
    s.workspace = result.workspaceSize;
    v->shapes.push_back(s);
    sh = &v->shapes.back();
  }
  if (sh->workspace > v->workspace_bytes) {
    // Work already queued (on any stream the context used) may still read the old workspace.
    if (v->workspace) {
      if (hipDeviceSynchronize() != hipSuccess) return bad("workspace sync", -1);
      (void)hipFree(v->workspace);
      v->workspace = nullptr;
      v->workspace_bytes = 0;
    }
    if (hipMalloc(&v->workspace, sh->workspace) != hipSuccess) return bad("workspace", -1);
    v->workspace_bytes = sh->workspace;
  }
  sh->last_use = ++v->tick;
  if (has_bias) {
    const void *bp = bias;
    const hipblasStatus_t st = hipblasLtMatmulDescSetAttribute(
        sh->desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bp, sizeof bp);
    if (st != HIPBLAS_STATUS_SUCCESS) return bad("bias pointer", (int)st);
  }
  const float alpha = 1.0f, beta = 0.0f;
  const hipblasStatus_t st =
      hipblasLtMatmul(v->handle, sh->desc, &alpha, w, sh->a, x, sh->b, &beta, y, sh->c, y, sh->c,
                      &sh->algo, v->workspace, sh->workspace, stream);
  if (st != HIPBLAS_STATUS_SUCCESS) return bad("matmul", (int)st);
  return true;
}

}  // namespace nva
