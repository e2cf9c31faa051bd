// The attention block's neighbours behind the C ABI: rms_norm, rope and
// matmul. Validation order and error text follow
// crates/metal-infer-core/src/ops.rs (rms_norm :722-755, rope :882-915,
// matmul :242-260); the kernel choice is MI355X-specific.
#include <hipblaslt/hipblaslt.h>

#include <array>
#include <map>
#include <string>

#include "kernels.hpp"
#include "runtime.hpp"

namespace mi {

// A GEMM planned once per (m, n, k, leading dimensions): hipBLASLt
// descriptors of out^T[n, m] = weight[n, k] . input^T[k, m] in column-major
// terms (A = weight read transposed, B = input), and the heuristic's first
// algorithm with the workspace it needs; `ok` false means hipBLASLt had no
// solution and the few-row kernel runs instead.
struct GemmPlan {
  bool ok = false;
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  size_t workspace = 0;
};

struct GemmState {
  hipblasLtHandle_t handle = nullptr;
  std::map<std::array<int64_t, 6>, GemmPlan> plans;
};

void release_gemm(Context *ctx) {
  GemmState *state = ctx->gemm;
  if (state == nullptr) return;
  for (auto &entry : state->plans) {
    GemmPlan &plan = entry.second;
    if (plan.a) hipblasLtMatrixLayoutDestroy(plan.a);
    if (plan.b) hipblasLtMatrixLayoutDestroy(plan.b);
    if (plan.c) hipblasLtMatrixLayoutDestroy(plan.c);
    if (plan.op) hipblasLtMatmulDescDestroy(plan.op);
  }
  if (state->handle) hipblasLtDestroy(state->handle);
  delete state;
  ctx->gemm = nullptr;
}

namespace {

// Largest workspace a GEMM plan may ask for (leased from the batch arena).
constexpr uint64_t kGemmWorkspaceBytes = 32ull << 20;

mi_status to_u32(int64_t value, const char *label, uint32_t *out) {
  if (value < 0 || (uint64_t)value > 0xffffffffull)
    return fail(MI_ERR_SHAPE, std::string(label) + " does not fit in u32");
  *out = (uint32_t)value;
  return MI_OK;
}

std::string shape_text(const mi_tensor &t) {
  std::string s = "[";
  for (int32_t i = 0; i < t.rank; ++i) {
    if (i) s += ", ";
    s += std::to_string(t.shape[i]);
  }
  return s + "]";
}

bool same_shape(const mi_tensor &a, const mi_tensor &b) {
  if (a.rank != b.rank) return false;
  for (int32_t i = 0; i < a.rank; ++i)
    if (a.shape[i] != b.shape[i]) return false;
  return true;
}

// The leading (row) dimensions of a rank 1..4 tensor as a kernel RowIndex.
kernels::RowIndex row_index(const mi_tensor &t) {
  int64_t dims[3] = {1, 1, 1}, strides[3] = {0, 0, 0};
  for (int32_t i = 0; i < t.rank - 1; ++i) {
    const int32_t slot = 3 - (t.rank - 1) + i;
    dims[slot] = t.shape[i];
    strides[slot] = t.stride[i];
  }
  return kernels::RowIndex{(uint32_t)dims[1], (uint32_t)dims[2], strides[0], strides[1],
                           strides[2]};
}

// The cached plan for this shape, made on first use. Fails only when the
// handle cannot be created.
mi_status gemm_plan(Context *ctx, uint32_t m, uint32_t n, uint32_t k, int64_t ldx, int64_t ldw,
                    int64_t ldo, GemmPlan **out) {
  if (ctx->gemm == nullptr) {
    auto *state = new GemmState();
    if (hipblasLtCreate(&state->handle) != HIPBLAS_STATUS_SUCCESS) {
      delete state;
      return fail(MI_ERR_RESOURCE, "hipblasLtCreate failed");
    }
    ctx->gemm = state;
  }
  const std::array<int64_t, 6> key{m, n, k, ldx, ldw, ldo};
  auto found = ctx->gemm->plans.find(key);
  if (found != ctx->gemm->plans.end()) {
    *out = &found->second;
    return MI_OK;
  }
  GemmPlan &plan = ctx->gemm->plans[key];
  *out = &plan;
  const hipblasOperation_t trans_a = HIPBLAS_OP_T, trans_b = HIPBLAS_OP_N;
  hipblasLtMatmulPreference_t pref = nullptr;
  bool made =
      hipblasLtMatmulDescCreate(&plan.op, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatmulDescSetAttribute(plan.op, HIPBLASLT_MATMUL_DESC_TRANSA, &trans_a,
                                      sizeof(trans_a)) == HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatmulDescSetAttribute(plan.op, HIPBLASLT_MATMUL_DESC_TRANSB, &trans_b,
                                      sizeof(trans_b)) == HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatrixLayoutCreate(&plan.a, HIP_R_16F, k, n, ldw) == HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatrixLayoutCreate(&plan.b, HIP_R_16F, k, m, ldx) == HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatrixLayoutCreate(&plan.c, HIP_R_16F, n, m, ldo) == HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
  if (made) {
    const uint64_t limit = kGemmWorkspaceBytes;
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &limit,
                                          sizeof(limit));
    hipblasLtMatmulHeuristicResult_t result[1];
    int returned = 0;
    if (hipblasLtMatmulAlgoGetHeuristic(ctx->gemm->handle, plan.op, plan.a, plan.b, plan.c,
                                        plan.c, pref, 1, result, &returned) ==
            HIPBLAS_STATUS_SUCCESS &&
        returned > 0 && result[0].state == HIPBLAS_STATUS_SUCCESS) {
      plan.algo = result[0].algo;
      plan.workspace = result[0].workspaceSize;
      plan.ok = true;
    }
  }
  if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  return MI_OK;
}

mi_status run_gemm(Batch *batch, const GemmPlan &plan, const mi_tensor &x, const mi_tensor &w,
                   const mi_tensor &out) {
  void *workspace = nullptr;
  mi_status st;
  if (plan.workspace > 0 &&
      (st = scratch_alloc(batch, plan.workspace, &workspace)) != MI_OK)
    return st;
  hipblasLtHandle_t handle = batch->ctx->gemm->handle;
  st = launch(batch, "gemm", [&](const kernels::Launch &l) {
    const float alpha = 1.0f, beta = 0.0f;
    if (l.start) hipEventRecord(l.start, l.stream);
    const hipblasStatus_t status =
        hipblasLtMatmul(handle, plan.op, &alpha, w.data, plan.a, x.data, plan.b, &beta, out.data,
                        plan.c, out.data, plan.c, &plan.algo, workspace, plan.workspace,
                        l.stream);
    if (l.stop) hipEventRecord(l.stop, l.stream);
    return status == HIPBLAS_STATUS_SUCCESS ? hipGetLastError() : hipErrorLaunchFailure;
  });
  // The batch's stream runs in order, so later work may reuse the range.
  if (workspace) scratch_free(batch->ctx, workspace);
  return st;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" {

mi_status mi_rms_norm(mi_batch *batch, const mi_tensor *input, const mi_tensor *weight,
                      float epsilon, const mi_tensor *out) {
  if (batch == nullptr || input == nullptr || weight == nullptr || out == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null batch or tensor");
  if (batch->committed) return fail(MI_ERR_RESOURCE, "batch was already committed");
  mi_status st;
  if ((st = require_f16(input)) != MI_OK || (st = require_f16(weight)) != MI_OK) return st;
  if (input->rank < 1) return fail(MI_ERR_SHAPE, "rms_norm requires rank >= 1");
  const int64_t width = input->shape[input->rank - 1];
  if (weight->rank != 1 || weight->shape[0] != width)
    return fail(MI_ERR_SHAPE, "rms_norm weight must have shape [" + std::to_string(width) + "]");
  if ((st = require_f16(out)) != MI_OK) return st;
  if (!same_shape(*input, *out))
    return fail(MI_ERR_SHAPE, "rms_norm output must have the input's shape");
  if (input->stride[input->rank - 1] != 1 || out->stride[out->rank - 1] != 1 ||
      weight->stride[0] != 1)
    return fail(MI_ERR_SHAPE, "rms_norm tensors need a unit innermost stride");
  kernels::RmsNormParams p{};
  if ((st = to_u32((int64_t)(element_count(*input) / (uint64_t)width), "rows", &p.rows)) != MI_OK ||
      (st = to_u32(width, "width", &p.width)) != MI_OK)
    return st;
  p.x = static_cast<const uint16_t *>(input->data);
  p.x_rows = row_index(*input);
  p.weight = static_cast<const uint16_t *>(weight->data);
  p.out = static_cast<uint16_t *>(out->data);
  p.o_rows = row_index(*out);
  p.epsilon = epsilon;
  const uint32_t cus = batch->ctx->compute_units;
  return launch(batch, "rms_norm",
                [&](const kernels::Launch &l) { return kernels::launch_rms_norm(p, cus, l); });
}

mi_status mi_rope(mi_batch *batch, const mi_tensor *input, uint64_t offset, float theta,
                  const mi_tensor *out) {
  if (batch == nullptr || input == nullptr || out == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null batch or tensor");
  if (batch->committed) return fail(MI_ERR_RESOURCE, "batch was already committed");
  mi_status st;
  if ((st = require_f16(input)) != MI_OK) return st;
  if (input->rank != 3) return fail(MI_ERR_SHAPE, "RoPE expects [tokens, heads, head_dim]");
  if (input->shape[2] % 2 != 0) return fail(MI_ERR_SHAPE, "RoPE head_dim must be even");
  if ((st = require_f16(out)) != MI_OK) return st;
  if (!same_shape(*input, *out))
    return fail(MI_ERR_SHAPE, "RoPE output must have the input's shape");
  if (input->stride[2] != 1 || out->stride[2] != 1)
    return fail(MI_ERR_SHAPE, "RoPE tensors need a unit innermost stride");
  kernels::RopeParams p{};
  if ((st = to_u32(input->shape[0], "tokens", &p.tokens)) != MI_OK ||
      (st = to_u32(input->shape[1], "heads", &p.heads)) != MI_OK ||
      (st = to_u32(input->shape[2], "head_dim", &p.head_dim)) != MI_OK)
    return st;
  if (offset > 0xffffffffull) return fail(MI_ERR_SHAPE, "offset does not fit in u32");
  p.offset = (uint32_t)offset;
  p.theta = theta;
  p.x = static_cast<const uint16_t *>(input->data);
  p.x_tok = input->stride[0], p.x_head = input->stride[1];
  p.out = static_cast<uint16_t *>(out->data);
  p.o_tok = out->stride[0], p.o_head = out->stride[1];
  return launch(batch, "rope", [&](const kernels::Launch &l) { return kernels::launch_rope(p, l); });
}

mi_status mi_matmul(mi_batch *batch, const mi_tensor *input, const mi_tensor *weight,
                    const mi_tensor *out) {
  if (batch == nullptr || input == nullptr || weight == nullptr || out == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "null batch or tensor");
  if (batch->committed) return fail(MI_ERR_RESOURCE, "batch was already committed");
  mi_status st;
  if ((st = require_f16(input)) != MI_OK || (st = require_f16(weight)) != MI_OK) return st;
  if (input->rank != 2) return fail(MI_ERR_SHAPE, "expected matrix, got " + shape_text(*input));
  if (weight->rank != 2) return fail(MI_ERR_SHAPE, "expected matrix, got " + shape_text(*weight));
  const int64_t m = input->shape[0], k = input->shape[1], n = weight->shape[0];
  if (weight->shape[1] != k)
    return fail(MI_ERR_SHAPE, "matmul inner dimensions differ: " + std::to_string(k) + " and " +
                                  std::to_string(weight->shape[1]));
  if ((st = require_f16(out)) != MI_OK) return st;
  if (out->rank != 2 || out->shape[0] != m || out->shape[1] != n)
    return fail(MI_ERR_SHAPE, "matmul output must have shape [" + std::to_string(m) + ", " +
                                  std::to_string(n) + "]");
  if (input->stride[1] != 1 || weight->stride[1] != 1 || out->stride[1] != 1)
    return fail(MI_ERR_SHAPE, "matmul tensors need a unit innermost stride");
  kernels::MatvecParams p{};
  if ((st = to_u32(m, "m", &p.m)) != MI_OK || (st = to_u32(n, "n", &p.n)) != MI_OK ||
      (st = to_u32(k, "k", &p.k)) != MI_OK)
    return st;
  // Row strides of single-row views are free; give them the packed value.
  const int64_t ldx = m > 1 ? input->stride[0] : k;
  const int64_t ldw = n > 1 ? weight->stride[0] : k;
  const int64_t ldo = m > 1 ? out->stride[0] : n;
  if (ldx < k || ldw < k || ldo < n)
    return fail(MI_ERR_SHAPE, "matmul rows overlap (row stride below the row length)");
  p.x = static_cast<const uint16_t *>(input->data), p.x_row = ldx;
  p.w = static_cast<const uint16_t *>(weight->data), p.w_row = ldw;
  p.out = static_cast<uint16_t *>(out->data), p.o_row = ldo;
  // 9 to 32 rows (the batched-decode o_proj): the skinny GEMM where the
  // grid fits the device; it measured 9.9 us against hipBLASLt's 12.1 us for
  // [32, 4096] x [4096, 4096]^T.
  const uint32_t cus = batch->ctx->compute_units;
  if (kernels::skinny_gemm_supported(p, cus))
    return launch(batch, "skinny_gemm",
                  [&](const kernels::Launch &l) { return kernels::launch_skinny_gemm(p, cus, l); });
  // Empty products (n or k of 0) stay on the few-row kernel: no launch for
  // n == 0, zeros for k == 0.
  if (p.m > kernels::kMatvecRows && p.n > 0 && p.k > 0) {
    GemmPlan *plan = nullptr;
    if ((st = gemm_plan(batch->ctx, p.m, p.n, p.k, ldx, ldw, ldo, &plan)) != MI_OK) return st;
    if (plan->ok) return run_gemm(batch, *plan, *input, *weight, *out);
  }
  return launch(batch, "matvec",
                [&](const kernels::Launch &l) { return kernels::launch_matvec(p, l); });
}

}  // extern "C"
