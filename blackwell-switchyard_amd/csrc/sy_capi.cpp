// The C ABI (include/switchyard.h): argument checks, planning and launches.
// Every check that can be made on the host is made before any device work,
// so bad arguments come back as negative sy_status codes. Nothing here
// allocates device memory.
#include <cstdlib>
#include <map>
#include <mutex>

#include "../../include/switchyard.h"
#include "sy_launch.hpp"

namespace sy {

namespace {

bool valid_dtype(int t) { return t == SY_F32 || t == SY_F16 || t == SY_BF16; }
int64_t esize(int t) { return t == SY_F32 ? 4 : 2; }
bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Row starts (pointer + k * row_stride elements) are all 16-byte aligned.
bool rows_aligned(const void* p, int64_t row_stride, int dtype) {
  return al16(p) && (row_stride * esize(dtype)) % 16 == 0;
}

int status(hipError_t e) { return e == hipSuccess ? SY_OK : (int)e; }

std::mutex g_mu;
std::map<int, int> g_cus;                                   // device -> CU count

hipError_t bwd_resources(const sy_plan& p, int dtype, bool stats, KernelRes* out) {
  if (dtype == SY_BF16) return bwd_vec_resources_bf16(p, stats, out);
  if (dtype == SY_F16) return bwd_vec_resources_f16(p, stats, out);
  return bwd_vec_resources_f32(p, stats, out);
}

// Persistent workgroup count of the backward: every CU filled at the
// kernel's register/LDS occupancy, never more than there are token slots.
// Deterministic in (plan, n_tok, stats, device), which keeps dw bit-stable.
int bwd_grid(const sy_plan& p, int64_t n_tok, int dtype, bool stats, int* grid) {
  int cus = 0;
  hipError_t e = cu_count(&cus);
  if (e != hipSuccess) return e == hipErrorNoDevice ? SY_ERR_DEVICE : (int)e;
  int per_cu = 4;
  if (p.family != SY_FAMILY_GENERIC) {
    KernelRes r;
    e = bwd_resources(p, dtype, stats, &r);
    if (e != hipSuccess) return (int)e;
    per_cu = r.blocks_per_cu;
  }
  // Tuning knob for measurement sweeps: workgroups per CU of the persistent grid.
  if (const char* env = std::getenv("SY_BWD_BLOCKS_PER_CU")) {
    const int k = std::atoi(env);
    if (k >= 1 && k <= 64) per_cu = k;
  }
  const int64_t slots = (n_tok + p.tokens_per_block - 1) / p.tokens_per_block;
  int64_t g = (int64_t)cus * per_cu;
  if (g > slots) g = slots;
  if (g < 1) g = 1;
  *grid = (int)g;
  return SY_OK;
}

hipError_t fwd_vec(const sy_plan& p, const FwdArgs& a, hipStream_t s) {
  if (a.v_dtype == SY_BF16) return launch_fwd_vec_bf16(p, a, s, nullptr);
  if (a.v_dtype == SY_F16) return launch_fwd_vec_f16(p, a, s, nullptr);
  return launch_fwd_vec_f32(p, a, s, nullptr);
}
hipError_t sol_vec(const sy_plan& p, const FwdArgs& a, hipStream_t s) {
  if (a.v_dtype == SY_BF16) return launch_sol_vec_bf16(p, a, s);
  if (a.v_dtype == SY_F16) return launch_sol_vec_f16(p, a, s);
  return launch_sol_vec_f32(p, a, s);
}
hipError_t batched_vec(const sy_plan& p, const BatchedArgs& a, hipStream_t s) {
  if (a.dtype == SY_BF16) return launch_batched_vec_bf16(p, a, s);
  if (a.dtype == SY_F16) return launch_batched_vec_f16(p, a, s);
  return launch_batched_vec_f32(p, a, s);
}
hipError_t bwd_vec(const sy_plan& p, const BwdArgs& a, int grid, hipStream_t s) {
  if (a.v_dtype == SY_BF16) return launch_bwd_vec_bf16(p, a, grid, s);
  if (a.v_dtype == SY_F16) return launch_bwd_vec_f16(p, a, grid, s);
  return launch_bwd_vec_f32(p, a, grid, s);
}

// Shared argument checks for v-shaped inputs.
int check_common(int64_t n_src, int64_t n_tok, int64_t d, int64_t src_stride, int v_dtype,
                 int w_dtype) {
  if (!valid_dtype(v_dtype) || !valid_dtype(w_dtype)) return SY_ERR_DTYPE;
  if (n_src < 1 || d < 1 || n_tok < 0) return SY_ERR_SHAPE;
  if (n_src > 0x7fffffff || d > 0x7fffffff / 16 || n_tok > ((int64_t)1 << 40)) return SY_ERR_SHAPE;
  if (n_src > 1 && src_stride < n_tok * d) return SY_ERR_STRIDE;
  return SY_OK;
}

}  // namespace

hipError_t cu_count(int* out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_cus.find(dev);
    if (it != g_cus.end()) {
      *out = it->second;
      return hipSuccess;
    }
  }
  int n = 0;
  e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lk(g_mu);
  g_cus[dev] = n;
  *out = n;
  return hipSuccess;
}

}  // namespace sy

using namespace sy;

extern "C" {

int sy_abi_version(void) { return SY_ABI_VERSION; }

int sy_plan_for(int op, int64_t n_src, int64_t n_q, int64_t d, int v_dtype, int w_dtype,
                int aligned, sy_plan* out) {
  return make_plan(op, n_src, n_q, d, v_dtype, w_dtype, aligned, out);
}

int sy_fwd(const void* v, const void* w, void* out, float* stats, int64_t n_src, int64_t n_tok,
           int64_t d, int64_t src_stride, int v_dtype, int w_dtype, float eps, void* stream) {
  // Empty tensors have NULL data pointers; with no tokens nothing is touched.
  if (n_tok != 0 && (v == nullptr || w == nullptr || out == nullptr)) return SY_ERR_NULL;
  int rc = check_common(n_src, n_tok, d, src_stride, v_dtype, w_dtype);
  if (rc != SY_OK) return rc;
  const bool aligned = rows_aligned(v, src_stride, v_dtype) && rows_aligned(v, d, v_dtype) &&
                       al16(w) && al16(out) && (d * esize(v_dtype)) % 16 == 0;
  sy_plan p;
  rc = make_plan(SY_OP_FWD, n_src, 0, d, v_dtype, w_dtype, aligned, &p);
  if (rc != SY_OK) return rc;
  apply_tile_override(SY_OP_FWD, n_src, d, &p);
  if (n_tok == 0) return SY_OK;
  const FwdArgs a{v, w, out, stats, (int)n_src, n_tok, (int)d, src_stride, v_dtype, w_dtype, eps};
  const hipStream_t s = (hipStream_t)stream;
  return status(p.family == SY_FAMILY_GENERIC ? launch_fwd_generic(a, s) : fwd_vec(p, a, s));
}

int sy_sol(const void* v, void* out, int64_t n_src, int64_t n_tok, int64_t d, int64_t src_stride,
           int dtype, void* stream) {
  if (n_tok != 0 && (v == nullptr || out == nullptr)) return SY_ERR_NULL;
  int rc = check_common(n_src, n_tok, d, src_stride, dtype, dtype);
  if (rc != SY_OK) return rc;
  const bool aligned = rows_aligned(v, src_stride, dtype) && rows_aligned(v, d, dtype) &&
                       al16(out) && (d * esize(dtype)) % 16 == 0;
  sy_plan p;
  rc = make_plan(SY_OP_SOL, n_src, 0, d, dtype, dtype, aligned, &p);
  if (rc != SY_OK) return rc;
  apply_tile_override(SY_OP_SOL, n_src, d, &p);
  if (n_tok == 0) return SY_OK;
  const FwdArgs a{v, nullptr, out, nullptr, (int)n_src, n_tok, (int)d, src_stride, dtype, dtype, 0.0f};
  const hipStream_t s = (hipStream_t)stream;
  return status(p.family == SY_FAMILY_GENERIC ? launch_sol_generic(a, s) : sol_vec(p, a, s));
}

int64_t sy_bwd_workspace_bytes(int64_t n_src, int64_t n_tok, int64_t d, int v_dtype, int w_dtype) {
  int rc = check_common(n_src, n_tok, d, n_tok * d, v_dtype, w_dtype);
  if (rc != SY_OK) return rc;
  if (n_tok == 0) return 0;
  // The vector plan assumes aligned buffers; a misaligned call falls back to
  // the generic kernel with its own grid, so size for the larger of the two.
  sy_plan pv, pg;
  rc = make_plan(SY_OP_BWD, n_src, 0, d, v_dtype, w_dtype, 1, &pv);
  if (rc != SY_OK) return rc;
  apply_tile_override(SY_OP_BWD, n_src, d, &pv);
  rc = make_plan(SY_OP_BWD, n_src, 0, d, v_dtype, w_dtype, 0, &pg);
  if (rc != SY_OK) return rc;
  int64_t g = 0;
  for (const sy_plan* pp : {&pv, &pg}) {
    for (bool st : {true, false}) {
      int gi = 0;
      rc = bwd_grid(*pp, n_tok, v_dtype, st, &gi);
      if (rc != SY_OK) return rc;
      if (gi > g) g = gi;
    }
  }
  return g * d * (int64_t)sizeof(float);
}

// Main backward kernel: dv and the fp32 dw partials. *rows_out receives the
// partial row count (the persistent grid).
static int bwd_main(const void* v, const void* w, const void* grad_out, const float* stats,
                    void* dv, void* workspace, int64_t workspace_bytes, int64_t n_src,
                    int64_t n_tok, int64_t d, int64_t src_stride, int v_dtype, int w_dtype,
                    float eps, hipStream_t s, int* rows_out) {
  *rows_out = 0;
  if (n_tok != 0 && (v == nullptr || w == nullptr || grad_out == nullptr || dv == nullptr))
    return SY_ERR_NULL;
  int rc = check_common(n_src, n_tok, d, src_stride, v_dtype, w_dtype);
  if (rc != SY_OK || n_tok == 0) return rc;
  const bool aligned = rows_aligned(v, src_stride, v_dtype) && rows_aligned(v, d, v_dtype) &&
                       al16(w) && al16(grad_out) && al16(dv) && al16(workspace) &&
                       (d * esize(v_dtype)) % 16 == 0;
  sy_plan p;
  rc = make_plan(SY_OP_BWD, n_src, 0, d, v_dtype, w_dtype, aligned, &p);
  if (rc != SY_OK) return rc;
  apply_tile_override(SY_OP_BWD, n_src, d, &p);
  int grid = 0;
  rc = bwd_grid(p, n_tok, v_dtype, stats != nullptr, &grid);
  if (rc != SY_OK) return rc;
  if (workspace == nullptr || workspace_bytes < (int64_t)grid * d * (int64_t)sizeof(float))
    return SY_ERR_WORKSPACE;
  const BwdArgs a{v, w, grad_out, stats, dv, nullptr, (float*)workspace, (int)n_src, n_tok, (int)d,
                  src_stride, v_dtype, w_dtype, eps};
  hipError_t e = p.family == SY_FAMILY_GENERIC ? launch_bwd_generic(a, grid, s)
                                               : bwd_vec(p, a, grid, s);
  if (e != hipSuccess) return (int)e;
  *rows_out = grid;
  return SY_OK;
}

int sy_bwd(const void* v, const void* w, const void* grad_out, const float* stats, void* dv,
           void* dw, void* workspace, int64_t workspace_bytes, int64_t n_src, int64_t n_tok,
           int64_t d, int64_t src_stride, int v_dtype, int w_dtype, float eps, void* stream) {
  // dw is written even when there are no tokens (it is then zero).
  if (dw == nullptr) return SY_ERR_NULL;
  const hipStream_t s = (hipStream_t)stream;
  int rows = 0;
  const int rc = bwd_main(v, w, grad_out, stats, dv, workspace, workspace_bytes, n_src, n_tok, d,
                          src_stride, v_dtype, w_dtype, eps, s, &rows);
  if (rc != SY_OK) return rc;
  return status(launch_dw_reduce((const float*)workspace, rows, (int)d, dw, w_dtype, s));
}

int sy_bwd_main(const void* v, const void* w, const void* grad_out, const float* stats, void* dv,
                void* workspace, int64_t workspace_bytes, int64_t n_src, int64_t n_tok, int64_t d,
                int64_t src_stride, int v_dtype, int w_dtype, float eps, void* stream) {
  int rows = 0;
  return bwd_main(v, w, grad_out, stats, dv, workspace, workspace_bytes, n_src, n_tok, d,
                  src_stride, v_dtype, w_dtype, eps, (hipStream_t)stream, &rows);
}

int64_t sy_bwd_partial_rows(int64_t n_src, int64_t n_tok, int64_t d, int v_dtype, int w_dtype,
                            int aligned, int has_stats) {
  int rc = check_common(n_src, n_tok, d, n_tok * d, v_dtype, w_dtype);
  if (rc != SY_OK) return rc;
  if (n_tok == 0) return 0;
  sy_plan p;
  rc = make_plan(SY_OP_BWD, n_src, 0, d, v_dtype, w_dtype, aligned, &p);
  if (rc != SY_OK) return rc;
  apply_tile_override(SY_OP_BWD, n_src, d, &p);
  int grid = 0;
  rc = bwd_grid(p, n_tok, v_dtype, has_stats != 0, &grid);
  return rc != SY_OK ? rc : grid;
}

int sy_kernel_info(int op, int64_t n_src, int64_t n_tok, int64_t d, int v_dtype, int w_dtype,
                   int32_t out[4]) {
  if (out == nullptr) return SY_ERR_NULL;
  int rc = check_common(n_src, n_tok, d, n_tok * d, v_dtype, w_dtype);
  if (rc != SY_OK) return rc;
  if (op != SY_OP_FWD && op != SY_OP_BWD) return SY_ERR_OP;
  sy_plan p;
  rc = make_plan(op, n_src, 0, d, v_dtype, w_dtype, 1, &p);
  if (rc != SY_OK) return rc;
  apply_tile_override(op, n_src, d, &p);
  out[0] = out[1] = out[2] = out[3] = 0;
  if (p.family == SY_FAMILY_GENERIC) return SY_OK;
  KernelRes r{0, 0, 0, 0};
  hipError_t e;
  if (op == SY_OP_FWD) {
    const FwdArgs a{nullptr, nullptr, nullptr, nullptr, (int)n_src, n_tok, (int)d, n_tok * d,
                    v_dtype, w_dtype, 0.0f};
    e = v_dtype == SY_BF16 ? launch_fwd_vec_bf16(p, a, nullptr, &r)
        : v_dtype == SY_F16 ? launch_fwd_vec_f16(p, a, nullptr, &r)
                            : launch_fwd_vec_f32(p, a, nullptr, &r);
  } else {
    e = bwd_resources(p, v_dtype, true, &r);
    if (e == hipSuccess) {
      rc = bwd_grid(p, n_tok, v_dtype, true, &r.grid);
      if (rc != SY_OK) return rc;
    }
  }
  if (e != hipSuccess) return e == hipErrorNoDevice ? SY_ERR_DEVICE : (int)e;
  out[0] = r.vgprs;
  out[1] = r.lds;
  out[2] = r.blocks_per_cu;
  out[3] = r.grid;
  return SY_OK;
}

int sy_dw_reduce(const float* partial, int64_t rows, int64_t d, void* dw, int w_dtype,
                 void* stream) {
  if (dw == nullptr || (rows > 0 && partial == nullptr)) return SY_ERR_NULL;
  if (!valid_dtype(w_dtype)) return SY_ERR_DTYPE;
  if (rows < 0 || rows > 0x7fffffff || d < 1 || d > 0x7fffffff / 16) return SY_ERR_SHAPE;
  return status(launch_dw_reduce(partial, (int)rows, (int)d, dw, w_dtype, (hipStream_t)stream));
}

int sy_fwd_batched(const void* v, const void* queries, void* out, int64_t n_src, int64_t n_q,
                   int64_t n_tok, int64_t d, int64_t src_stride, int dtype, float eps,
                   void* stream) {
  if (n_tok != 0 && (v == nullptr || queries == nullptr || out == nullptr)) return SY_ERR_NULL;
  int rc = check_common(n_src, n_tok, d, src_stride, dtype, dtype);
  if (rc != SY_OK) return rc;
  if (n_q < 1 || n_q > 0x7fffffff) return SY_ERR_SHAPE;
  const bool aligned = rows_aligned(v, src_stride, dtype) && rows_aligned(v, d, dtype) &&
                       al16(queries) && al16(out) && (d * esize(dtype)) % 16 == 0;
  sy_plan p;
  rc = make_plan(SY_OP_BATCHED, n_src, n_q, d, dtype, dtype, aligned, &p);
  if (rc != SY_OK) return rc;
  apply_tile_override(SY_OP_BATCHED, n_src, d, &p);
  if (n_tok == 0) return SY_OK;
  const hipStream_t s = (hipStream_t)stream;
  if (p.family == SY_FAMILY_RESIDENT) {
    const BatchedArgs a{v, queries, out, (int)n_src, (int)n_q, n_tok, (int)d, src_stride, dtype, eps};
    return status(batched_vec(p, a, s));
  }
  // One forward launch per query, written straight into out[s].
  const int64_t es = esize(dtype);
  for (int64_t q = 0; q < n_q; ++q) {
    rc = sy_fwd(v, (const char*)queries + q * d * es, (char*)out + q * n_tok * d * es, nullptr,
                n_src, n_tok, d, src_stride, dtype, dtype, eps, stream);
    if (rc != SY_OK) return rc;
  }
  return SY_OK;
}

int64_t sy_probe_grid(int64_t bytes) {
  // 256 threads x 4 chunks in flight per workgroup; up to 32768 workgroups
  // (the grid that reached the highest read bandwidth on MI355X).
  if (bytes <= 0) return 1;
  const int64_t g = (bytes / 16 + 1023) / 1024;
  return g < 1 ? 1 : (g > 32768 ? 32768 : g);
}

int sy_bw_probe(int kind, const void* src, void* dst, int64_t bytes, void* stream) {
  if (kind < 0 || kind > 2) return SY_ERR_OP;
  if (bytes <= 0 || bytes % 16 != 0) return SY_ERR_SHAPE;
  if ((kind != 1 && src == nullptr) || dst == nullptr) return SY_ERR_NULL;
  if ((kind != 1 && !al16(src)) || (kind != 0 && !al16(dst))) return SY_ERR_SHAPE;
  return status(launch_probe(kind, src, dst, bytes, (int)sy_probe_grid(bytes), (hipStream_t)stream));
}

const char* sy_strerror(int code) {
  switch (code) {
    case SY_OK: return "success";
    case SY_ERR_NULL: return "switchyard: a required pointer is NULL";
    case SY_ERR_SHAPE: return "switchyard: a size is out of range";
    case SY_ERR_DTYPE: return "switchyard: unsupported dtype";
    case SY_ERR_WORKSPACE: return "switchyard: backward workspace missing or too small";
    case SY_ERR_STRIDE: return "switchyard: source stride smaller than n_tok * D";
    case SY_ERR_DEVICE: return "switchyard: no usable HIP device";
    case SY_ERR_OP: return "switchyard: unknown operation";
    default: break;
  }
  if (code > 0) return hipGetErrorString((hipError_t)code);
  return "switchyard: unknown status";
}

}  // extern "C"
