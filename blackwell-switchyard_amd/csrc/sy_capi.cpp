// The C ABI (include/switchyard.h): argument checks, planning and launches.
// Every check that can be made on the host is made before any device work,
// so bad arguments come back as negative sy_status codes. Nothing here
// allocates device memory.
#include <atomic>
#include <map>
#include <mutex>

#include "../../include/switchyard.h"
#include "sy_launch.hpp"

// Workspace of sy_bwd_static: the dw partial rows of callers that cannot
// allocate. One copy per GPU, at that GPU's own address; host code uses the
// address hipGetSymbolAddress returns for the current device, never this name.
static __device__ __align__(256) float scratch[SY_STATIC_WORKSPACE_BYTES / sizeof(float)];

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

// Device address of `scratch` per device (resolved on the first sy_bwd_static
// call on that device, with the device current).
std::mutex g_scratch_mu;
std::map<int, void*> g_scratch;

// Measurement overrides (sy_tuning_set). g_tuning_on is read on every launch
// without the lock; the struct itself only under it.
std::mutex g_tuning_mu;
std::atomic<bool> g_tuning_on{false};
sy_tuning g_tuning{};

// variant: 0 operator over stacked rows, 1 over per-row pointers, 2 the
// (o, m, l) gradient over stacked rows (BwdVariant in sy_kernels.hpp).
hipError_t bwd_resources(const sy_plan& p, int dtype, bool stats, int variant, KernelRes* out) {
  if (dtype == SY_BF16) return bwd_vec_resources_bf16(p, stats, variant, out);
  if (dtype == SY_F16) return bwd_vec_resources_f16(p, stats, variant, out);
  return bwd_vec_resources_f32(p, stats, variant, out);
}

// Persistent workgroup count of the backward: every CU filled at the
// kernel's register/LDS occupancy, never more than there are token slots.
// Deterministic in (plan, n_tok, stats, addressing, device), which keeps dw
// bit-stable.
int bwd_grid(const sy_plan& p, int64_t n_tok, int dtype, bool stats, int variant, int* grid) {
  int cus = 0;
  hipError_t e = cu_count(&cus);
  if (e != hipSuccess) return e == hipErrorNoDevice ? SY_ERR_DEVICE : (int)e;
  int per_cu = 4;
  if (p.family != SY_FAMILY_GENERIC) {
    KernelRes r;
    e = bwd_resources(p, dtype, stats, variant, &r);
    if (e != hipSuccess) return (int)e;
    per_cu = r.blocks_per_cu;
  }
  // Measurement override (sy_tuning_set): workgroups per CU of the persistent grid.
  sy_tuning t;
  if (tuning_snapshot(&t) && t.bwd_blocks_per_cu > 0) per_cu = t.bwd_blocks_per_cu;
  const int64_t slots = (n_tok + p.tokens_per_block - 1) / p.tokens_per_block;
  int64_t g = (int64_t)cus * per_cu;
  if (g > slots) g = slots;
  if (g < 1) g = 1;
  *grid = (int)g;
  return SY_OK;
}

// The backward's plan for a launch: the shape's plan with the token-count
// rule and any override applied; a 32-row tile (which exists for the stacked
// operator gradient with stats only) becomes the generic kernel for every
// other caller.
int bwd_plan(int64_t n_src, int64_t n_tok, int64_t d, int v_dtype, int w_dtype, int aligned,
             bool stats, int variant, sy_plan* p) {
  int rc = make_plan(SY_OP_BWD, n_src, 0, d, v_dtype, w_dtype, aligned, p, stats);
  if (rc != SY_OK) return rc;
  apply_tile_rules(SY_OP_BWD, n_src, n_tok, d, p);
  if (p->family != SY_FAMILY_GENERIC && p->rows_per_tile > 16 && (!stats || variant != 0))
    rc = make_plan(SY_OP_BWD, n_src, 0, d, v_dtype, w_dtype, 0, p, stats);
  return rc;
}

// Partial rows the backward's workspace provides: the largest persistent
// grid of the plans an aligned call takes (every variant, with and without
// forward stats) -- vector tiles, and the generic kernel where an aligned
// variant has no tile (17 <= N <= 32 without stats, over per-row pointers or
// for the (o, m, l) gradient; every variant past 32 rows). A call whose buffers
// are not 16-byte aligned also runs the generic kernel, which is persistent
// over tokens at any grid and is capped to this count, so misalignment alone
// does not widen the workspace (2 MiB instead of 8 at N=9, D=2048 on 256 CUs).
// Capping the aligned generic variants to the 32-row tile's grid instead ran
// them 3x slower (N=24 / N=32 at T=4096, D=2048, no stats, on MI355X: 3070 /
// 4060 us on 256 workgroups against 976 / 1323 us on 1024).
int workspace_rows(int64_t n_src, int64_t n_tok, int64_t d, int v_dtype, int w_dtype, int* rows) {
  int g = 0;
  for (bool st : {true, false}) {
    for (int var : {0, 1, 2}) {
      sy_plan p;
      int rc = bwd_plan(n_src, n_tok, d, v_dtype, w_dtype, 1, st, var, &p);
      if (rc != SY_OK) return rc;
      int gi = 0;
      rc = bwd_grid(p, n_tok, v_dtype, st, var, &gi);
      if (rc != SY_OK) return rc;
      if (gi > g) g = gi;
    }
  }
  *rows = g;
  return SY_OK;
}

// The backward's grid for plan p: bwd_grid, capped to workspace_rows for the
// generic kernel.
int bwd_grid_for(const sy_plan& p, int64_t n_src, int64_t n_tok, int64_t d, int v_dtype,
                 int w_dtype, bool stats, int variant, int* grid) {
  int rc = bwd_grid(p, n_tok, v_dtype, stats, variant, grid);
  if (rc != SY_OK || p.family != SY_FAMILY_GENERIC) return rc;
  int rows = 0;
  rc = workspace_rows(n_src, n_tok, d, v_dtype, w_dtype, &rows);
  if (rc != SY_OK) return rc;
  if (*grid > rows) *grid = rows;
  return SY_OK;
}

// Plan of the batched backward for this token count: the matrix-core kernel
// only where its dv offsets fit.
int bwd_batched_plan(int64_t n_src, int64_t n_q, int64_t n_tok, int64_t d, int dtype, int aligned,
                     int64_t v_stride_bytes, sy_plan* p) {
  int rc = make_plan(SY_OP_BWD_BATCHED, n_src, n_q, d, dtype, dtype, aligned, p);
  if (rc == SY_OK && p->family == SY_FAMILY_MATRIX &&
      !bwd_matrix_offsets_fit(n_src, n_tok, d, v_stride_bytes))
    rc = make_plan(SY_OP_BWD_BATCHED, n_src, n_q, d, dtype, dtype, aligned, p, 1, 0);
  return rc;
}

// Persistent grid of the batched backward (also sizes its workspace).
int bwd_batched_grid(const sy_plan& p, int64_t n_src, int64_t n_q, int64_t n_tok, int64_t d,
                     int dtype, int* grid) {
  int cus = 0;
  hipError_t e = cu_count(&cus);
  if (e != hipSuccess) return e == hipErrorNoDevice ? SY_ERR_DEVICE : (int)e;
  if (p.family == SY_FAMILY_MATRIX) {
    BwdBatchedArgs a{};
    a.n_src = (int)n_src;
    a.n_q = (int)n_q;
    a.n_tok = n_tok;
    a.d = (int)d;
    a.dtype = dtype;
    KernelRes r;
    e = launch_bwd_batched_matrix(a, 0, nullptr, &r);
    if (e != hipSuccess) return (int)e;
    *grid = r.grid;
    return SY_OK;
  }
  int per_cu = 2;
  if (p.family != SY_FAMILY_GENERIC) {
    KernelRes r;
    e = dtype == SY_BF16 ? bwd_batched_vec_resources_bf16(p, &r)
        : dtype == SY_F16 ? bwd_batched_vec_resources_f16(p, &r)
                          : bwd_batched_vec_resources_f32(p, &r);
    if (e != hipSuccess) return (int)e;
    per_cu = r.blocks_per_cu;
  }
  const int64_t slots = (n_tok + p.tokens_per_block - 1) / p.tokens_per_block;
  int64_t g = (int64_t)cus * per_cu;
  if (g > slots) g = slots;
  if (g < 1) g = 1;
  *grid = (int)g;
  return SY_OK;
}

// Partial-row groups sy_bwd_batched_workspace_bytes provides: the grid of the
// plan an aligned call takes when the matrix kernel's offsets fit. The other
// plans (a source stride past the matrix kernel's 32-bit offsets, misaligned
// buffers) are persistent over tokens at any grid and are capped to it.
int batched_workspace_rows(int64_t n_src, int64_t n_q, int64_t n_tok, int64_t d, int dtype,
                           int* rows) {
  sy_plan p;
  const int rc = make_plan(SY_OP_BWD_BATCHED, n_src, n_q, d, dtype, dtype, 1, &p, 1, 1);
  if (rc != SY_OK) return rc;
  return bwd_batched_grid(p, n_src, n_q, n_tok, d, dtype, rows);
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
int check_sizes(int64_t n_src, int64_t n_tok, int64_t d, int v_dtype, int w_dtype) {
  if (!valid_dtype(v_dtype) || !valid_dtype(w_dtype)) return SY_ERR_DTYPE;
  if (n_src < 1 || d < 1 || n_tok < 0) return SY_ERR_SHAPE;
  if (n_src > 0x7fffffff || d > 0x7fffffff / 16 || n_tok > ((int64_t)1 << 40)) return SY_ERR_SHAPE;
  return SY_OK;
}
int check_common(int64_t n_src, int64_t n_tok, int64_t d, int64_t src_stride, int v_dtype,
                 int w_dtype) {
  const int rc = check_sizes(n_src, n_tok, d, v_dtype, w_dtype);
  if (rc != SY_OK) return rc;
  if (n_src > 1 && src_stride < n_tok * d) return SY_ERR_STRIDE;
  return SY_OK;
}

// Row tables. `rows_ok` reports whether every row start is 16-byte aligned so
// that the vector kernels may be used (token rows then stay aligned when
// D * itemsize is a multiple of 16, checked by the callers).
RowTable stacked_rows(const void* base, int64_t n_src, int64_t stride, int dtype, bool* rows_ok) {
  RowTable t{};
  const int64_t sb = stride * esize(dtype);
  for (int n = 0; n < kTableRows && n < n_src; ++n)
    t.p[n] = const_cast<char*>(static_cast<const char*>(base)) + n * sb;
  t.stride_bytes = sb;
  *rows_ok = al16(base) && sb % 16 == 0;
  return t;
}

// A caller's list of N row pointers (N <= kTableRows). SY_ERR_NULL if any is NULL.
int listed_rows(const void* const* rows, int64_t n_src, RowTable* t, bool* rows_ok) {
  *t = RowTable{};
  *rows_ok = true;
  if (rows == nullptr) return SY_ERR_NULL;
  if (n_src > kTableRows) return SY_ERR_SHAPE;
  for (int n = 0; n < n_src; ++n) {
    if (rows[n] == nullptr) return SY_ERR_NULL;
    t->p[n] = const_cast<void*>(rows[n]);
    *rows_ok = *rows_ok && al16(rows[n]);
  }
  return SY_OK;
}

}  // namespace

// The current device's copy of `scratch`. Errors: SY_ERR_DEVICE without a
// device, or the hipError_t of the symbol lookup.
int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e == hipErrorNoDevice ? SY_ERR_DEVICE : (int)e;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  auto it = g_scratch.find(dev);
  if (it != g_scratch.end()) {
    *out = it->second;
    return SY_OK;
  }
  void* p = nullptr;
  e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || p == nullptr) return e != hipSuccess ? (int)e : SY_ERR_DEVICE;
  g_scratch[dev] = p;
  *out = p;
  return SY_OK;
}

bool tuning_snapshot(sy_tuning* out) {
  if (!g_tuning_on.load(std::memory_order_acquire)) return false;
  std::lock_guard<std::mutex> lk(g_tuning_mu);
  if (!g_tuning_on.load(std::memory_order_relaxed)) return false;
  *out = g_tuning;
  return true;
}

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

namespace {

bool vec_rows(bool rows_ok, int64_t d, int dtype) { return rows_ok && (d * esize(dtype)) % 16 == 0; }

// Forward of the operator (normalize = 1) or of attn_with_stats (normalize = 0
// with m_out/l_out) over any row table. Sizes are already checked.
int fwd_impl(const RowTable& v, bool v_ok, const void* w, void* out, float* stats, float* m_out,
             float* l_out, int normalize, int64_t n_src, int64_t n_tok, int64_t d, int v_dtype,
             int w_dtype, float eps, hipStream_t s) {
  const bool aligned = vec_rows(v_ok, d, v_dtype) && al16(w) && al16(out);
  sy_plan p;
  const int rc = make_plan(SY_OP_FWD, n_src, 0, d, v_dtype, w_dtype, aligned, &p);
  if (rc != SY_OK) return rc;
  apply_tile_rules(SY_OP_FWD, n_src, n_tok, d, &p);
  if (n_tok == 0) return SY_OK;
  const FwdArgs a{v,      w,       out,     stats,   m_out, l_out, normalize, (int)n_src,
                  n_tok,  (int)d,  v_dtype, w_dtype, eps};
  return status(p.family == SY_FAMILY_GENERIC ? launch_fwd_generic(a, s) : fwd_vec(p, a, s));
}

// Main backward kernel over row tables: dv and the fp32 dw partials.
// *rows_out receives the partial row count (the persistent grid).
int bwd_main_impl(const RowTable& v, bool v_ok, const void* w, const void* g, const float* stats,
                  const float* gm, const float* gl, const RowTable& dv, bool dv_ok, bool listed,
                  void* workspace, int64_t workspace_bytes, int64_t n_src, int64_t n_tok,
                  int64_t d, int v_dtype, int w_dtype, float eps, hipStream_t s, int* rows_out) {
  *rows_out = 0;
  if (n_tok == 0) return SY_OK;
  const bool aligned = vec_rows(v_ok && dv_ok, d, v_dtype) && al16(w) && al16(g) && al16(workspace);
  sy_plan p;
  const int variant = listed ? 1 : (gm != nullptr ? 2 : 0);
  int rc = bwd_plan(n_src, n_tok, d, v_dtype, w_dtype, aligned, stats != nullptr, variant, &p);
  if (rc != SY_OK) return rc;
  int grid = 0;
  rc = bwd_grid_for(p, n_src, n_tok, d, v_dtype, w_dtype, stats != nullptr, variant, &grid);
  if (rc != SY_OK) return rc;
  if (workspace == nullptr || workspace_bytes < (int64_t)grid * d * (int64_t)sizeof(float))
    return SY_ERR_WORKSPACE;
  const BwdArgs a{v,      w,       g,     stats,  gm,      gl,      dv,  (float*)workspace, listed,
                  (int)n_src, n_tok, (int)d, v_dtype, w_dtype, eps};
  const hipError_t e =
      p.family == SY_FAMILY_GENERIC ? launch_bwd_generic(a, grid, s) : bwd_vec(p, a, grid, s);
  if (e != hipSuccess) return (int)e;
  *rows_out = grid;
  return SY_OK;
}

// Main kernel then the fixed-order dw reduction (dw is written even with no
// tokens: it is then zero).
int bwd_impl(const RowTable& v, bool v_ok, const void* w, const void* g, const float* stats,
             const float* gm, const float* gl, const RowTable& dv, bool dv_ok, bool listed, void* dw,
             void* workspace, int64_t workspace_bytes, int64_t n_src, int64_t n_tok, int64_t d,
             int v_dtype, int w_dtype, float eps, hipStream_t s) {
  int rows = 0;
  const int rc = bwd_main_impl(v, v_ok, w, g, stats, gm, gl, dv, dv_ok, listed, workspace,
                               workspace_bytes, n_src, n_tok, d, v_dtype, w_dtype, eps, s, &rows);
  if (rc != SY_OK) return rc;
  return status(launch_dw_reduce((const float*)workspace, rows, (int)d, dw, w_dtype, s));
}

// Batched forward: the resident kernel, else one forward launch per query
// written straight into out[q] (and m_out[q], l_out[q]).
int batched_impl(const RowTable& v, bool v_ok, const void* q, void* out, float* m_out, float* l_out,
                 int normalize, int64_t n_src, int64_t n_q, int64_t n_tok, int64_t d, int dtype,
                 float eps, hipStream_t s) {
  const bool aligned = vec_rows(v_ok, d, dtype) && al16(q) && al16(out);
  sy_plan p;
  int rc = make_plan(SY_OP_BATCHED, n_src, n_q, d, dtype, dtype, aligned, &p);
  if (rc != SY_OK) return rc;
  apply_tile_override(SY_OP_BATCHED, n_src, d, &p);
  if (n_tok == 0) return SY_OK;
  // The matrix kernel's store offsets are 32-bit; past that, per-query launches.
  if (p.family == SY_FAMILY_MATRIX && !matrix_batched_offsets_fit(n_q, n_tok, d))
    p.family = SY_FAMILY_PER_QUERY;
  if (p.family == SY_FAMILY_RESIDENT || p.family == SY_FAMILY_MATRIX) {
    const BatchedArgs a{v,          q,        out,   m_out,  l_out, normalize,
                        (int)n_src, (int)n_q, n_tok, (int)d, dtype, eps};
    return status(p.family == SY_FAMILY_MATRIX ? launch_batched_matrix(a, s, nullptr)
                                               : batched_vec(p, a, s));
  }
  const int64_t es = esize(dtype);
  for (int64_t k = 0; k < n_q; ++k) {
    rc = fwd_impl(v, v_ok, (const char*)q + k * d * es, (char*)out + k * n_tok * d * es, nullptr,
                  m_out ? m_out + k * n_tok : nullptr, l_out ? l_out + k * n_tok : nullptr,
                  normalize, n_src, n_tok, d, dtype, dtype, eps, s);
    if (rc != SY_OK) return rc;
  }
  return SY_OK;
}

// Stacked-layout source table with the stride check already done.
RowTable stacked(const void* v, int64_t n_src, int64_t stride, int dtype, bool* ok) {
  return stacked_rows(v, n_src, stride, dtype, ok);
}

// Pointer-list source table: sizes checked, N within the table.
int listed(const void* const* rows, int64_t n_src, int64_t n_tok, RowTable* t, bool* ok) {
  if (n_src > kTableRows) return SY_ERR_SHAPE;
  if (n_tok == 0) {
    *t = RowTable{};
    *ok = true;
    return SY_OK;
  }
  return listed_rows(rows, n_src, t, ok);
}

}  // namespace

extern "C" {

int sy_abi_version(void) { return SY_ABI_VERSION; }

int sy_plan_for(int op, int64_t n_src, int64_t n_q, int64_t d, int v_dtype, int w_dtype,
                int aligned, sy_plan* out) {
  return make_plan(op, n_src, n_q, d, v_dtype, w_dtype, aligned, out);
}

int sy_plan_for_tokens(int op, int64_t n_src, int64_t n_q, int64_t n_tok, int64_t d, int v_dtype,
                       int w_dtype, int aligned, sy_plan* out) {
  if (out == nullptr) return SY_ERR_NULL;
  if (n_tok < 0) return SY_ERR_SHAPE;
  const int rc = make_plan(op, n_src, n_q, d, v_dtype, w_dtype, aligned, out);
  if (rc != SY_OK) return rc;
  if (op == SY_OP_FWD || op == SY_OP_BWD) apply_tile_rules(op, n_src, n_tok, d, out);
  return SY_OK;
}

int sy_fwd(const void* v, const void* w, void* out, float* stats, int64_t n_src, int64_t n_tok,
           int64_t d, int64_t src_stride, int v_dtype, int w_dtype, float eps, void* stream) {
  // Empty tensors have NULL data pointers; with no tokens nothing is touched.
  if (n_tok != 0 && (v == nullptr || w == nullptr || out == nullptr)) return SY_ERR_NULL;
  const int rc = check_common(n_src, n_tok, d, src_stride, v_dtype, w_dtype);
  if (rc != SY_OK) return rc;
  bool ok = false;
  const RowTable t = stacked(v, n_src, src_stride, v_dtype, &ok);
  return fwd_impl(t, ok, w, out, stats, nullptr, nullptr, 1, n_src, n_tok, d, v_dtype, w_dtype, eps,
                  (hipStream_t)stream);
}

int sy_fwd_table(const void* const* v_rows, const void* w, void* out, float* stats, int64_t n_src,
                 int64_t n_tok, int64_t d, int v_dtype, int w_dtype, float eps, void* stream) {
  if (n_tok != 0 && (v_rows == nullptr || w == nullptr || out == nullptr)) return SY_ERR_NULL;
  int rc = check_sizes(n_src, n_tok, d, v_dtype, w_dtype);
  if (rc != SY_OK) return rc;
  RowTable t;
  bool ok = false;
  rc = listed(v_rows, n_src, n_tok, &t, &ok);
  if (rc != SY_OK) return rc;
  return fwd_impl(t, ok, w, out, stats, nullptr, nullptr, 1, n_src, n_tok, d, v_dtype, w_dtype, eps,
                  (hipStream_t)stream);
}

int sy_attn_with_stats(const void* v, const void* w, void* o, float* m, float* l, float* stats,
                       int64_t n_src, int64_t n_tok, int64_t d, int64_t src_stride, int v_dtype,
                       int w_dtype, float eps, void* stream) {
  if (n_tok != 0 &&
      (v == nullptr || w == nullptr || o == nullptr || m == nullptr || l == nullptr))
    return SY_ERR_NULL;
  const int rc = check_common(n_src, n_tok, d, src_stride, v_dtype, w_dtype);
  if (rc != SY_OK) return rc;
  bool ok = false;
  const RowTable t = stacked(v, n_src, src_stride, v_dtype, &ok);
  return fwd_impl(t, ok, w, o, stats, m, l, 0, n_src, n_tok, d, v_dtype, w_dtype, eps,
                  (hipStream_t)stream);
}

int sy_attn_with_stats_merge(const void* v, const void* w, const void* o1, const float* m1,
                             const float* l1, void* out, float* m, float* l, int64_t n_src,
                             int64_t n_tok, int64_t d, int64_t src_stride, int v_dtype,
                             int w_dtype, float eps, int normalize, void* stream) {
  if (n_tok != 0 && (v == nullptr || w == nullptr || o1 == nullptr || m1 == nullptr ||
                     l1 == nullptr || out == nullptr || m == nullptr || l == nullptr))
    return SY_ERR_NULL;
  int rc = check_common(n_src, n_tok, d, src_stride, v_dtype, w_dtype);
  if (rc != SY_OK) return rc;
  if (normalize != 0 && normalize != 1) return SY_ERR_OP;
  bool ok = false;
  RowTable t = stacked(v, n_src, src_stride, v_dtype, &ok);
  const hipStream_t s = (hipStream_t)stream;
  // The prior's o1 rides in the register tile as row n_src: a resident tile
  // of n_src + 1 rows, addressed through the table's row pointers.
  const bool aligned = vec_rows(ok, d, v_dtype) && al16(w) && al16(out) && al16(o1);
  sy_plan p;
  rc = make_plan(SY_OP_FWD, n_src + 1, 0, d, v_dtype, w_dtype, aligned, &p);
  if (rc != SY_OK) return rc;
  apply_tile_rules(SY_OP_FWD, n_src + 1, n_tok, d, &p, /*chunked_ok=*/false);
  if (n_tok == 0) return SY_OK;
  if (p.family == SY_FAMILY_RESIDENT && n_src + 1 <= kTableRows && p.rows_per_tile >= n_src + 1) {
    t.p[n_src] = const_cast<void*>(o1);
    FwdArgs a{t,      w,       out,     nullptr, m,  l,  normalize, (int)n_src,
              n_tok,  (int)d,  v_dtype, w_dtype, eps, m1, l1};
    return status(fwd_vec(p, a, s));
  }
  // Beyond the resident tiles (more rows, unaligned rows, mixed dtypes): this
  // group's (o, m, l) into out, m, l, then the merge over them in place.
  rc = fwd_impl(t, ok, w, out, nullptr, m, l, 0, n_src, n_tok, d, v_dtype, w_dtype, eps, s);
  if (rc != SY_OK) return rc;
  const bool vec = al16(o1) && al16(out) && (d * esize(v_dtype)) % 16 == 0;
  MergeArgs ma{o1, m1, l1, out, m, l, out, m, l, n_tok, (int)d};
  ma.normalize = normalize;
  return status(launch_merge(ma, v_dtype, vec, s));
}

int sy_sol(const void* v, void* out, int64_t n_src, int64_t n_tok, int64_t d, int64_t src_stride,
           int dtype, void* stream) {
  if (n_tok != 0 && (v == nullptr || out == nullptr)) return SY_ERR_NULL;
  int rc = check_common(n_src, n_tok, d, src_stride, dtype, dtype);
  if (rc != SY_OK) return rc;
  bool ok = false;
  const RowTable t = stacked(v, n_src, src_stride, dtype, &ok);
  const bool aligned = vec_rows(ok, d, dtype) && al16(out);
  sy_plan p;
  rc = make_plan(SY_OP_SOL, n_src, 0, d, dtype, dtype, aligned, &p);
  if (rc != SY_OK) return rc;
  apply_tile_override(SY_OP_SOL, n_src, d, &p);
  if (n_tok == 0) return SY_OK;
  const FwdArgs a{t,     nullptr, out,   nullptr, nullptr, nullptr, 1, (int)n_src,
                  n_tok, (int)d,  dtype, dtype,   0.0f};
  const hipStream_t s = (hipStream_t)stream;
  return status(p.family == SY_FAMILY_GENERIC ? launch_sol_generic(a, s) : sol_vec(p, a, s));
}

int64_t sy_bwd_workspace_bytes(int64_t n_src, int64_t n_tok, int64_t d, int v_dtype, int w_dtype) {
  int rc = check_sizes(n_src, n_tok, d, v_dtype, w_dtype);
  if (rc != SY_OK) return rc;
  if (n_tok == 0) return 0;
  int rows = 0;
  rc = workspace_rows(n_src, n_tok, d, v_dtype, w_dtype, &rows);
  if (rc != SY_OK) return rc;
  return rows * d * (int64_t)sizeof(float);
}

int sy_bwd(const void* v, const void* w, const void* grad_out, const float* stats, void* dv,
           void* dw, void* workspace, int64_t workspace_bytes, int64_t n_src, int64_t n_tok,
           int64_t d, int64_t src_stride, int v_dtype, int w_dtype, float eps, void* stream) {
  if (dw == nullptr) return SY_ERR_NULL;
  if (n_tok != 0 && (v == nullptr || w == nullptr || grad_out == nullptr || dv == nullptr))
    return SY_ERR_NULL;
  const int rc = check_common(n_src, n_tok, d, src_stride, v_dtype, w_dtype);
  if (rc != SY_OK) return rc;
  bool vok = false, dok = false;
  const RowTable tv = stacked(v, n_src, src_stride, v_dtype, &vok);
  const RowTable td = stacked(dv, n_src, n_tok * d, v_dtype, &dok);
  return bwd_impl(tv, vok, w, grad_out, stats, nullptr, nullptr, td, dok, false, dw, workspace,
                  workspace_bytes, n_src, n_tok, d, v_dtype, w_dtype, eps, (hipStream_t)stream);
}

int sy_bwd_static(const void* v, const void* w, const void* grad_out, const float* stats, void* dv,
                  void* dw, int64_t n_src, int64_t n_tok, int64_t d, int64_t src_stride, int v_dtype,
                  int w_dtype, float eps, void* stream) {
  if (dw == nullptr) return SY_ERR_NULL;
  if (n_tok != 0 && (v == nullptr || w == nullptr || grad_out == nullptr || dv == nullptr))
    return SY_ERR_NULL;
  int rc = check_common(n_src, n_tok, d, src_stride, v_dtype, w_dtype);
  if (rc != SY_OK) return rc;
  if (n_tok != 0) {
    // The size the array must hold, as sy_bwd_workspace_bytes reports it.
    int rows = 0;
    rc = workspace_rows(n_src, n_tok, d, v_dtype, w_dtype, &rows);
    if (rc != SY_OK) return rc;
    if ((int64_t)rows * d * (int64_t)sizeof(float) > SY_STATIC_WORKSPACE_BYTES) return SY_ERR_WORKSPACE;
  }
  void* ws = nullptr;
  rc = scratch_address(&ws);
  if (rc != SY_OK) return rc;
  bool vok = false, dok = false;
  const RowTable tv = stacked(v, n_src, src_stride, v_dtype, &vok);
  const RowTable td = stacked(dv, n_src, n_tok * d, v_dtype, &dok);
  return bwd_impl(tv, vok, w, grad_out, stats, nullptr, nullptr, td, dok, false, dw, ws,
                  SY_STATIC_WORKSPACE_BYTES, n_src, n_tok, d, v_dtype, w_dtype, eps,
                  (hipStream_t)stream);
}

int sy_bwd_table(const void* const* v_rows, const void* w, const void* grad_out,
                 const float* stats, void* const* dv_rows, void* dw, void* workspace,
                 int64_t workspace_bytes, int64_t n_src, int64_t n_tok, int64_t d, int v_dtype,
                 int w_dtype, float eps, void* stream) {
  if (dw == nullptr) return SY_ERR_NULL;
  if (n_tok != 0 &&
      (v_rows == nullptr || w == nullptr || grad_out == nullptr || dv_rows == nullptr))
    return SY_ERR_NULL;
  int rc = check_sizes(n_src, n_tok, d, v_dtype, w_dtype);
  if (rc != SY_OK) return rc;
  RowTable tv, td;
  bool vok = false, dok = false;
  rc = listed(v_rows, n_src, n_tok, &tv, &vok);
  if (rc != SY_OK) return rc;
  rc = listed(reinterpret_cast<const void* const*>(dv_rows), n_src, n_tok, &td, &dok);
  if (rc != SY_OK) return rc;
  return bwd_impl(tv, vok, w, grad_out, stats, nullptr, nullptr, td, dok, true, dw, workspace,
                  workspace_bytes, n_src, n_tok, d, v_dtype, w_dtype, eps, (hipStream_t)stream);
}

int sy_attn_with_stats_bwd(const void* v, const void* w, const void* grad_o, const float* grad_m,
                           const float* grad_l, const float* stats, void* dv, void* dw,
                           void* workspace, int64_t workspace_bytes, int64_t n_src, int64_t n_tok,
                           int64_t d, int64_t src_stride, int v_dtype, int w_dtype, float eps,
                           void* stream) {
  if (dw == nullptr) return SY_ERR_NULL;
  if (n_tok != 0 && (v == nullptr || w == nullptr || grad_o == nullptr || grad_m == nullptr ||
                     grad_l == nullptr || dv == nullptr))
    return SY_ERR_NULL;
  const int rc = check_common(n_src, n_tok, d, src_stride, v_dtype, w_dtype);
  if (rc != SY_OK) return rc;
  bool vok = false, dok = false;
  const RowTable tv = stacked(v, n_src, src_stride, v_dtype, &vok);
  const RowTable td = stacked(dv, n_src, n_tok * d, v_dtype, &dok);
  return bwd_impl(tv, vok, w, grad_o, stats, grad_m, grad_l, td, dok, false, dw, workspace,
                  workspace_bytes, n_src, n_tok, d, v_dtype, w_dtype, eps, (hipStream_t)stream);
}

int sy_bwd_main(const void* v, const void* w, const void* grad_out, const float* stats, void* dv,
                void* workspace, int64_t workspace_bytes, int64_t n_src, int64_t n_tok, int64_t d,
                int64_t src_stride, int v_dtype, int w_dtype, float eps, void* stream) {
  if (n_tok != 0 && (v == nullptr || w == nullptr || grad_out == nullptr || dv == nullptr))
    return SY_ERR_NULL;
  const int rc = check_common(n_src, n_tok, d, src_stride, v_dtype, w_dtype);
  if (rc != SY_OK) return rc;
  bool vok = false, dok = false;
  const RowTable tv = stacked(v, n_src, src_stride, v_dtype, &vok);
  const RowTable td = stacked(dv, n_src, n_tok * d, v_dtype, &dok);
  int rows = 0;
  return bwd_main_impl(tv, vok, w, grad_out, stats, nullptr, nullptr, td, dok, false, workspace,
                       workspace_bytes, n_src, n_tok, d, v_dtype, w_dtype, eps,
                       (hipStream_t)stream, &rows);
}

int64_t sy_bwd_partial_rows(int64_t n_src, int64_t n_tok, int64_t d, int v_dtype, int w_dtype,
                            int aligned, int has_stats) {
  int rc = check_sizes(n_src, n_tok, d, v_dtype, w_dtype);
  if (rc != SY_OK) return rc;
  if (n_tok == 0) return 0;
  sy_plan p;
  rc = bwd_plan(n_src, n_tok, d, v_dtype, w_dtype, aligned, has_stats != 0, 0, &p);
  if (rc != SY_OK) return rc;
  int grid = 0;
  rc = bwd_grid_for(p, n_src, n_tok, d, v_dtype, w_dtype, has_stats != 0, 0, &grid);
  return rc != SY_OK ? rc : grid;
}

int sy_kernel_info(int op, int64_t n_src, int64_t n_tok, int64_t d, int v_dtype, int w_dtype,
                   int32_t out[4]) {
  if (out == nullptr) return SY_ERR_NULL;
  int rc = check_sizes(n_src, n_tok, d, v_dtype, w_dtype);
  if (rc != SY_OK) return rc;
  if (op != SY_OP_FWD && op != SY_OP_BWD) return SY_ERR_OP;
  sy_plan p;
  rc = make_plan(op, n_src, 0, d, v_dtype, w_dtype, 1, &p);
  if (rc != SY_OK) return rc;
  apply_tile_rules(op, n_src, n_tok, d, &p);
  out[0] = out[1] = out[2] = out[3] = 0;
  if (p.family == SY_FAMILY_GENERIC) return SY_OK;
  KernelRes r{0, 0, 0, 0};
  hipError_t e;
  if (op == SY_OP_FWD) {
    const FwdArgs a{RowTable{}, nullptr, nullptr, nullptr, nullptr, nullptr, 1, (int)n_src,
                    n_tok,      (int)d,  v_dtype, w_dtype, 0.0f};
    e = v_dtype == SY_BF16 ? launch_fwd_vec_bf16(p, a, nullptr, &r)
        : v_dtype == SY_F16 ? launch_fwd_vec_f16(p, a, nullptr, &r)
                            : launch_fwd_vec_f32(p, a, nullptr, &r);
  } else {
    e = bwd_resources(p, v_dtype, true, 0, &r);
    if (e == hipSuccess) {
      rc = bwd_grid(p, n_tok, v_dtype, true, 0, &r.grid);
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
  const int rc = check_common(n_src, n_tok, d, src_stride, dtype, dtype);
  if (rc != SY_OK) return rc;
  if (n_q < 1 || n_q > 0x7fffffff) return SY_ERR_SHAPE;
  bool ok = false;
  const RowTable t = stacked(v, n_src, src_stride, dtype, &ok);
  return batched_impl(t, ok, queries, out, nullptr, nullptr, 1, n_src, n_q, n_tok, d, dtype, eps,
                      (hipStream_t)stream);
}

int sy_fwd_batched_table(const void* const* v_rows, const void* queries, void* out, int64_t n_src,
                         int64_t n_q, int64_t n_tok, int64_t d, int dtype, float eps,
                         void* stream) {
  if (n_tok != 0 && (v_rows == nullptr || queries == nullptr || out == nullptr)) return SY_ERR_NULL;
  int rc = check_sizes(n_src, n_tok, d, dtype, dtype);
  if (rc != SY_OK) return rc;
  if (n_q < 1 || n_q > 0x7fffffff) return SY_ERR_SHAPE;
  RowTable t;
  bool ok = false;
  rc = listed(v_rows, n_src, n_tok, &t, &ok);
  if (rc != SY_OK) return rc;
  return batched_impl(t, ok, queries, out, nullptr, nullptr, 1, n_src, n_q, n_tok, d, dtype, eps,
                      (hipStream_t)stream);
}

int sy_batched_with_stats(const void* v, const void* queries, void* o, float* m, float* l,
                          int64_t n_src, int64_t n_q, int64_t n_tok, int64_t d, int64_t src_stride,
                          int dtype, float eps, void* stream) {
  if (n_tok != 0 && (v == nullptr || queries == nullptr || o == nullptr || m == nullptr ||
                     l == nullptr))
    return SY_ERR_NULL;
  const int rc = check_common(n_src, n_tok, d, src_stride, dtype, dtype);
  if (rc != SY_OK) return rc;
  if (n_q < 1 || n_q > 0x7fffffff) return SY_ERR_SHAPE;
  bool ok = false;
  const RowTable t = stacked(v, n_src, src_stride, dtype, &ok);
  return batched_impl(t, ok, queries, o, m, l, 0, n_src, n_q, n_tok, d, dtype, eps,
                      (hipStream_t)stream);
}

int64_t sy_bwd_batched_workspace_bytes(int64_t n_src, int64_t n_q, int64_t n_tok, int64_t d,
                                       int dtype) {
  int rc = check_sizes(n_src, n_tok, d, dtype, dtype);
  if (rc != SY_OK) return rc;
  if (n_q < 1 || n_q > 0x7fffffff) return SY_ERR_SHAPE;
  if (n_tok == 0) return 0;
  int rows = 0;
  rc = batched_workspace_rows(n_src, n_q, n_tok, d, dtype, &rows);
  if (rc != SY_OK) return rc;
  const int64_t g = rows;
  return g * n_q * d * (int64_t)sizeof(float);
}

int sy_bwd_batched(const void* v, const void* queries, const void* grad_out, void* dv, void* dq,
                   void* workspace, int64_t workspace_bytes, int64_t n_src, int64_t n_q,
                   int64_t n_tok, int64_t d, int64_t src_stride, int dtype, float eps,
                   void* stream) {
  if (dq == nullptr) return SY_ERR_NULL;
  if (n_tok != 0 &&
      (v == nullptr || queries == nullptr || grad_out == nullptr || dv == nullptr))
    return SY_ERR_NULL;
  int rc = check_common(n_src, n_tok, d, src_stride, dtype, dtype);
  if (rc != SY_OK) return rc;
  if (n_q < 1 || n_q > 0x7fffffff || n_q * d > 0x7fffffff / 16) return SY_ERR_SHAPE;
  const hipStream_t s = (hipStream_t)stream;
  bool vok = false, dok = false;
  const RowTable tv = stacked(v, n_src, src_stride, dtype, &vok);
  const RowTable td = stacked(dv, n_src, n_tok * d, dtype, &dok);
  const bool aligned = vec_rows(vok && dok, d, dtype) && al16(queries) && al16(grad_out) &&
                       al16(workspace);
  sy_plan p;
  rc = bwd_batched_plan(n_src, n_q, n_tok, d, dtype, aligned, src_stride * esize(dtype), &p);
  if (rc != SY_OK) return rc;
  int grid = 0;
  if (n_tok != 0) {
    rc = bwd_batched_grid(p, n_src, n_q, n_tok, d, dtype, &grid);
    if (rc != SY_OK) return rc;
    int cap = 0;
    rc = batched_workspace_rows(n_src, n_q, n_tok, d, dtype, &cap);
    if (rc != SY_OK) return rc;
    if (grid > cap) grid = cap;
    if (workspace == nullptr || workspace_bytes < (int64_t)grid * n_q * d * (int64_t)sizeof(float))
      return SY_ERR_WORKSPACE;
    const BwdBatchedArgs a{tv,         queries,    grad_out, td,     (float*)workspace,
                           (int)n_src, (int)n_q,   n_tok,    (int)d, dtype,
                           eps};
    hipError_t e;
    if (p.family == SY_FAMILY_GENERIC) {
      e = launch_bwd_batched_generic(a, grid, s);
    } else if (p.family == SY_FAMILY_MATRIX) {
      e = launch_bwd_batched_matrix(a, grid, s, nullptr);
    } else {
      e = dtype == SY_BF16 ? launch_bwd_batched_vec_bf16(p, a, grid, s)
          : dtype == SY_F16 ? launch_bwd_batched_vec_f16(p, a, grid, s)
                            : launch_bwd_batched_vec_f32(p, a, grid, s);
    }
    if (e != hipSuccess) return (int)e;
  }
  // dq[s][c] = sum over the grid's partial rows, fixed order (zero without tokens).
  return status(launch_dw_reduce((const float*)workspace, grid, (int)(n_q * d), dq, dtype, s));
}

int sy_merge_stats(const void* o1, const float* m1, const float* l1, const void* o2,
                   const float* m2, const float* l2, void* o, float* m, float* l, int64_t n_tok,
                   int64_t d, int dtype, void* stream) {
  if (!valid_dtype(dtype)) return SY_ERR_DTYPE;
  if (n_tok < 0 || n_tok > ((int64_t)1 << 40) || d < 1 || d > 0x7fffffff / 16) return SY_ERR_SHAPE;
  if (n_tok == 0) return SY_OK;
  if (!o1 || !m1 || !l1 || !o2 || !m2 || !l2 || !o || !m || !l) return SY_ERR_NULL;
  const bool vec = al16(o1) && al16(o2) && al16(o) && (d * esize(dtype)) % 16 == 0;
  const MergeArgs a{o1, m1, l1, o2, m2, l2, o, m, l, n_tok, (int)d};
  return status(launch_merge(a, dtype, vec, (hipStream_t)stream));
}

int sy_merge_stats_bwd(const void* o1, const float* m1, const float* l1, const void* o2,
                       const float* m2, const float* l2, const void* grad_o, const float* grad_m,
                       const float* grad_l, void* do1, float* dm1, float* dl1, void* do2,
                       float* dm2, float* dl2, int64_t n_tok, int64_t d, int dtype,
                       void* stream) {
  if (!valid_dtype(dtype)) return SY_ERR_DTYPE;
  if (n_tok < 0 || n_tok > ((int64_t)1 << 40) || d < 1 || d > 0x7fffffff / 16) return SY_ERR_SHAPE;
  if (n_tok == 0) return SY_OK;
  if (!o1 || !m1 || !l1 || !o2 || !m2 || !l2 || !grad_o || !grad_m || !grad_l || !do1 || !dm1 ||
      !dl1 || !do2 || !dm2 || !dl2)
    return SY_ERR_NULL;
  const bool vec = al16(o1) && al16(o2) && al16(grad_o) && al16(do1) && al16(do2) &&
                   (d * esize(dtype)) % 16 == 0;
  const MergeBwdArgs a{o1,  m1,  l1,  o2,  m2,  l2,  grad_o, grad_m,  grad_l,
                       do1, dm1, dl1, do2, dm2, dl2, n_tok,  (int)d};
  return status(launch_merge_bwd(a, dtype, vec, (hipStream_t)stream));
}

int64_t sy_probe_grid(int64_t bytes) {
  // 256 threads x 4 chunks in flight per workgroup; up to 32768 workgroups
  // (the grid that reached the highest read bandwidth on MI355X).
  if (bytes <= 0) return 1;
  const int64_t g = (bytes / 16 + 1023) / 1024;
  return g < 1 ? 1 : (g > 32768 ? 32768 : g);
}

int sy_bw_probe(int kind, const void* src, void* dst, int64_t bytes, void* stream) {
  if (kind < 0 || kind > 3) return SY_ERR_OP;
  if (bytes <= 0 || bytes % 16 != 0 || (kind == 3 && bytes % 144 != 0)) return SY_ERR_SHAPE;
  if ((kind != 1 && src == nullptr) || dst == nullptr) return SY_ERR_NULL;
  if ((kind != 1 && !al16(src)) || (kind != 0 && !al16(dst))) return SY_ERR_SHAPE;
  const int64_t grid = kind == 3 ? sy_probe_grid(bytes / 9 * 4) : sy_probe_grid(bytes);
  return status(launch_probe(kind, src, dst, bytes, (int)grid, (hipStream_t)stream));
}

int sy_tuning_set(const sy_tuning* t) {
  if (t != nullptr) {
    for (const int32_t* f : {t->fwd_tile, t->bwd_tile, t->batched_tile, t->sol_tile})
      for (int k = 0; k < 3; ++k)
        if (f[k] < 0 || f[k] > 64) return SY_ERR_SHAPE;
    if (t->bwd_blocks_per_cu < 0 || t->bwd_blocks_per_cu > 64) return SY_ERR_SHAPE;
    if (t->mx_slots < 0 || t->mx_slots > 2) return SY_ERR_SHAPE;
    if (t->bmx_waves != 0 && t->bmx_waves != 4) return SY_ERR_SHAPE;
  }
  std::lock_guard<std::mutex> lk(g_tuning_mu);
  if (t == nullptr) {
    g_tuning = sy_tuning{};
    g_tuning_on.store(false, std::memory_order_release);
  } else {
    g_tuning = *t;
    g_tuning_on.store(true, std::memory_order_release);
  }
  return SY_OK;
}

int sy_tuning_get(sy_tuning* out) {
  if (out == nullptr) return SY_ERR_NULL;
  if (!tuning_snapshot(out)) *out = sy_tuning{};
  return SY_OK;
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
