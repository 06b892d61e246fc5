// Host-side plumbing between the C ABI (sy_capi.cpp) and the kernel
// translation units. No torch types, no allocation.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/switchyard.h"
#include "sy_device.hpp"

namespace sy {

// Compile-time register tiles that exist for the vector (16-byte) kernels:
// X(waves_per_token, chunks_per_lane, rows_per_tile). rows_per_tile 16 is
// only built with <= 2 chunks per lane (64 chunks = 256 VGPRs would spill).
#define SY_TILES(X)                                                                     \
  X(1, 1, 4) X(1, 1, 9) X(1, 1, 16) X(1, 2, 4) X(1, 2, 9) X(1, 2, 16) X(1, 4, 4) X(1, 4, 9) \
  X(2, 1, 4) X(2, 1, 9) X(2, 1, 16) X(2, 2, 4) X(2, 2, 9) X(2, 2, 16) X(2, 4, 4) X(2, 4, 9) \
  X(4, 1, 4) X(4, 1, 9) X(4, 1, 16) X(4, 2, 4) X(4, 2, 9) X(4, 2, 16) X(4, 4, 4) X(4, 4, 9) \
  X(8, 1, 4) X(8, 1, 9) X(8, 1, 16) X(8, 2, 4) X(8, 2, 9) X(8, 2, 16) X(8, 4, 4) X(8, 4, 9)

// Backward-only tiles with four chunks per lane and 16 rows: 256 tile VGPRs,
// which fit only at one wave per SIMD (512 registers, 256-thread workgroups).
#define SY_BWD_WIDE_TILES(X) X(1, 4, 16) X(2, 4, 16)
// Backward-only tiles of 32 rows, one or two chunks per lane (128 or 256 tile
// VGPRs; two waves per SIMD, or one), for 16 < N <= 32 with the forward's stats on stacked rows: the
// operator's gradient as the autograd op calls it; and of 64 rows, one chunk
// per lane (256 tile VGPRs, one wave per SIMD), for 32 < N <= 64. Other
// callers at that N (no stats, per-row pointers, the (o, m, l) gradient) run
// the generic kernel.
#define SY_BWD_TALL_TILES(X) \
  X(2, 1, 32) X(4, 1, 32) X(2, 2, 32) X(4, 2, 32) X(2, 1, 64) X(4, 1, 64)
constexpr int kTallRows = 32;
constexpr int kTallerRows = 64;

// Largest N the generic kernels accept (their per-token scalars live in LDS).
constexpr int64_t kGenericMaxN = 4096;
// Largest query count of the resident batched kernel.
constexpr int64_t kBatchedMaxQ = 16;
// Register-resident batched backward: at most this many sources and queries.
constexpr int64_t kBwdBatchedMaxN = 9;
constexpr int64_t kBwdBatchedMaxQ = 8;
// Batched forward on the matrix cores (sy_matrix.hip): 16-bit inputs, at most
// 16 sources and 16 queries (one MFMA tile each way), D in {512, 1024, 1536,
// 2048} (four waves x 32-column MFMA steps; a wave keeps its query slice in
// registers) and D = 4096 with N <= 9 (eight waves of 512 columns; the LDS
// holds ten 8 KiB rows). Its stores address four query rows from one buffer resource, so
// 4 * n_tok * D * 2 bytes must stay below 2^31 (else the per-query path runs).
// Below kMatrixMinQ queries the register-tiled kernel is faster (config 3
// shape, MI355X, register tile vs matrix cores: 2 queries 38.4 vs 50.0 us, 3:
// 46.4 vs 50.8, 4: 53.5 vs 52.4, 5: 60.4 vs 53.8).
constexpr int64_t kMatrixMaxRows = 16;
constexpr int64_t kMatrixMaxQ = 16;
constexpr int64_t kMatrixMinQ = 4;
inline bool matrix_batched_fits(int64_t n_src, int64_t n_q, int64_t d, int dtype) {
  return (dtype == SY_BF16 || dtype == SY_F16) && n_src >= 1 && n_src <= kMatrixMaxRows &&
         n_q >= kMatrixMinQ && n_q <= kMatrixMaxQ &&
         (d == 512 || d == 1024 || d == 1536 || d == 2048 || (d == 4096 && n_src <= 9));
}
inline bool matrix_batched_offsets_fit(int64_t n_q, int64_t n_tok, int64_t d) {
  return 4 * n_tok * d * 2 < ((int64_t)1 << 31) && n_q * n_tok * 4 < ((int64_t)1 << 31);
}
// Batched backward on the matrix cores (sy_matrix.hip): 16-bit inputs, at most
// 8 queries (g and the queries share the 16 columns of one MFMA tile), D in
// {512, 1024, 1536, 2048}, and the workgroup's LDS within 160 KiB: 16 rows of
// g and queries, the source rows and a zero row (dynamic), plus the logit
// exchange, the coefficient tables and the dv staging (static, the kernel's
// own arithmetic: 9 or 16 staged rows, SC-column store rounds). Eight waves
// per workgroup (two per SIMD) at D = 1024 and 2048 (config 3 on MI355X:
// 103.6 vs 105.9 us with four; D = 1024: 66.6 vs 67.8 us), four at D = 512
// (N=4 S=8: 41.5 vs 48.6 us) and 1536. The 16-row tile at D = 2048 would
// spill registers: there N <= 9. Buffer offsets stay below 2^31: the dv rows
// of a token (n_src - 1 strides) and the rows one staging load covers.
constexpr int64_t kBwdMatrixMaxQ = 8;
constexpr int bwd_matrix_waves(int64_t d) { return d == 1024 || d == 2048 ? 8 : 4; }
// dv store round width (columns) of the (rows, 32-column steps, waves) tile.
constexpr int bwd_matrix_store_cols(int nr, int ks, int w) {
  return w == 8 ? (ks >= 8 ? 64 : (32 * ks < 128 ? 32 * ks : 128))
                : (nr <= 9 && ks % 8 == 0 ? 256 : 128);
}
inline int64_t bwd_matrix_dynamic_lds(int64_t n_src, int64_t d) {
  return (16 + n_src + 1) * (d * 2 + 16);
}
inline int64_t bwd_matrix_lds(int64_t n_src, int64_t d) {
  const int w = bwd_matrix_waves(d);
  const int ks = (int)(d / (32 * w));
  const int64_t nr = n_src <= 9 ? 9 : 16;
  const int64_t sc = bwd_matrix_store_cols((int)nr, ks, w);
  const int64_t rows_per_store = 64 / (sc / 8);
  const int64_t rounds = (nr + rows_per_store - 1) / rows_per_store * rows_per_store;
  const int64_t staged = rounds > nr ? rounds : nr + 1;
  const int64_t fixed = w * (2 * 64 * 16 + 2 * 16 * 4 + 24 * 20 * 4 + staged * (sc * 2 + 16));
  return fixed + bwd_matrix_dynamic_lds(n_src, d);
}
inline bool bwd_matrix_fits(int64_t n_src, int64_t n_q, int64_t d, int dtype) {
  return (dtype == SY_BF16 || dtype == SY_F16) && n_src >= 1 && n_src <= kMatrixMaxRows &&
         n_q >= 1 && n_q <= kBwdMatrixMaxQ && (d == 512 || d == 1024 || d == 1536 || d == 2048) &&
         (n_src <= 9 || d < 2048) && bwd_matrix_lds(n_src, d) <= 160 * 1024;
}
inline bool bwd_matrix_offsets_fit(int64_t n_src, int64_t n_tok, int64_t d, int64_t v_stride_bytes) {
  const int64_t cpr = d / (8 * bwd_matrix_waves(d));  // 16-byte chunks of a wave's slice
  const int64_t rpl = cpr <= 32 && 64 % cpr == 0 ? 64 / cpr : 1;  // rows per staging load
  const int64_t g_stride = n_tok * d * 2;  // g and dv rows
  const int64_t limit = ((int64_t)1 << 31) - d * 2;
  return (n_src - 1) * g_stride < limit && (rpl - 1) * g_stride < limit &&
         (rpl - 1) * v_stride_bytes < limit;
}
// Dynamic LDS the generic kernels may request (bytes).
constexpr int64_t kGenericMaxLds = 64 * 1024;
// LDS of the generic batched backward: per-(query, row) alpha and da, per-row
// c and r, the row-scalar scratch and the block-reduction scratch.
inline int64_t bwd_batched_generic_lds(int64_t n_src, int64_t n_q) {
  return (2 * n_q * n_src + 5 * n_src + 257) * (int64_t)sizeof(float);
}

// Source rows are addressed through a RowTable (sy_device.hpp) in every
// launch: the stacked layout and a per-source pointer list look the same to
// the kernels.
struct FwdArgs {
  RowTable v;
  const void* w;
  void* out;
  float* stats;   // [2][N][n_tok] logits and r, or nullptr
  float* m_out;   // [n_tok] max logit, or nullptr (then l_out is nullptr too)
  float* l_out;   // [n_tok] sum of exp(logit - m)
  int normalize;  // 1: out = o / l (the operator); 0: out = o (attn_with_stats)
  int n_src;
  int64_t n_tok;
  int d;
  int v_dtype;
  int w_dtype;
  float eps;
  // Phase 2 of the two-phase schedule (resident tiles only): row n_src of v
  // is a prior group's o1, these its m1 and l1 [n_tok]; nullptr otherwise.
  const float* prior_m = nullptr;
  const float* prior_l = nullptr;
};

struct BwdArgs {
  RowTable v;
  const void* w;
  const void* g;
  const float* stats;
  const float* gm;  // dL/dm [n_tok] for the (o, m, l) gradient, or nullptr
  const float* gl;  // dL/dl [n_tok]
  RowTable dv;
  float* partial;   // [grid][d] fp32
  bool listed;      // v and dv rows from per-row pointers (else stacked; gm must be null)
  int n_src;
  int64_t n_tok;
  int d;
  int v_dtype;
  int w_dtype;
  float eps;
};

struct BatchedArgs {
  RowTable v;
  const void* q;
  void* out;
  float* m_out;  // [S][n_tok] or nullptr
  float* l_out;  // [S][n_tok]
  int normalize;
  int n_src;
  int n_q;
  int64_t n_tok;
  int d;
  int dtype;
  float eps;
};

struct BwdBatchedArgs {
  RowTable v;
  const void* q;     // [S][d]
  const void* g;     // [S][n_tok][d]
  RowTable dv;
  float* partial;    // [grid][S][d] fp32
  int n_src;
  int n_q;
  int64_t n_tok;
  int d;
  int dtype;
  float eps;
};

// Pure shape arithmetic (sy_plan.cpp). `has_stats` matters to SY_OP_BWD only:
// whether the forward's logits and r are passed (the operator's path, and what
// sy_plan_for reports) or recomputed. `matrix_ok` = 0 leaves the matrix-core
// batched backward out (its dv offsets do not fit the token count).
int make_plan(int op, int64_t n_src, int64_t n_q, int64_t d, int v_dtype, int w_dtype, int aligned,
              sy_plan* out, int has_stats = 1, int matrix_ok = 1);

// Measurement overrides installed with sy_tuning_set (sy_capi.cpp). Returns
// false (and leaves *out untouched) when none are installed, which is the
// default: then no launch depends on anything but shape, dtype, alignment
// and device.
bool tuning_snapshot(sy_tuning* out);

// Launch-time tile override from sy_tuning_set (sy_plan.cpp); sy_plan_for
// never applies it.
void apply_tile_override(int op, int64_t n_src, int64_t d, sy_plan* p);
// The plan's tile for n_tok tokens: the token-count rule (wider tiles when
// there are few tokens per CU, forward and backward), then any sy_tuning_set
// tile override. Every launch and size query of the forward and backward
// applies it, so grids and workspaces agree. `chunked_ok` false keeps the
// forward over 10-16 rows resident (callers that need a resident tile).
void apply_tile_rules(int op, int64_t n_src, int64_t n_tok, int64_t d, sy_plan* p,
                      bool chunked_ok = true);

// Launches the matrix-core batched forward (a.n_src etc. must pass
// matrix_batched_fits). With `info` != nullptr fills it and launches nothing.
struct KernelRes;
hipError_t launch_batched_matrix(const BatchedArgs& a, hipStream_t s, KernelRes* info);
// Launches the matrix-core batched backward on `grid` workgroups (a must pass
// bwd_matrix_fits and bwd_matrix_offsets_fit; 1 <= grid <= n_tok). With
// `info` != nullptr fills it (resources and the grid it would choose) and
// launches nothing.
hipError_t launch_bwd_batched_matrix(const BwdBatchedArgs& a, int grid, hipStream_t s,
                                     KernelRes* info);

// Device queries, cached per device (sy_capi.cpp).
hipError_t cu_count(int* out);
// Device address of sy_bwd_static's workspace on the current device.
int scratch_address(void** out);

// Register/LDS footprint of one kernel instantiation, the workgroups per CU
// that footprint allows, and (when filled by a launcher) the launch grid.
struct KernelRes {
  int vgprs;
  int lds;
  int blocks_per_cu;
  int grid;
};

// Per-dtype vector-kernel launchers (sy_inst.hip built once per dtype).
// launch_fwd_vec_* with `info` != nullptr fills it and launches nothing.
// `grid` for the backward is the persistent workgroup count.
#define SY_DECLARE_VEC(NAME)                                                                   \
  hipError_t launch_fwd_vec_##NAME(const sy_plan& p, const FwdArgs& a, hipStream_t s,          \
                                   KernelRes* info);                                           \
  hipError_t launch_sol_vec_##NAME(const sy_plan& p, const FwdArgs& a, hipStream_t s);         \
  hipError_t launch_batched_vec_##NAME(const sy_plan& p, const BatchedArgs& a, hipStream_t s); \
  hipError_t launch_bwd_vec_##NAME(const sy_plan& p, const BwdArgs& a, int grid, hipStream_t s); \
  hipError_t bwd_vec_resources_##NAME(const sy_plan& p, bool stats, int variant, KernelRes* out); \
  hipError_t launch_bwd_batched_vec_##NAME(const sy_plan& p, const BwdBatchedArgs& a, int grid, \
                                           hipStream_t s);                                    \
  hipError_t bwd_batched_vec_resources_##NAME(const sy_plan& p, KernelRes* out);
SY_DECLARE_VEC(bf16)
SY_DECLARE_VEC(f16)
SY_DECLARE_VEC(f32)
#undef SY_DECLARE_VEC

// Merge of two (o, m, l) partial results and its gradient (sy_merge.hip).
// `vec` selects the 16-byte path (every row start 16-byte aligned).
struct MergeArgs {
  const void* o1;
  const float* m1;
  const float* l1;
  const void* o2;
  const float* m2;
  const float* l2;
  void* o;
  float* m;
  float* l;
  int64_t n_tok;
  int d;
  int normalize = 0;  // 1: o = merged o / merged l (the operator's output)
};
struct MergeBwdArgs {
  const void* o1;
  const float* m1;
  const float* l1;
  const void* o2;
  const float* m2;
  const float* l2;
  const void* go;
  const float* gm;
  const float* gl;
  void* do1;
  float* dm1;
  float* dl1;
  void* do2;
  float* dm2;
  float* dl2;
  int64_t n_tok;
  int d;
};
hipError_t launch_merge(const MergeArgs& a, int dtype, bool vec, hipStream_t s);
hipError_t launch_merge_bwd(const MergeBwdArgs& a, int dtype, bool vec, hipStream_t s);

// Generic kernels, the dw reduction and the probes (sy_generic.hip).
hipError_t launch_fwd_generic(const FwdArgs& a, hipStream_t s);
hipError_t launch_sol_generic(const FwdArgs& a, hipStream_t s);
hipError_t launch_bwd_generic(const BwdArgs& a, int grid, hipStream_t s);
hipError_t launch_bwd_batched_generic(const BwdBatchedArgs& a, int grid, hipStream_t s);
hipError_t launch_dw_reduce(const float* partial, int rows, int d, void* dw, int w_dtype,
                            hipStream_t s);
hipError_t launch_probe(int kind, const void* src, void* dst, int64_t bytes, int grid,
                        hipStream_t s);

}  // namespace sy
