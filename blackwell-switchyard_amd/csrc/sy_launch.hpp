// Host-side plumbing between the C ABI (sy_capi.cpp) and the kernel
// translation units. No torch types, no allocation.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/switchyard.h"

namespace sy {

// Compile-time register tiles that exist for the vector (16-byte) kernels:
// X(waves_per_token, chunks_per_lane, rows_per_tile). rows_per_tile 16 is
// only built with <= 2 chunks per lane (64 chunks = 256 VGPRs would spill).
#define SY_TILES(X)                                                                     \
  X(1, 1, 4) X(1, 1, 9) X(1, 1, 16) X(1, 2, 4) X(1, 2, 9) X(1, 2, 16) X(1, 4, 4) X(1, 4, 9) \
  X(2, 1, 4) X(2, 1, 9) X(2, 1, 16) X(2, 2, 4) X(2, 2, 9) X(2, 2, 16) X(2, 4, 4) X(2, 4, 9) \
  X(4, 1, 4) X(4, 1, 9) X(4, 1, 16) X(4, 2, 4) X(4, 2, 9) X(4, 2, 16) X(4, 4, 4) X(4, 4, 9) \
  X(8, 1, 4) X(8, 1, 9) X(8, 1, 16) X(8, 2, 4) X(8, 2, 9) X(8, 2, 16) X(8, 4, 4) X(8, 4, 9)

// Largest N the generic kernels accept (their per-token scalars live in LDS).
constexpr int64_t kGenericMaxN = 4096;
// Largest query count of the resident batched kernel.
constexpr int64_t kBatchedMaxQ = 16;

struct FwdArgs {
  const void* v;
  const void* w;
  void* out;
  float* stats;
  int n_src;
  int64_t n_tok;
  int d;
  int64_t src_stride;
  int v_dtype;
  int w_dtype;
  float eps;
};

struct BwdArgs {
  const void* v;
  const void* w;
  const void* g;
  const float* stats;
  void* dv;
  void* dw;
  float* partial;  // [grid][d] fp32
  int n_src;
  int64_t n_tok;
  int d;
  int64_t src_stride;
  int v_dtype;
  int w_dtype;
  float eps;
};

struct BatchedArgs {
  const void* v;
  const void* q;
  void* out;
  int n_src;
  int n_q;
  int64_t n_tok;
  int d;
  int64_t src_stride;
  int dtype;
  float eps;
};

// Pure shape arithmetic (sy_plan.cpp).
int make_plan(int op, int64_t n_src, int64_t n_q, int64_t d, int v_dtype, int w_dtype, int aligned,
              sy_plan* out);

// Launch-time tile override from the SY_TILE_* environment variables
// (sy_plan.cpp); sy_plan_for never applies it.
void apply_tile_override(int op, int64_t n_src, int64_t d, sy_plan* p);

// Device queries, cached per device (sy_capi.cpp).
hipError_t cu_count(int* out);

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
  hipError_t bwd_vec_resources_##NAME(const sy_plan& p, bool stats, KernelRes* out);
SY_DECLARE_VEC(bf16)
SY_DECLARE_VEC(f16)
SY_DECLARE_VEC(f32)
#undef SY_DECLARE_VEC

// Generic kernels, the dw reduction and the probes (sy_generic.hip).
hipError_t launch_fwd_generic(const FwdArgs& a, hipStream_t s);
hipError_t launch_sol_generic(const FwdArgs& a, hipStream_t s);
hipError_t launch_bwd_generic(const BwdArgs& a, int grid, hipStream_t s);
hipError_t launch_dw_reduce(const float* partial, int rows, int d, void* dw, int w_dtype,
                            hipStream_t s);
hipError_t launch_probe(int kind, const void* src, void* dst, int64_t bytes, int grid,
                        hipStream_t s);

}  // namespace sy
