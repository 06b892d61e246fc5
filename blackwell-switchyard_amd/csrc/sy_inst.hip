// Instantiates the register-tiled kernels for one dtype and maps a plan onto
// them. Built three times: -DSY_TAG=BF16 -DSY_NAME=bf16, F16/f16, F32/f32.
#include "sy_kernels.hpp"
#include "sy_launch.hpp"

#if !defined(SY_TAG) || !defined(SY_NAME)
#error "build with -DSY_TAG=<BF16|F16|F32> -DSY_NAME=<bf16|f16|f32>"
#endif

#define SY_CAT2(a, b) a##b
#define SY_CAT(a, b) SY_CAT2(a, b)
#define SY_FN(base) SY_CAT(base, SY_NAME)

namespace sy {

namespace {
using T = SY_TAG;
using St = T::storage;

bool tile_is(const sy_plan& p, int w, int vpl, int nr) {
  return p.waves_per_token == w && p.chunks_per_lane == vpl && p.rows_per_tile == nr;
}

int64_t blocks_for(const sy_plan& p, int64_t n_tok) {
  return (n_tok + p.tokens_per_block - 1) / p.tokens_per_block;
}
}  // namespace

hipError_t SY_FN(launch_fwd_vec_)(const sy_plan& p, const FwdArgs& a, hipStream_t s) {
  const float inv_d = 1.0f / (float)a.d;
  const dim3 grid((unsigned)blocks_for(p, a.n_tok));
#define X(W_, V_, N_)                                                                      \
  if (tile_is(p, W_, V_, N_)) {                                                            \
    hipLaunchKernelGGL((k_fwd<T, W_, V_, N_>), grid, dim3(FwdGeom<W_>::kBlock), 0, s,      \
                       (const St*)a.v, (const St*)a.w, (St*)a.out, a.stats, a.n_src, a.n_tok, \
                       a.d, a.src_stride, a.eps, inv_d);                                   \
    return hipGetLastError();                                                              \
  }
  SY_TILES(X)
#undef X
  return hipErrorInvalidConfiguration;
}

hipError_t SY_FN(launch_sol_vec_)(const sy_plan& p, const FwdArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)blocks_for(p, a.n_tok));
#define X(W_, V_, N_)                                                                       \
  if (tile_is(p, W_, V_, N_)) {                                                             \
    hipLaunchKernelGGL((k_sol<T, W_, V_, N_>), grid, dim3(FwdGeom<W_>::kBlock), 0, s,       \
                       (const St*)a.v, (St*)a.out, a.n_src, a.n_tok, a.d, a.src_stride);     \
    return hipGetLastError();                                                               \
  }
  SY_TILES(X)
#undef X
  return hipErrorInvalidConfiguration;
}

hipError_t SY_FN(launch_batched_vec_)(const sy_plan& p, const BatchedArgs& a, hipStream_t s) {
  const float inv_d = 1.0f / (float)a.d;
  const dim3 grid((unsigned)blocks_for(p, a.n_tok));
#define X(W_, V_, N_)                                                                          \
  if (tile_is(p, W_, V_, N_)) {                                                                \
    hipLaunchKernelGGL((k_batched<T, W_, V_, N_>), grid, dim3(FwdGeom<W_>::kBlock), 0, s,      \
                       (const St*)a.v, (const St*)a.q, (St*)a.out, a.n_src, a.n_q, a.n_tok, a.d, \
                       a.src_stride, a.eps, inv_d);                                            \
    return hipGetLastError();                                                                  \
  }
  SY_TILES(X)
#undef X
  return hipErrorInvalidConfiguration;
}

hipError_t SY_FN(launch_bwd_vec_)(const sy_plan& p, const BwdArgs& a, int grid, hipStream_t s) {
  const float inv_d = 1.0f / (float)a.d;
  const int64_t slots = (int64_t)grid * p.tokens_per_block;
  const int n_iter = (int)((a.n_tok + slots - 1) / slots);
#define X(W_, V_, N_)                                                                         \
  if (tile_is(p, W_, V_, N_)) {                                                               \
    hipLaunchKernelGGL((k_bwd<T, W_, V_, N_>), dim3(grid), dim3(BwdGeom<W_>::kBlock), 0, s,   \
                       (const St*)a.v, (const St*)a.w, (const St*)a.g, a.stats, (St*)a.dv,     \
                       a.partial, a.n_src, a.n_tok, a.d, a.src_stride, a.eps, inv_d, n_iter);  \
    return hipGetLastError();                                                                 \
  }
  SY_TILES(X)
#undef X
  return hipErrorInvalidConfiguration;
}

hipError_t SY_FN(bwd_vec_blocks_per_cu_)(const sy_plan& p, int* out) {
#define X(W_, V_, N_)                                                                          \
  if (tile_is(p, W_, V_, N_))                                                                  \
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(out, k_bwd<T, W_, V_, N_>,              \
                                                        BwdGeom<W_>::kBlock, 0);
  SY_TILES(X)
#undef X
  return hipErrorInvalidConfiguration;
}

}  // namespace sy
