// Instantiates the register-tiled kernels for one dtype and maps a plan onto
// them. Built three times: -DSY_TAG=BF16 -DSY_NAME=bf16, F16/f16, F32/f32.
#include <algorithm>

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

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Persistent grid = CUs x the workgroups one CU holds at this kernel's
// register and LDS footprint (unified 512-entry VGPR file per SIMD lane, at
// most 8 waves per SIMD, 160 KiB LDS per CU), capped by the token slots.
int launch_grid(const KernelRes& res, int64_t n_tok, int tpb) {
  int cus = 0;
  if (cu_count(&cus) != hipSuccess || cus < 1) cus = 1;
  const int64_t g = std::min<int64_t>((int64_t)cus * res.blocks_per_cu, cdiv(n_tok, tpb));
  return (int)std::max<int64_t>(1, g);
}

template <class K>
KernelRes resources_of(K* kernel, int block_threads) {
  KernelRes r{0, 0, 1, 0};
  hipFuncAttributes a;
  if (hipFuncGetAttributes(&a, reinterpret_cast<const void*>(kernel)) != hipSuccess) return r;
  r.vgprs = a.numRegs;
  r.lds = (int)a.sharedSizeBytes;
  const int alloc = std::max(8, ((a.numRegs + 7) / 8) * 8);
  const int waves_simd = std::min(8, 512 / alloc);
  const int by_waves = waves_simd * 4 / (block_threads / 64);
  const int by_lds = r.lds > 0 ? (160 * 1024) / r.lds : 64;
  r.blocks_per_cu = std::max(1, std::min(by_waves, by_lds));
  return r;
}
}  // namespace

hipError_t SY_FN(launch_fwd_vec_)(const sy_plan& p, const FwdArgs& a, hipStream_t s,
                                 KernelRes* info) {
  const float inv_d = 1.0f / (float)a.d;
  const bool res = p.family == SY_FAMILY_RESIDENT;
#define X(W_, V_, N_)                                                                        \
  if (tile_is(p, W_, V_, N_)) {                                                              \
    constexpr int kB = FwdGeom<W_>::kBlock, kT = FwdGeom<W_>::kTpb;                          \
    if (res) {                                                                               \
      static const KernelRes kr = resources_of(k_fwd_res<T, W_, V_, N_>, kB);                \
      const int grid = launch_grid(kr, a.n_tok, kT);                                         \
      if (info) {                                                                            \
        *info = kr;                                                                          \
        info->grid = grid;                                                                   \
        return hipSuccess;                                                                   \
      }                                                                                      \
      const int n_iter = (int)cdiv(a.n_tok, (int64_t)grid * kT);                             \
      if (a.prior_m != nullptr) {                                                            \
        if (a.n_src + 1 > N_) return hipErrorInvalidConfiguration;                           \
        if constexpr (W_ == 1) {                                                             \
          static const KernelRes km = resources_of(k_fwd_res<T, W_, V_, N_, true, true>, kB); \
          if (n_iter <= 2 && km.blocks_per_cu >= kr.blocks_per_cu) {                         \
            hipLaunchKernelGGL((k_fwd_res<T, W_, V_, N_, true, true>), dim3(grid), dim3(kB), \
                               0, s, a.v, (const St*)a.w, (St*)a.out, a.stats, a.m_out,      \
                               a.l_out, a.normalize, a.n_src, a.n_tok, a.d, a.eps, inv_d,    \
                               n_iter, a.prior_m, a.prior_l);                                \
            return hipGetLastError();                                                        \
          }                                                                                  \
        }                                                                                    \
        hipLaunchKernelGGL((k_fwd_res<T, W_, V_, N_, true>), dim3(grid), dim3(kB), 0, s, a.v, \
                           (const St*)a.w, (St*)a.out, a.stats, a.m_out, a.l_out,            \
                           a.normalize, a.n_src, a.n_tok, a.d, a.eps, inv_d, n_iter,         \
                           a.prior_m, a.prior_l);                                            \
        return hipGetLastError();                                                            \
      }                                                                                      \
      if constexpr (W_ == 1) {                                                               \
        /* at most two tokens a wave: the final token in one pass (k_fwd_res, FIN) */        \
        static const KernelRes kf = resources_of(k_fwd_res<T, W_, V_, N_, false, true>, kB); \
        if (n_iter <= 2 && kf.blocks_per_cu >= kr.blocks_per_cu) {                           \
          hipLaunchKernelGGL((k_fwd_res<T, W_, V_, N_, false, true>), dim3(grid), dim3(kB), 0, \
                             s, a.v, (const St*)a.w, (St*)a.out, a.stats, a.m_out, a.l_out,  \
                             a.normalize, a.n_src, a.n_tok, a.d, a.eps, inv_d, n_iter,       \
                             nullptr, nullptr);                                              \
          return hipGetLastError();                                                          \
        }                                                                                    \
      }                                                                                      \
      hipLaunchKernelGGL((k_fwd_res<T, W_, V_, N_>), dim3(grid), dim3(kB), 0, s, a.v,        \
                         (const St*)a.w, (St*)a.out, a.stats, a.m_out, a.l_out, a.normalize, \
                         a.n_src, a.n_tok, a.d, a.eps, inv_d, n_iter, nullptr, nullptr);     \
    } else {                                                                                 \
      if (a.prior_m != nullptr) return hipErrorInvalidConfiguration;                         \
      const int64_t grid = cdiv(a.n_tok, kT);                                                \
      if (info) {                                                                            \
        *info = resources_of(k_fwd<T, W_, V_, N_>, kB);                                      \
        info->grid = (int)grid;                                                              \
        return hipSuccess;                                                                   \
      }                                                                                      \
      hipLaunchKernelGGL((k_fwd<T, W_, V_, N_>), dim3((unsigned)grid), dim3(kB), 0, s, a.v,  \
                         (const St*)a.w, (St*)a.out, a.stats, a.m_out, a.l_out, a.normalize, \
                         a.n_src, a.n_tok, a.d, a.eps, inv_d);                               \
    }                                                                                        \
    return hipGetLastError();                                                                \
  }
  SY_TILES(X)
#undef X
  return hipErrorInvalidConfiguration;
}

hipError_t SY_FN(launch_sol_vec_)(const sy_plan& p, const FwdArgs& a, hipStream_t s) {
  const bool res = p.family == SY_FAMILY_RESIDENT;
#define X(W_, V_, N_)                                                                          \
  if (tile_is(p, W_, V_, N_)) {                                                                \
    constexpr int kB = FwdGeom<W_>::kBlock, kT = FwdGeom<W_>::kTpb;                            \
    if (res) {                                                                                 \
      static const KernelRes kr = resources_of(k_sol_res<T, W_, V_, N_>, kB);                  \
      hipLaunchKernelGGL((k_sol_res<T, W_, V_, N_>), dim3(launch_grid(kr, a.n_tok, kT)),       \
                         dim3(kB), 0, s, a.v, (St*)a.out, a.n_src, a.n_tok, a.d);              \
    } else {                                                                                   \
      hipLaunchKernelGGL((k_sol<T, W_, V_, N_>), dim3((unsigned)cdiv(a.n_tok, kT)), dim3(kB), 0, \
                         s, a.v, (St*)a.out, a.n_src, a.n_tok, a.d);                           \
    }                                                                                          \
    return hipGetLastError();                                                                  \
  }
  SY_TILES(X)
#undef X
  return hipErrorInvalidConfiguration;
}

hipError_t SY_FN(launch_batched_vec_)(const sy_plan& p, const BatchedArgs& a, hipStream_t s) {
  const float inv_d = 1.0f / (float)a.d;
#define X(W_, V_, N_)                                                                            \
  if (tile_is(p, W_, V_, N_)) {                                                                  \
    constexpr int kB = FwdGeom<W_>::kBlock, kT = FwdGeom<W_>::kTpb;                              \
    hipLaunchKernelGGL((k_batched<T, W_, V_, N_>), dim3((unsigned)cdiv(a.n_tok, kT)), dim3(kB), 0, \
                       s, a.v, (const St*)a.q, (St*)a.out, a.m_out, a.l_out, a.normalize,        \
                       a.n_src, a.n_q, a.n_tok, a.d, a.eps, inv_d);                              \
    return hipGetLastError();                                                                    \
  }
  SY_TILES(X)
#undef X
  return hipErrorInvalidConfiguration;
}

// The backward's grid must be known before launch (it sizes the workspace),
// so it is computed here from the instantiation's resources.
// variant: a BwdVariant (kBwdStacked, kBwdListed, kBwdStatsGrad).
hipError_t SY_FN(bwd_vec_resources_)(const sy_plan& p, bool stats, int variant, KernelRes* out) {
  if (variant < 0 || variant > 2) return hipErrorInvalidValue;
  // 32- and 64-row tiles exist for the stacked operator gradient with stats only.
#define X(W_, V_, N_)                                                                        \
  if (tile_is(p, W_, V_, N_)) {                                                              \
    if (!stats || variant != kBwdStacked) return hipErrorInvalidConfiguration;              \
    static const KernelRes r =                                                               \
        resources_of(k_bwd_tall<T, W_, V_, N_>, TallGeom<W_, V_, N_>::kBlock);               \
    *out = r;                                                                                \
    return hipSuccess;                                                                       \
  }
  SY_BWD_TALL_TILES(X)
#undef X
#define X(W_, V_, N_)                                                                        \
  if (tile_is(p, W_, V_, N_)) {                                                              \
    constexpr int kB = BwdGeom<W_, V_>::kBlock;                                              \
    static const KernelRes r[2][3] = {                                                       \
        {resources_of(k_bwd<T, W_, V_, N_, false, kBwdStacked>, kB),                         \
         resources_of(k_bwd<T, W_, V_, N_, false, kBwdListed>, kB),                          \
         resources_of(k_bwd<T, W_, V_, N_, false, kBwdStatsGrad>, kB)},                      \
        {resources_of(k_bwd<T, W_, V_, N_, true, kBwdStacked>, kB),                          \
         resources_of(k_bwd<T, W_, V_, N_, true, kBwdListed>, kB),                           \
         resources_of(k_bwd<T, W_, V_, N_, true, kBwdStatsGrad>, kB)}};                      \
    *out = r[stats ? 1 : 0][variant];                                                        \
    return hipSuccess;                                                                       \
  }
  SY_TILES(X)
  SY_BWD_WIDE_TILES(X)
#undef X
  return hipErrorInvalidConfiguration;
}

hipError_t SY_FN(launch_bwd_vec_)(const sy_plan& p, const BwdArgs& a, int grid, hipStream_t s) {
  const float inv_d = 1.0f / (float)a.d;
  const int64_t slots = (int64_t)grid * p.tokens_per_block;
  const int n_iter = (int)cdiv(a.n_tok, slots);
#define X(W_, V_, N_)                                                                        \
  if (tile_is(p, W_, V_, N_)) {                                                              \
    if (a.stats == nullptr || a.listed || a.gm != nullptr) return hipErrorInvalidConfiguration; \
    hipLaunchKernelGGL((k_bwd_tall<T, W_, V_, N_>), dim3(grid), dim3(TallGeom<W_, V_, N_>::kBlock), 0, \
                       s, a.v, (const St*)a.w, (const St*)a.g, a.stats, a.dv, a.partial,       \
                       a.n_src, a.n_tok, a.d, inv_d, n_iter);                                 \
    return hipGetLastError();                                                                 \
  }
  SY_BWD_TALL_TILES(X)
#undef X
#define SY_BWD_LAUNCH(W_, V_, N_, ST_, LI_)                                                  \
  hipLaunchKernelGGL((k_bwd<T, W_, V_, N_, ST_, LI_>), dim3(grid), dim3(BwdGeom<W_, V_>::kBlock), 0, \
                     s, a.v, (const St*)a.w, (const St*)a.g, a.stats, a.gm, a.gl, a.dv, a.partial, \
                     a.n_src, a.n_tok, a.d, a.eps, inv_d, n_iter)
#define X(W_, V_, N_)                                                                        \
  if (tile_is(p, W_, V_, N_)) {                                                              \
    const int var = a.listed ? kBwdListed : (a.gm != nullptr ? kBwdStatsGrad : kBwdStacked);  \
    if (a.stats != nullptr) {                                                                \
      if (var == kBwdListed) SY_BWD_LAUNCH(W_, V_, N_, true, kBwdListed);                    \
      else if (var == kBwdStatsGrad) SY_BWD_LAUNCH(W_, V_, N_, true, kBwdStatsGrad);         \
      else SY_BWD_LAUNCH(W_, V_, N_, true, kBwdStacked);                                     \
    } else {                                                                                 \
      if (var == kBwdListed) SY_BWD_LAUNCH(W_, V_, N_, false, kBwdListed);                   \
      else if (var == kBwdStatsGrad) SY_BWD_LAUNCH(W_, V_, N_, false, kBwdStatsGrad);        \
      else SY_BWD_LAUNCH(W_, V_, N_, false, kBwdStacked);                                    \
    }                                                                                        \
    return hipGetLastError();                                                                \
  }
  SY_TILES(X)
  SY_BWD_WIDE_TILES(X)
#undef X
#undef SY_BWD_LAUNCH
  return hipErrorInvalidConfiguration;
}

// Batched backward tiles: one chunk per lane, W waves per token, NR rows,
// up to kBwdBatchedMaxQ queries.
#define SY_BB_TILES(X) X(1, 4) X(1, 9) X(2, 4) X(2, 9) X(4, 4) X(4, 9) X(8, 4) X(8, 9)

hipError_t SY_FN(bwd_batched_vec_resources_)(const sy_plan& p, KernelRes* out) {
  // Sized by the variant with a runtime row count (the larger footprint).
#define X(W_, N_)                                                                             \
  if (tile_is(p, W_, 1, N_)) {                                                                \
    static const KernelRes kr = resources_of(                                                 \
        k_bwd_batched<T, W_, N_, (int)kBwdBatchedMaxQ, false>, FwdGeom<W_>::kBlock);            \
    *out = kr;                                                                                \
    return hipSuccess;                                                                        \
  }
  SY_BB_TILES(X)
#undef X
  return hipErrorInvalidConfiguration;
}

hipError_t SY_FN(launch_bwd_batched_vec_)(const sy_plan& p, const BwdBatchedArgs& a, int grid,
                                         hipStream_t s) {
  const float inv_d = 1.0f / (float)a.d;
  const int n_iter = (int)cdiv(a.n_tok, (int64_t)grid * p.tokens_per_block);
#define SY_BB_LAUNCH(W_, N_, EX_)                                                             \
  hipLaunchKernelGGL((k_bwd_batched<T, W_, N_, (int)kBwdBatchedMaxQ, EX_>), dim3(grid),       \
                     dim3(FwdGeom<W_>::kBlock), 0, s, a.v, (const St*)a.q, (const St*)a.g,    \
                     a.dv, a.partial, a.n_src, a.n_q, a.n_tok, a.d, a.eps, inv_d, n_iter)
#define X(W_, N_)                                                                             \
  if (tile_is(p, W_, 1, N_)) {                                                                \
    if (a.n_src == N_) SY_BB_LAUNCH(W_, N_, true);                                            \
    else SY_BB_LAUNCH(W_, N_, false);                                                         \
    return hipGetLastError();                                                                 \
  }
  SY_BB_TILES(X)
#undef X
#undef SY_BB_LAUNCH
  return hipErrorInvalidConfiguration;
}

}  // namespace sy
