// Merging two partial attention results (o, m, l) over disjoint source groups,
// and its gradient. Reference: src/switchyard/reference.py:218-233
// (merge_online_softmax, Algorithm 1 line 12 of the paper):
//     m = max(m1, m2), s_i = exp(m_i - m), o = s_1 o_1 + s_2 o_2, l = s_1 l_1 + s_2 l_2.
// Gradient (k = the group holding the max, group 1 on a tie, j the other):
//     do_i = s_i g_o,  dl_i = s_i g_l,  ds_i = <g_o, o_i> + g_l l_i,
//     dm_j = s_j ds_j, dm_k = g_m - s_j ds_j.
// One wavefront per token; lanes stride over the row in 16-byte chunks when
// every row start is 16-byte aligned, element by element otherwise. HBM-bound
// element-wise work: 2 row reads + 1 row write forward, 3 reads + 2 writes back.
// Loads are streamed (non-temporal); stores take the default write-back
// policy, unlike the operator's kernels: on MI355X at 4096 x 2048 bf16 the
// gradient runs in 15.6-15.8 us against 17.1-17.4 us with streamed stores
// (forward 10.5 against 10.6-11.0 us). Each pass issues four chunks' loads a
// lane (a whole 4 KiB row) before its arithmetic: forward 9.8 against 10.9 us
// one chunk at a time, gradient 15.5 against 15.7 us.
#include <algorithm>

#include "sy_device.hpp"
#include "sy_launch.hpp"

namespace sy {

namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;
constexpr int kU = 4;  // 16-byte chunks a lane loads per pass (a 4 KiB row at once)

template <class T, bool VEC>
__global__ void __launch_bounds__(kBlock)
k_merge(const void* __restrict__ o1, const float* __restrict__ m1, const float* __restrict__ l1,
        const void* __restrict__ o2, const float* __restrict__ m2, const float* __restrict__ l2,
        void* __restrict__ o, float* __restrict__ m, float* __restrict__ l, int64_t n_tok, int d,
        int normalize) {
  using S = typename T::storage;
  constexpr int CE = T::ce;
  const int lane = threadIdx.x & 63;
  const int64_t stride = (int64_t)gridDim.x * kWaves;
  for (int64_t tok = (int64_t)blockIdx.x * kWaves + wave_id(); tok < n_tok; tok += stride) {
    const float a = m1[tok], b = m2[tok];
    const float mm = fmaxf(a, b);
    const float e1 = expf(a - mm), e2 = expf(b - mm);
    const float ll = fmaf(e1, l1[tok], e2 * l2[tok]);
    // normalize: the row weights carry 1 / l, so o / l costs no extra pass.
    const float inv = normalize ? 1.0f / ll : 1.0f;
    const float s1 = e1 * inv, s2 = e2 * inv;
    if constexpr (VEC) {
      const uint32_t row_bytes = (uint32_t)d * sizeof(S);
      const auto r1 = make_rsrc(static_cast<const S*>(o1) + tok * d, row_bytes);
      const auto r2 = make_rsrc(static_cast<const S*>(o2) + tok * d, row_bytes);
      const auto ro = make_rsrc(static_cast<S*>(o) + tok * d, row_bytes);
      // kU chunks a lane per pass, all loads issued before the arithmetic
      // (chunks past the row read 0 and their stores are dropped by the
      // resource's range check).
      for (uint32_t off0 = lane * 16u; off0 < row_bytes; off0 += kU * 64u * 16u) {
        i32x4_t x[kU], y[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          x[u] = ld16_stream(r1, off0 + u * 1024u);
          y[u] = ld16_stream(r2, off0 + u * 1024u);
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          float f[CE];
#pragma unroll
          for (int e = 0; e < CE; ++e) f[e] = fmaf(s1, elem<T>(x[u], e), s2 * elem<T>(y[u], e));
          st16(ro, off0 + u * 1024u, pack<T>(f));
        }
      }
    } else {
      for (int k = lane; k < d; k += 64) {
        const int64_t i = tok * d + k;
        store_elem(o, i, fmaf(s1, load_elem(o1, i, T::code), s2 * load_elem(o2, i, T::code)),
                   T::code);
      }
    }
    if (lane == 0) {
      m[tok] = mm;
      l[tok] = ll;
    }
  }
}

template <class T, bool VEC>
__global__ void __launch_bounds__(kBlock)
k_merge_bwd(const void* __restrict__ o1, const float* __restrict__ m1, const float* __restrict__ l1,
            const void* __restrict__ o2, const float* __restrict__ m2, const float* __restrict__ l2,
            const void* __restrict__ go, const float* __restrict__ gm, const float* __restrict__ gl,
            void* __restrict__ do1, float* __restrict__ dm1, float* __restrict__ dl1,
            void* __restrict__ do2, float* __restrict__ dm2, float* __restrict__ dl2, int64_t n_tok,
            int d) {
  using S = typename T::storage;
  constexpr int CE = T::ce;
  const int lane = threadIdx.x & 63;
  const int64_t stride = (int64_t)gridDim.x * kWaves;
  for (int64_t tok = (int64_t)blockIdx.x * kWaves + wave_id(); tok < n_tok; tok += stride) {
    const float a = m1[tok], b = m2[tok];
    const float mm = fmaxf(a, b);
    const float s1 = expf(a - mm), s2 = expf(b - mm);
    float dot1 = 0.0f, dot2 = 0.0f;
    if constexpr (VEC) {
      const uint32_t row_bytes = (uint32_t)d * sizeof(S);
      const int64_t base = tok * d;
      const auto r1 = make_rsrc(static_cast<const S*>(o1) + base, row_bytes);
      const auto r2 = make_rsrc(static_cast<const S*>(o2) + base, row_bytes);
      const auto rg = make_rsrc(static_cast<const S*>(go) + base, row_bytes);
      const auto w1 = make_rsrc(static_cast<S*>(do1) + base, row_bytes);
      const auto w2 = make_rsrc(static_cast<S*>(do2) + base, row_bytes);
      for (uint32_t off0 = lane * 16u; off0 < row_bytes; off0 += kU * 64u * 16u) {
        i32x4_t x[kU], y[kU], g[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          x[u] = ld16_stream(r1, off0 + u * 1024u);
          y[u] = ld16_stream(r2, off0 + u * 1024u);
          g[u] = ld16_stream(rg, off0 + u * 1024u);
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          float f1[CE], f2[CE];
#pragma unroll
          for (int e = 0; e < CE; ++e) {
            const float ge = elem<T>(g[u], e);
            dot1 = fmaf(ge, elem<T>(x[u], e), dot1);
            dot2 = fmaf(ge, elem<T>(y[u], e), dot2);
            f1[e] = s1 * ge;
            f2[e] = s2 * ge;
          }
          st16(w1, off0 + u * 1024u, pack<T>(f1));
          st16(w2, off0 + u * 1024u, pack<T>(f2));
        }
      }
    } else {
      for (int k = lane; k < d; k += 64) {
        const int64_t i = tok * d + k;
        const float ge = load_elem(go, i, T::code);
        dot1 = fmaf(ge, load_elem(o1, i, T::code), dot1);
        dot2 = fmaf(ge, load_elem(o2, i, T::code), dot2);
        store_elem(do1, i, s1 * ge, T::code);
        store_elem(do2, i, s2 * ge, T::code);
      }
    }
    dot1 = wave_sum(dot1);
    dot2 = wave_sum(dot2);
    if (lane == 0) {
      const float glv = gl[tok], gmv = gm[tok];
      const float ds1 = fmaf(glv, l1[tok], dot1), ds2 = fmaf(glv, l2[tok], dot2);
      dl1[tok] = s1 * glv;
      dl2[tok] = s2 * glv;
      if (a >= b) {  // group 1 holds the max (m = m1, s1 = 1)
        dm2[tok] = s2 * ds2;
        dm1[tok] = gmv - s2 * ds2;
      } else {
        dm1[tok] = s1 * ds1;
        dm2[tok] = gmv - s1 * ds1;
      }
    }
  }
}

unsigned merge_grid(int64_t n_tok) {
  int cus = 0;
  if (cu_count(&cus) != hipSuccess || cus < 1) cus = 1;
  const int64_t want = (n_tok + kWaves - 1) / kWaves;
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(want, (int64_t)cus * 8));
}

template <class T>
hipError_t merge_t(const MergeArgs& a, bool vec, hipStream_t s) {
  const unsigned grid = merge_grid(a.n_tok);
  if (vec) {
    hipLaunchKernelGGL((k_merge<T, true>), dim3(grid), dim3(kBlock), 0, s, a.o1, a.m1, a.l1, a.o2,
                       a.m2, a.l2, a.o, a.m, a.l, a.n_tok, a.d, a.normalize);
  } else {
    hipLaunchKernelGGL((k_merge<T, false>), dim3(grid), dim3(kBlock), 0, s, a.o1, a.m1, a.l1, a.o2,
                       a.m2, a.l2, a.o, a.m, a.l, a.n_tok, a.d, a.normalize);
  }
  return hipGetLastError();
}

template <class T>
hipError_t merge_bwd_t(const MergeBwdArgs& a, bool vec, hipStream_t s) {
  const unsigned grid = merge_grid(a.n_tok);
  if (vec) {
    hipLaunchKernelGGL((k_merge_bwd<T, true>), dim3(grid), dim3(kBlock), 0, s, a.o1, a.m1, a.l1,
                       a.o2, a.m2, a.l2, a.go, a.gm, a.gl, a.do1, a.dm1, a.dl1, a.do2, a.dm2,
                       a.dl2, a.n_tok, a.d);
  } else {
    hipLaunchKernelGGL((k_merge_bwd<T, false>), dim3(grid), dim3(kBlock), 0, s, a.o1, a.m1, a.l1,
                       a.o2, a.m2, a.l2, a.go, a.gm, a.gl, a.do1, a.dm1, a.dl1, a.do2, a.dm2,
                       a.dl2, a.n_tok, a.d);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_merge(const MergeArgs& a, int dtype, bool vec, hipStream_t s) {
  if (dtype == SY_BF16) return merge_t<BF16>(a, vec, s);
  if (dtype == SY_F16) return merge_t<F16>(a, vec, s);
  return merge_t<F32>(a, vec, s);
}

hipError_t launch_merge_bwd(const MergeBwdArgs& a, int dtype, bool vec, hipStream_t s) {
  if (dtype == SY_BF16) return merge_bwd_t<BF16>(a, vec, s);
  if (dtype == SY_F16) return merge_bwd_t<F16>(a, vec, s);
  return merge_bwd_t<F32>(a, vec, s);
}

}  // namespace sy
