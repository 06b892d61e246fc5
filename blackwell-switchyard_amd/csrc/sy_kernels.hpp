// Register-tiled Block AttnRes kernels for gfx950.
//
// Geometry. A token's [N, D] tile is spread over W wavefronts: lane l of wave
// `seg` owns the 16-byte chunks c = (seg*64 + l) + j*64*W, j < VPL, of every
// source row, so each buffer_load_dwordx4 of a wave reads 1 KiB of contiguous
// row memory. Rows past N are never loaded; chunks past the row end read as 0
// through the buffer descriptor's range check and are never stored.
//
// Per token the kernels need only 2-3 wave-uniform scalars per source row
// (sum of squares, query dot, grad dot). Tiles of up to 9 rows sum them all
// at once with one transposed cross-lane sum (tsum), larger tiles one DPP
// reduction per scalar; when W > 1 the W partial sums meet in LDS and are added
// in segment order, so every wave of the token computes bit-identical softmax
// weights.
//
// Reference: src/switchyard/triton_op.py:50-78 (_fwd_resident),
// :81-117 (_fwd_tiled), :153-191 (_speed_of_light), :194-264 (_bwd_resident),
// :378-414 (_fwd_batched_resident). The tiling, the online merge across row
// chunks and the deterministic dw reduction are this build's own design.
#pragma once

#include "sy_device.hpp"

namespace sy {

// x, hidden from the optimiser: a comparison against it cannot be hoisted and
// kept live. The row guards `n < rows` of the resident kernels otherwise
// become 64-bit predicates held for the whole kernel and spilled into VGPR
// lanes (the 32-row backward: ~140 SGPR spills; the forward: 46 -> 16 and
// 30.2 -> 29.8 us at config 2; k_bwd up to 9 rows: 55.9 -> 55.6 us).
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+s"(x));
  return x;
}


// Forward-shaped kernels: 256-thread workgroups (or one token per workgroup
// when a token needs more than four waves).
template <int W>
struct FwdGeom {
  static constexpr int kBlock = (64 * W > 256) ? 64 * W : 256;
  static constexpr int kTpb = kBlock / (64 * W);
};

// Backward: persistent workgroups of bwd_block(W, VPL, NR) threads; kTpb
// token slots run side by side.
template <int W, int VPL, int NR = 0>
struct BwdGeom {
  static constexpr int kBlock = bwd_block(W, VPL, NR);
  static constexpr int kTpb = kBlock / (64 * W);
};

// Sum wave-uniform per-row values across the W waves of each token slot.
// vals is G groups of NR rows (vals[grp*NR + n]); entries with grp < groups and
// n < rows take part. Lane 0 of every wave publishes; after one barrier each
// wave adds the W contributions in segment order. `buf` must not be rewritten
// until every wave has passed the next barrier, which callers ensure by
// alternating two buffers. All register indices are compile-time constants.
template <int W, int G, int NR, int TPB>
__device__ __forceinline__ void cross_wave_sum(float (&vals)[G * NR], int groups, int rows,
                                               float (&buf)[TPB][W][G * NR], int slot, int seg,
                                               int lane) {
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < G * NR; ++i)
      if (i / NR < groups && i % NR < rows) buf[slot][seg][i] = vals[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < G * NR; ++i) {
    if (i / NR < groups && i % NR < rows) {
      float s = buf[slot][0][i];
#pragma unroll
      for (int k = 1; k < W; ++k) s += buf[slot][k][i];
      vals[i] = s;
    }
  }
}

// The same totals from per-lane partials tv[i] (i < G*NR, zero past the live
// rows) by one transposed sum (tsum): with W == 1 each total is read from the
// lane that holds it; with W > 1 those lanes publish the wave's partials with
// one LDS store and, after one barrier, every wave adds the W partials in
// segment order as cross_wave_sum does. Used for tiles of at most 9 rows: at
// 16 rows the 16 live partials cost the backward tile registers (N=16, D=2048:
// backward 97.9 vs 97.0 us), while at 9 rows one tsum replaces 9-18 wave_sums
// (config 2: backward 56.1 vs 57.2 us, forward 29.3 vs 29.6).
template <int W, int G, int NR, int TPB, int P>
__device__ __forceinline__ void row_sums_transposed(const float (&tv)[P], float (&part)[G * NR],
                                                    int groups, int rows,
                                                    float (&buf)[TPB][W][G * NR], int slot,
                                                    int seg, int lane) {
  static_assert(P >= G * NR, "one value per lane slot");
  const float s = tsum<P>(tv, lane);
  if constexpr (W == 1) {
#pragma unroll
    for (int i = 0; i < G * NR; ++i)
      part[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), tsum_lane<P>(i)));
  } else {
    const int i = tsum_row<P>(lane);
    if (lane == tsum_lane<P>(i) && i < G * NR) buf[slot][seg][i] = s;
    __syncthreads();
#pragma unroll
    for (int q = 0; q < G * NR; ++q) {
      if (q / NR < groups && q % NR < rows) {
        float t = buf[slot][0][q];
#pragma unroll
        for (int k = 1; k < W; ++k) t += buf[slot][k][q];
        part[q] = t;
      }
    }
  }
}

// ------------------------------------------------------------------ forward
//
// One token per W waves. Rows are processed in chunks of NR; when N <= NR
// there is one chunk and v is read exactly once with no rescaling. Larger N
// merges chunks with the online-softmax update (running max m, running sum l,
// accumulator rescaled by exp(m_old - m_new)), which still reads v once.
//
// Optional outputs: stats[n*n_tok + t] = logit, stats[(N+n)*n_tok + t] = r_n;
// m_out[t] = max logit and l_out[t] = sum_n exp(logit_n - m) (both or neither).
// normalize = 0 stores the unnormalised o = sum_n exp(logit_n - m) v_n instead
// of o / l (reference src/switchyard/reference.py:194-215, attn_with_stats).
template <class T, int W, int VPL, int NR>
__global__ void __launch_bounds__(FwdGeom<W>::kBlock)
k_fwd(const RowTable v, const typename T::storage* __restrict__ w,
      typename T::storage* __restrict__ out, float* __restrict__ stats, float* __restrict__ m_out,
      float* __restrict__ l_out, int normalize, int n_src, int64_t n_tok, int d, float eps,
      float inv_d) {
  using S = typename T::storage;
  constexpr int CE = T::ce;
  constexpr int TPB = FwdGeom<W>::kTpb;
  constexpr uint32_t kStep = 64u * W * 16u;
  __shared__ float red[2][TPB][W][2 * NR];

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int slot = wave / W;
  const int seg = wave % W;
  int64_t tok = (int64_t)blockIdx.x * TPB + slot;
  const bool live = tok < n_tok;
  if constexpr (W == 1 || TPB == 1) {
    if (!live) return;  // no barrier is shared with another token slot
  }
  if (!live) tok = n_tok - 1;  // keep the slot's waves in step for the barriers

  const uint32_t row_bytes = (uint32_t)d * sizeof(S);
  const uint32_t lane_off = (uint32_t)(seg * 64 + lane) * 16u;

  i32x4_t wq[VPL];
  {
    const auto wr = make_rsrc(w, row_bytes);
#pragma unroll
    for (int j = 0; j < VPL; ++j) wq[j] = ld16(wr, lane_off + j * kStep);
  }

  float m_run = -INFINITY, l_run = 0.0f;
  float acc[VPL][CE];
#pragma unroll
  for (int j = 0; j < VPL; ++j)
#pragma unroll
    for (int e = 0; e < CE; ++e) acc[j][e] = 0.0f;

  int it = 0;
  for (int c0 = 0; c0 < n_src; c0 += NR, ++it) {
    const int rows = min(NR, n_src - c0);
    i32x4_t x[NR][VPL];
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      if (n < rows) {
        const auto r = make_rsrc(row_of<const S>(v, c0 + n) + tok * d, row_bytes);
#pragma unroll
        for (int j = 0; j < VPL; ++j) x[n][j] = ld16_stream(r, lane_off + j * kStep);
      }
    }

    // part[n] = sum of squares, part[NR + n] = query dot of row c0 + n.
    float part[2 * NR];
    if constexpr (NR <= 9) {
      constexpr int P = pow2_at_least(2 * NR);
      float tv[P];
#pragma unroll
      for (int i = 0; i < P; ++i) tv[i] = 0.0f;
#pragma unroll
      for (int n = 0; n < NR; ++n) {
        if (n < rows) {
          float ss = 0.0f, dt = 0.0f;
#pragma unroll
          for (int j = 0; j < VPL; ++j) {
            ss = dot<T>(x[n][j], x[n][j], ss);
            dt = dot<T>(x[n][j], wq[j], dt);
          }
          tv[n] = ss;
          tv[NR + n] = dt;
        }
      }
      row_sums_transposed<W, 2, NR, TPB, P>(tv, part, 2, rows, red[it & 1], slot, seg, lane);
    } else {
#pragma unroll
      for (int n = 0; n < NR; ++n) {
        if (n < rows) {
          float ss = 0.0f, dt = 0.0f;
#pragma unroll
          for (int j = 0; j < VPL; ++j) {
            ss = dot<T>(x[n][j], x[n][j], ss);
            dt = dot<T>(x[n][j], wq[j], dt);
          }
          part[n] = wave_sum(ss);
          part[NR + n] = wave_sum(dt);
        }
      }
      if constexpr (W > 1) cross_wave_sum<W, 2, NR, TPB>(part, 2, rows, red[it & 1], slot, seg, lane);
    }

    float lg[NR];
    float cm = m_run;
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      if (n < rows) {
        const float r = rsqrtf(fmaf(part[n], inv_d, eps));
        lg[n] = part[NR + n] * r;
        cm = fmaxf(cm, lg[n]);
        if (stats != nullptr && seg == 0 && lane == 0 && live) {
          stats[(int64_t)(c0 + n) * n_tok + tok] = lg[n];
          stats[(int64_t)(n_src + c0 + n) * n_tok + tok] = r;
        }
      }
    }
    if (it > 0) {
      const float sc = expf(m_run - cm);
      l_run *= sc;
#pragma unroll
      for (int j = 0; j < VPL; ++j)
#pragma unroll
        for (int e = 0; e < CE; ++e) acc[j][e] *= sc;
    }
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      if (n < rows) {
        const float p = expf(lg[n] - cm);
        l_run += p;
#pragma unroll
        for (int j = 0; j < VPL; ++j)
#pragma unroll
          for (int e = 0; e < CE; ++e) acc[j][e] = fmaf(p, elem<T>(x[n][j], e), acc[j][e]);
      }
    }
    m_run = cm;
  }

  if (!live) return;
  if (m_out != nullptr && seg == 0 && lane == 0) {
    m_out[tok] = m_run;
    l_out[tok] = l_run;
  }
  const float inv_l = normalize ? 1.0f / l_run : 1.0f;
  const auto orr = make_rsrc(out + tok * d, row_bytes);
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    float f[CE];
#pragma unroll
    for (int e = 0; e < CE; ++e) f[e] = acc[j][e] * inv_l;
    st16_stream(orr, lane_off + j * kStep, pack<T>(f));
  }
}

// ------------------------------------------------------------ speed of light
//
// Same bytes, geometry and launch shape as k_fwd, no softmax: out = sum_n v_n.
template <class T, int W, int VPL, int NR>
__global__ void __launch_bounds__(FwdGeom<W>::kBlock)
k_sol(const RowTable v, typename T::storage* __restrict__ out, int n_src, int64_t n_tok, int d) {
  using S = typename T::storage;
  constexpr int CE = T::ce;
  constexpr int TPB = FwdGeom<W>::kTpb;
  constexpr uint32_t kStep = 64u * W * 16u;
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int64_t tok = (int64_t)blockIdx.x * TPB + wave / W;
  if (tok >= n_tok) return;
  const uint32_t row_bytes = (uint32_t)d * sizeof(S);
  const uint32_t lane_off = (uint32_t)((wave % W) * 64 + lane) * 16u;

  float acc[VPL][CE];
#pragma unroll
  for (int j = 0; j < VPL; ++j)
#pragma unroll
    for (int e = 0; e < CE; ++e) acc[j][e] = 0.0f;
  for (int c0 = 0; c0 < n_src; c0 += NR) {
    const int rows = min(NR, n_src - c0);
    i32x4_t x[NR][VPL];
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      if (n < rows) {
        const auto r = make_rsrc(row_of<const S>(v, c0 + n) + tok * d, row_bytes);
#pragma unroll
        for (int j = 0; j < VPL; ++j) x[n][j] = ld16_stream(r, lane_off + j * kStep);
      }
    }
#pragma unroll
    for (int n = 0; n < NR; ++n)
      if (n < rows)
#pragma unroll
        for (int j = 0; j < VPL; ++j)
#pragma unroll
          for (int e = 0; e < CE; ++e) acc[j][e] += elem<T>(x[n][j], e);
  }
  const auto orr = make_rsrc(out + tok * d, row_bytes);
#pragma unroll
  for (int j = 0; j < VPL; ++j) st16_stream(orr, lane_off + j * kStep, pack<T>(acc[j]));
}

// ----------------------------------------------------------------- batched
//
// S queries against one register-resident tile (N <= NR): the inverse RMS of
// each row is computed once, then each query costs one dot reduction per row,
// a softmax and a weighted sum. v is read once for all S outputs.
template <class T, int W, int VPL, int NR>
__global__ void __launch_bounds__(FwdGeom<W>::kBlock)
k_batched(const RowTable v, const typename T::storage* __restrict__ q,
          typename T::storage* __restrict__ out, float* __restrict__ m_out,
          float* __restrict__ l_out, int normalize, int n_src, int n_q, int64_t n_tok, int d,
          float eps, float inv_d) {
  using S = typename T::storage;
  constexpr int CE = T::ce;
  constexpr int TPB = FwdGeom<W>::kTpb;
  constexpr uint32_t kStep = 64u * W * 16u;
  __shared__ float red[2][TPB][W][NR];

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int slot = wave / W;
  const int seg = wave % W;
  int64_t tok = (int64_t)blockIdx.x * TPB + slot;
  const bool live = tok < n_tok;
  if constexpr (W == 1 || TPB == 1) {
    if (!live) return;
  }
  if (!live) tok = n_tok - 1;
  const uint32_t row_bytes = (uint32_t)d * sizeof(S);
  const uint32_t lane_off = (uint32_t)(seg * 64 + lane) * 16u;
  const int rows = n_src;  // host guarantees n_src <= NR

  i32x4_t x[NR][VPL];
#pragma unroll
  for (int n = 0; n < NR; ++n) {
    if (n < rows) {
      const auto r = make_rsrc(row_of<const S>(v, n) + tok * d, row_bytes);
#pragma unroll
      for (int j = 0; j < VPL; ++j) x[n][j] = ld16_stream(r, lane_off + j * kStep);
    }
  }
  float rinv[NR];
  int it = 0;
  if constexpr (NR <= 9) {
    constexpr int P = pow2_at_least(NR);
    float tv[P];
#pragma unroll
    for (int i = 0; i < P; ++i) tv[i] = 0.0f;
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      if (n < rows) {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < VPL; ++j) ss = dot<T>(x[n][j], x[n][j], ss);
        tv[n] = ss;
      }
    }
    row_sums_transposed<W, 1, NR, TPB, P>(tv, rinv, 1, rows, red[it++ & 1], slot, seg, lane);
  } else {
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      if (n < rows) {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < VPL; ++j) ss = dot<T>(x[n][j], x[n][j], ss);
        rinv[n] = wave_sum(ss);
      }
    }
    if constexpr (W > 1) cross_wave_sum<W, 1, NR, TPB>(rinv, 1, rows, red[it++ & 1], slot, seg, lane);
  }
#pragma unroll
  for (int n = 0; n < NR; ++n)
    if (n < rows) rinv[n] = rsqrtf(fmaf(rinv[n], inv_d, eps));

  for (int s = 0; s < n_q; ++s) {
    i32x4_t qq[VPL];
    const auto qr = make_rsrc(q + (int64_t)s * d, row_bytes);
#pragma unroll
    for (int j = 0; j < VPL; ++j) qq[j] = ld16(qr, lane_off + j * kStep);
    float lg[NR];
    if constexpr (NR <= 9) {
      constexpr int P = pow2_at_least(NR);
      float tv[P];
#pragma unroll
      for (int i = 0; i < P; ++i) tv[i] = 0.0f;
#pragma unroll
      for (int n = 0; n < NR; ++n) {
        if (n < rows) {
          float dt = 0.0f;
#pragma unroll
          for (int j = 0; j < VPL; ++j) dt = dot<T>(x[n][j], qq[j], dt);
          tv[n] = dt;
        }
      }
      row_sums_transposed<W, 1, NR, TPB, P>(tv, lg, 1, rows, red[it++ & 1], slot, seg, lane);
    } else {
#pragma unroll
      for (int n = 0; n < NR; ++n) {
        if (n < rows) {
          float dt = 0.0f;
#pragma unroll
          for (int j = 0; j < VPL; ++j) dt = dot<T>(x[n][j], qq[j], dt);
          lg[n] = wave_sum(dt);
        }
      }
      if constexpr (W > 1) cross_wave_sum<W, 1, NR, TPB>(lg, 1, rows, red[it++ & 1], slot, seg, lane);
    }
    float m = -INFINITY;
#pragma unroll
    for (int n = 0; n < NR; ++n)
      if (n < rows) {
        lg[n] *= rinv[n];
        m = fmaxf(m, lg[n]);
      }
    float l = 0.0f;
    float acc[VPL][CE];
#pragma unroll
    for (int j = 0; j < VPL; ++j)
#pragma unroll
      for (int e = 0; e < CE; ++e) acc[j][e] = 0.0f;
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      if (n < rows) {
        const float p = expf(lg[n] - m);
        l += p;
#pragma unroll
        for (int j = 0; j < VPL; ++j)
#pragma unroll
          for (int e = 0; e < CE; ++e) acc[j][e] = fmaf(p, elem<T>(x[n][j], e), acc[j][e]);
      }
    }
    if (live) {
      if (m_out != nullptr && seg == 0 && lane == 0) {
        m_out[(int64_t)s * n_tok + tok] = m;
        l_out[(int64_t)s * n_tok + tok] = l;
      }
      const float inv_l = normalize ? 1.0f / l : 1.0f;
      const auto orr = make_rsrc(out + ((int64_t)s * n_tok + tok) * d, row_bytes);
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        float f[CE];
#pragma unroll
        for (int e = 0; e < CE; ++e) f[e] = acc[j][e] * inv_l;
        st16_stream(orr, lane_off + j * kStep, pack<T>(f));
      }
    }
  }
}

// ------------------------------------------- resident forward, pipelined
//
// Persistent variant of the forward for N <= NR (one chunk). Token slot s of
// workgroup b handles tokens b*TPB + s + k*gridDim.x*TPB. The tile registers
// are refilled as they are consumed: as soon as row n of the current token has
// been accumulated into the output, row n of the slot's next token is loaded
// into the same registers. The next token's loads are therefore in flight
// during this token's weighted sum, output store and the loop overhead, with no
// extra registers. `n_iter` is the slot trip count of the busiest slot; slots
// with fewer tokens re-read their last token and store nothing, so when W > 1
// every wave of the workgroup meets the same barriers.
//
// MERGE: phase 2 of the two-phase schedule in the same pass (reference
// src/switchyard/reference.py:195-233, attn_with_stats then
// merge_online_softmax). Row n_src of the table is a prior group's
// unnormalised o1 (v's dtype), pm/pl its m1, l1 per token. It rides in the
// tile as one more row, refilled like the sources, and enters the sum with
// weight s1 = exp(m1 - M), M = max(m1, max_n logit_n):
//     o = s1 o1 + sum_n exp(logit_n - M) v_n,   l = s1 l1 + sum_n exp(logit_n - M)
// so the group's own o is never rounded or written (the merge kernel would
// re-read it), and out is o / l (normalize) or o with (M, l).
//
// FIN (one wave per token): a wave's final token, whose rows have
// no later loads to overlap, folds each row in as soon as it lands instead of
// waiting for all rows before the softmax: per-row sums (one two-value
// transposed sum), weights exp(logit_n - logit_0) relative to row 0's logit
// (with MERGE, relative to the prior's m1, the prior entering with weight 1
// and its l1; acc and l rescaled if a later row's logit exceeds the
// reference by 32, so no weight exceeds e^32), and the reference folded out
// at the end (o / l is
// invariant to it; m_out, l_out and an unnormalised o are taken relative to
// the max). Only the last row's work then follows the last load. Launched for
// at most two tokens per wave: config 2's forward 29.5 -> 29.0 us, T = 2048
// 16.7 -> 16.4, T = 1024 11.2 -> 10.9 (MI355X, same kernel otherwise); with
// four or more tokens per wave the variant's loop ran 0.3-0.4 us a token
// slower (T = 8192: 56.1 vs 56.5; T = 16384: 111.9 vs 113.3). A final token's
// weights carry a different rounding than the two-pass form's, so a token's
// bits depend on whether it is its wave's last (both within one rounding).
template <class T, int W, int VPL, int NR, bool MERGE = false, bool FIN = false>
__global__ void __launch_bounds__(FwdGeom<W>::kBlock)
k_fwd_res(const RowTable v, const typename T::storage* __restrict__ w,
          typename T::storage* __restrict__ out, float* __restrict__ stats,
          float* __restrict__ m_out, float* __restrict__ l_out, int normalize, int n_src,
          int64_t n_tok, int d, float eps, float inv_d, int n_iter,
          const float* __restrict__ pm = nullptr, const float* __restrict__ pl = nullptr) {
  using S = typename T::storage;
  constexpr int CE = T::ce;
  constexpr int TPB = FwdGeom<W>::kTpb;
  constexpr uint32_t kStep = 64u * W * 16u;
  __shared__ float red[2][TPB][W][2 * NR];

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int slot = wave / W;
  const int seg = wave % W;
  const int64_t slots = (int64_t)gridDim.x * TPB;
  const int64_t first = (int64_t)blockIdx.x * TPB + slot;
  int iters = n_iter;
  if constexpr (W == 1) {
    // Independent waves: each runs exactly its own tokens.
    if (first >= n_tok) return;
    iters = (int)((n_tok - first + slots - 1) / slots);
  }
  const uint32_t row_bytes = (uint32_t)d * sizeof(S);
  const uint32_t lane_off = (uint32_t)(seg * 64 + lane) * 16u;
  const int rows = n_src;  // host guarantees n_src <= NR (n_src + 1 with MERGE)
  const int tile_rows = MERGE ? n_src + 1 : n_src;
  // MERGE: lane 0 holds the token's m1, lane 1 its l1, fetched one token
  // ahead by one vector load (a per-lane address, so no scalar-cache wait
  // sits at the use).
  const float* pstat_src = (lane & 1) ? pl : pm;

  i32x4_t wq[VPL];
  {
    const auto wr = make_rsrc(w, row_bytes);
#pragma unroll
    for (int j = 0; j < VPL; ++j) wq[j] = ld16(wr, lane_off + j * kStep);
  }
  i32x4_t x[NR][VPL];
  float pstat = 0.0f;
  {
    const int64_t t0 = first < n_tok ? first : n_tok - 1;
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      if (n < opaque(tile_rows)) {
        const auto r = make_rsrc(row_of<const S>(v, n) + t0 * d, row_bytes);
#pragma unroll
        for (int j = 0; j < VPL; ++j) x[n][j] = ld16_stream(r, lane_off + j * kStep);
      }
    }
    if constexpr (MERGE) {
      if (lane < 2) pstat = pstat_src[t0];
    }
  }

  for (int k = 0; k < iters; ++k) {
    const int64_t tok = first + (int64_t)k * slots;
    const bool live = tok < n_tok;
    const bool more = k + 1 < iters;
    const int64_t nxt = tok + slots < n_tok ? tok + slots : n_tok - 1;
    float pm_tok = 0.0f, pl_tok = 0.0f;
    if constexpr (MERGE) {
      pm_tok = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pstat), 0));
      pl_tok = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pstat), 1));
      if (more && lane < 2) pstat = pstat_src[nxt];
    }
    if constexpr (FIN) {
      static_assert(W == 1, "the one-pass final token is for one-wave tokens");
      if (!more) {
        float acc[VPL][CE];
#pragma unroll
        for (int j = 0; j < VPL; ++j)
#pragma unroll
          for (int e = 0; e < CE; ++e) acc[j][e] = 0.0f;
        float lg[NR], rr[NR];
        // Reference logit: row 0's, or with MERGE the prior's m1, which is
        // known before any row lands (the prior then enters with weight 1
        // and its l1).
        float mref = MERGE ? pm_tok : 0.0f, l = 0.0f, m = MERGE ? pm_tok : -INFINITY;
#pragma unroll
        for (int n = 0; n < NR; ++n) {
          if (n < opaque(tile_rows)) {
            const bool prior = MERGE && n == rows;
            float lgn = pm_tok;
            if (!prior) {
              float ss = 0.0f, dt = 0.0f;
#pragma unroll
              for (int j = 0; j < VPL; ++j) {
                ss = dot<T>(x[n][j], x[n][j], ss);
                dt = dot<T>(x[n][j], wq[j], dt);
              }
              const float pv[2] = {ss, dt};
              const float s2 = tsum<2>(pv, lane);  // lanes 0..31: ss, 32..63: dt
              const float ssum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s2), 0));
              const float dsum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s2), 32));
              rr[n] = rsqrtf(fmaf(ssum, inv_d, eps));
              lg[n] = dsum * rr[n];
              lgn = lg[n];
              m = fmaxf(m, lgn);
            }
            if (!MERGE && n == 0) {
              mref = lgn;
            } else if (lgn > mref + 32.0f) {
              const float sc = expf(mref - lgn);
              l *= sc;
#pragma unroll
              for (int j = 0; j < VPL; ++j)
#pragma unroll
                for (int e = 0; e < CE; ++e) acc[j][e] *= sc;
              mref = lgn;
            }
            const float p = expf(lgn - mref);
            l = prior ? fmaf(p, pl_tok, l) : l + p;
#pragma unroll
            for (int j = 0; j < VPL; ++j)
#pragma unroll
              for (int e = 0; e < CE; ++e) acc[j][e] = fmaf(p, elem<T>(x[n][j], e), acc[j][e]);
          }
        }
        const float adj = expf(mref - m);  // from the reference to the max
        if (stats != nullptr) {
          float sv = 0.0f;
#pragma unroll
          for (int n = 0; n < NR; ++n) {
            sv = lane == n ? lg[n] : sv;
            sv = lane == 32 + n ? rr[n] : sv;
          }
          const int i = lane & 31;
          if (i < rows) stats[(int64_t)((lane >> 5) * n_src + i) * n_tok + tok] = sv;
        }
        if (m_out != nullptr && lane == 0) {
          m_out[tok] = m;
          l_out[tok] = l * adj;
        }
        const float inv_l = normalize ? 1.0f / l : adj;
        const auto orr = make_rsrc(out + tok * d, row_bytes);
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
          float f[CE];
#pragma unroll
          for (int e = 0; e < CE; ++e) f[e] = acc[j][e] * inv_l;
          st16_stream(orr, lane_off + j * kStep, pack<T>(f));
        }
        break;
      }
    }

    float part[2 * NR];
    if constexpr (NR <= 9) {
      constexpr int P = pow2_at_least(2 * NR);
      float tv[P];
#pragma unroll
      for (int i = 0; i < P; ++i) tv[i] = 0.0f;
#pragma unroll
      for (int n = 0; n < NR; ++n) {
        if (n < opaque(rows)) {
          float ss = 0.0f, dt = 0.0f;
#pragma unroll
          for (int j = 0; j < VPL; ++j) {
            ss = dot<T>(x[n][j], x[n][j], ss);
            dt = dot<T>(x[n][j], wq[j], dt);
          }
          tv[n] = ss;
          tv[NR + n] = dt;
        }
      }
      row_sums_transposed<W, 2, NR, TPB, P>(tv, part, 2, rows, red[k & 1], slot, seg, lane);
    } else {
#pragma unroll
      for (int n = 0; n < NR; ++n) {
        if (n < opaque(rows)) {
          float ss = 0.0f, dt = 0.0f;
#pragma unroll
          for (int j = 0; j < VPL; ++j) {
            ss = dot<T>(x[n][j], x[n][j], ss);
            dt = dot<T>(x[n][j], wq[j], dt);
          }
          part[n] = wave_sum(ss);
          part[NR + n] = wave_sum(dt);
        }
      }
      if constexpr (W > 1) cross_wave_sum<W, 2, NR, TPB>(part, 2, rows, red[k & 1], slot, seg, lane);
    }

    float lg[NR];
    float m = -INFINITY;
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      if constexpr (MERGE) lg[n] = -INFINITY;  // the prior row's slot: weight s1
      if (n < opaque(rows)) {
        const float r = rsqrtf(fmaf(part[n], inv_d, eps));
        lg[n] = part[NR + n] * r;
        part[n] = r;
        m = fmaxf(m, lg[n]);
      }
    }
    float acc[VPL][CE];
#pragma unroll
    for (int j = 0; j < VPL; ++j)
#pragma unroll
      for (int e = 0; e < CE; ++e) acc[j][e] = 0.0f;
    float l = 0.0f;
    float s1 = 0.0f;
    if constexpr (MERGE) {
      m = fmaxf(m, pm_tok);
      s1 = expf(pm_tok - m);
    }
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      if (n < opaque(tile_rows)) {
        const bool prior = MERGE && n == rows;
        const float p = prior ? s1 : expf(lg[n] - m);
        if (!prior) l += p;
#pragma unroll
        for (int j = 0; j < VPL; ++j)
#pragma unroll
          for (int e = 0; e < CE; ++e) acc[j][e] = fmaf(p, elem<T>(x[n][j], e), acc[j][e]);
        if (more) {
          const auto r = make_rsrc(row_of<const S>(v, n) + nxt * d, row_bytes);
#pragma unroll
          for (int j = 0; j < VPL; ++j) x[n][j] = ld16_stream(r, lane_off + j * kStep);
        }
      }
    }
    if constexpr (MERGE) l = fmaf(s1, pl_tok, l);
    if (live) {
      if (stats != nullptr && seg == 0) {
        // One store instruction for the token's 2N statistics (lane i < N the
        // logit of row i, lane 32 + i its r) instead of 2N single-lane ones.
        float sv = 0.0f;
#pragma unroll
        for (int n = 0; n < NR; ++n) {
          sv = lane == n ? lg[n] : sv;
          sv = lane == 32 + n ? part[n] : sv;
        }
        const int i = lane & 31;
        if (i < rows) stats[(int64_t)((lane >> 5) * n_src + i) * n_tok + tok] = sv;
      }
      if (m_out != nullptr && seg == 0 && lane == 0) {
        m_out[tok] = m;
        l_out[tok] = l;
      }
      const float inv_l = normalize ? 1.0f / l : 1.0f;
      const auto orr = make_rsrc(out + tok * d, row_bytes);
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        float f[CE];
#pragma unroll
        for (int e = 0; e < CE; ++e) f[e] = acc[j][e] * inv_l;
        st16_stream(orr, lane_off + j * kStep, pack<T>(f));
      }
    }
  }
}

// ------------------------------------------ resident speed of light, pipelined
//
// The ceiling for k_fwd_res: same bytes, grid, slot loop and prefetch, no
// softmax (out = sum_n v_n).
template <class T, int W, int VPL, int NR>
__global__ void __launch_bounds__(FwdGeom<W>::kBlock)
k_sol_res(const RowTable v, typename T::storage* __restrict__ out, int n_src, int64_t n_tok,
          int d) {
  using S = typename T::storage;
  constexpr int CE = T::ce;
  constexpr int TPB = FwdGeom<W>::kTpb;
  constexpr uint32_t kStep = 64u * W * 16u;
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int64_t slots = (int64_t)gridDim.x * TPB;
  const int64_t first = (int64_t)blockIdx.x * TPB + wave / W;
  if (first >= n_tok) return;  // no barriers in this kernel
  const int iters = (int)((n_tok - first + slots - 1) / slots);
  const uint32_t row_bytes = (uint32_t)d * sizeof(S);
  const uint32_t lane_off = (uint32_t)((wave % W) * 64 + lane) * 16u;
  const int rows = n_src;

  i32x4_t x[NR][VPL];
#pragma unroll
  for (int n = 0; n < NR; ++n) {
    if (n < opaque(rows)) {
      const auto r = make_rsrc(row_of<const S>(v, n) + first * d, row_bytes);
#pragma unroll
      for (int j = 0; j < VPL; ++j) x[n][j] = ld16_stream(r, lane_off + j * kStep);
    }
  }
  for (int k = 0; k < iters; ++k) {
    const int64_t tok = first + (int64_t)k * slots;
    const bool more = k + 1 < iters;
    float acc[VPL][CE];
#pragma unroll
    for (int j = 0; j < VPL; ++j)
#pragma unroll
      for (int e = 0; e < CE; ++e) acc[j][e] = 0.0f;
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      if (n < opaque(rows)) {
#pragma unroll
        for (int j = 0; j < VPL; ++j)
#pragma unroll
          for (int e = 0; e < CE; ++e) acc[j][e] += elem<T>(x[n][j], e);
        if (more) {
          const auto r = make_rsrc(row_of<const S>(v, n) + (tok + slots) * d, row_bytes);
#pragma unroll
          for (int j = 0; j < VPL; ++j) x[n][j] = ld16_stream(r, lane_off + j * kStep);
        }
      }
    }
    const auto orr = make_rsrc(out + tok * d, row_bytes);
#pragma unroll
    for (int j = 0; j < VPL; ++j) st16_stream(orr, lane_off + j * kStep, pack<T>(acc[j]));
  }
}

// ----------------------------------------------------------------- backward
//
// Persistent and pipelined like k_fwd_res (N <= NR). Per token, with
// r_n = rsqrt(ssq_n/D + eps), logit_n = a_n r_n, alpha = softmax(logit),
// G_n = <g, v_n> (derivation of triton_op.py:205-214):
//     S        = sum_n alpha_n G_n
//     dlogit_n = alpha_n (G_n - S)      [evaluated relative to the top row's G]
//     da_n     = dlogit_n r_n
//     c_n      = 2 dssq_n = -dlogit_n a_n r_n^3 / D = -dlogit_n logit_n r_n^2 / D
//     dv_n     = alpha_n g + da_n w + c_n v_n
//     dw      += sum_n da_n v_n
// STATS: logit_n and r_n come from the forward's stats, so only G_n is reduced
// over D; otherwise a_n and ssq_n are recomputed as in the forward.
// gm != nullptr selects the gradient of the unnormalised triple (o, m, l) of
// attn_with_stats instead: g is dL/do, gm/gl are dL/dm and dL/dl per token.
// With p_n = exp(logit_n - m) and k the (first) row holding the max logit,
//     dlogit_n = p_n (G_n + gl)                              n != k
//     dlogit_k = gm - sum_{n != k} p_n (G_n + gl)           (p_k = 1, m = logit_k)
// and dv_n = p_n g + da_n w + c_n v_n with da_n, c_n as above.
// VAR (a BwdVariant) fixes at compile time what the kernel is: the operator's
// gradient over stacked rows (base + n*stride), the same over per-row pointers
// for v and dv (the pointer-list entry points), or the (o, m, l) gradient over
// stacked rows. Each variant keeps only its own scalar code and addressing:
// per-row pointers cost two SGPRs a row and the (o, m, l) algebra extra VALU,
// which the operator's kernel does not pay.
// grad_out and each source row are refilled with the next token's data as soon
// as they have been consumed. The per-token scalars (logit_n and r_n from the
// stats, and gm/gl) are fetched one token ahead by a single vector load, lane
// i < 16 holding logit_i, lane 16 + i r_i, lanes 32/33 gm/gl, and broadcast
// with readlane: read as uniform scalars they would be scalar loads waited on
// one by one in every token's critical path.
// dw: each slot accumulates in registers; at the end the slots are folded in
// a fixed tree through LDS and the workgroup writes one fp32 row of `partial`.
// No float atomics anywhere, so dw is bit-reproducible for a given grid.
enum BwdVariant { kBwdStacked = 0, kBwdListed = 1, kBwdStatsGrad = 2 };

template <class T, int W, int VPL, int NR, bool STATS, int VAR>
__global__ void __launch_bounds__((BwdGeom<W, VPL, NR>::kBlock))
k_bwd(const RowTable v, const typename T::storage* __restrict__ w,
      const typename T::storage* __restrict__ g, const float* __restrict__ stats,
      const float* __restrict__ gm, const float* __restrict__ gl, const RowTable dv,
      float* __restrict__ partial, int n_src, int64_t n_tok, int d, float eps, float inv_d,
      int n_iter) {
  constexpr bool LISTED = VAR == kBwdListed;
  constexpr bool GRAD_STATS = VAR == kBwdStatsGrad;
  using S = typename T::storage;
  constexpr int CE = T::ce;
  constexpr int TPB = BwdGeom<W, VPL, NR>::kTpb;
  constexpr uint32_t kStep = 64u * W * 16u;
  constexpr int kLaneFloats = VPL * CE;  // dw values a lane accumulates
  constexpr int G = STATS ? 1 : 3;       // per-row scalars reduced over D
  // Slot fold buffer: the upper half of the live slots parks its dw here. The
  // +1 pad keeps the lane-strided writes free of bank conflicts.
  constexpr int kFH = TPB > 1 ? TPB / 2 : 1;
  constexpr int kFW = TPB > 1 ? W : 1;
  constexpr int kFL = TPB > 1 ? 64 : 1;
  __shared__ float red[2][TPB][W][G * NR];
  __shared__ float fold[kFH][kFW][kFL][kLaneFloats + 1];

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int slot = wave / W;
  const int seg = wave % W;
  const uint32_t row_bytes = (uint32_t)d * sizeof(S);
  const uint32_t lane_off = (uint32_t)(seg * 64 + lane) * 16u;
  const int64_t slots = (int64_t)gridDim.x * TPB;
  const int64_t first = (int64_t)blockIdx.x * TPB + slot;
  const int rows = n_src;  // host guarantees n_src <= NR
  // Row guards: opaque up to 9 rows (backward 55.6 vs 55.9 us at config 2), plain at 16
  // rows, where the opaque form measured 0.2 us slower.
  auto live_row = [&](int n) {
    if constexpr (NR <= 9) return n < opaque(rows);
    else return n < rows;
  };
  int iters = n_iter;
  if constexpr (W == 1) {
    // No barrier inside the loop: each wave runs only its own tokens.
    iters = first < n_tok ? (int)((n_tok - first + slots - 1) / slots) : 0;
  }

  // Eight waves of four 16-bit chunks share each SIMD two by two (256 VGPRs a
  // wave): there w and the token's grad_out stay packed and are widened where
  // they are used, which frees the 32 VGPRs their fp32 copies would take
  // beyond the packed ones (at 9 rows the copies spill 92 VGPRs).
  // (The fp32 copies below are then dead code.)
  constexpr bool kLean = W == 8 && VPL == 4 && CE == 8;
  // dv store policy: nt plus the device-scope bit for 16-bit 9-row tiles whose
  // wave slice spans four chunks (MI355X, backward main kernel, bf16 T=4096, two
  // interleaved rounds: D=2048 55.5 -> 55.1 us, D=4096 110.4 -> 109.3, D=8192
  // 223.2 -> 221.5), nt alone elsewhere (N=4 27.6 vs 28.8, N=16 97.4 vs 98.2,
  // fp32 N=9 111.8 vs 112.7, D=1024 B=4 (two chunks) 118.9 vs 119.5 with the bit).
  constexpr int kDvAux = CE == 8 && NR == 9 && W * VPL >= 4 ? SY_DV_STORE_AUX : SY_STREAM_STORE_AUX;
  float wf[VPL][CE];
  i32x4_t wq[VPL];
  {
    const auto wr = make_rsrc(w, row_bytes);
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      wq[j] = ld16(wr, lane_off + j * kStep);
#pragma unroll
      for (int e = 0; e < CE; ++e) wf[j][e] = elem<T>(wq[j], e);
    }
  }
  float dwa[VPL][CE];
#pragma unroll
  for (int j = 0; j < VPL; ++j)
#pragma unroll
    for (int e = 0; e < CE; ++e) dwa[j][e] = 0.0f;

  i32x4_t x[NR][VPL];
  i32x4_t gq[VPL];
  {
    const int64_t t0 = first < n_tok ? first : n_tok - 1;
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      if (live_row(n)) {
        const auto r = make_rsrc(row_at<LISTED, const S>(v, n) + t0 * d, row_bytes);
#pragma unroll
        for (int j = 0; j < VPL; ++j) x[n][j] = ld16_stream(r, lane_off + j * kStep);
      }
    }
    const auto gr = make_rsrc(g + t0 * d, row_bytes);
#pragma unroll
    for (int j = 0; j < VPL; ++j) gq[j] = ld16_stream(gr, lane_off + j * kStep);
  }
  // Lanes per statistic: 16 (lanes 32 and 33 then carry gm, gl), or 32 for
  // the 32-row tile, whose stats fill the wave (logits in lanes 0..31, r in
  // 32..63) and which exists only for the operator's gradient with stats.
  constexpr int kSL = NR <= 16 ? 16 : 32;
  static_assert(NR <= 32, "token scalars are spread over the lanes of one wave");
  static_assert(NR <= 16 || (STATS && !GRAD_STATS && !LISTED),
                "the 32-row tile serves the stacked operator gradient with stats only");
  // The token scalars of token t for this lane (see above); 0 for idle lanes.
  auto scalars_of = [&](int64_t t) -> float {
    const int i = lane & (kSL - 1);
    if constexpr (STATS) {
      if (lane < 2 * kSL && i < rows) return stats[(int64_t)((lane / kSL) * n_src + i) * n_tok + t];
    }
    if constexpr (GRAD_STATS) {
      if (lane == 32) return gm[t];
      if (lane == 33) return gl[t];
    }
    return 0.0f;
  };
  [[maybe_unused]] float sc_next = 0.0f;
  if constexpr (STATS || GRAD_STATS) sc_next = scalars_of(first < n_tok ? first : n_tok - 1);

  for (int k = 0; k < iters; ++k) {
    const int64_t tok_raw = first + (int64_t)k * slots;
    const bool live = tok_raw < n_tok;
    const int64_t tok = live ? tok_raw : n_tok - 1;
    const bool more = k + 1 < iters;
    const int64_t nxt = tok_raw + slots < n_tok ? tok_raw + slots : n_tok - 1;
    [[maybe_unused]] const float sc = sc_next;
    if constexpr (STATS || GRAD_STATS) {
      if (more) sc_next = scalars_of(nxt);
    }
    auto scalar = [&](int i) -> float {
      return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sc), i));
    };

    // part[n] grad dot; without stats also part[NR + n] query dot and
    // part[2*NR + n] sum of squares.
    float part[G * NR];
    if constexpr (NR <= 9) {
      constexpr int P = pow2_at_least(G * NR);
      float tv[P];
#pragma unroll
      for (int i = 0; i < P; ++i) tv[i] = 0.0f;
#pragma unroll
      for (int n = 0; n < NR; ++n) {
        if (live_row(n)) {
          float gg = 0.0f;
#pragma unroll
          for (int j = 0; j < VPL; ++j) gg = dot<T>(x[n][j], gq[j], gg);
          tv[n] = gg;
          if constexpr (!STATS) {
            float dt = 0.0f, ss = 0.0f;
#pragma unroll
            for (int j = 0; j < VPL; ++j) {
              dt = dot<T>(x[n][j], wq[j], dt);
              ss = dot<T>(x[n][j], x[n][j], ss);
            }
            tv[NR + n] = dt;
            tv[2 * NR + n] = ss;
          }
        }
      }
      row_sums_transposed<W, G, NR, TPB, P>(tv, part, G, rows, red[k & 1], slot, seg, lane);
    } else {
#pragma unroll
      for (int n = 0; n < NR; ++n) {
        if (live_row(n)) {
          float gg = 0.0f;
#pragma unroll
          for (int j = 0; j < VPL; ++j) gg = dot<T>(x[n][j], gq[j], gg);
          part[n] = wave_sum(gg);
          if constexpr (!STATS) {
            float dt = 0.0f, ss = 0.0f;
#pragma unroll
            for (int j = 0; j < VPL; ++j) {
              dt = dot<T>(x[n][j], wq[j], dt);
              ss = dot<T>(x[n][j], x[n][j], ss);
            }
            part[NR + n] = wave_sum(dt);
            part[2 * NR + n] = wave_sum(ss);
          }
        }
      }
      if constexpr (W > 1) cross_wave_sum<W, G, NR, TPB>(part, G, rows, red[k & 1], slot, seg, lane);
    }

    // gref = G of the row with the largest logit. Measuring G from it makes
    // the softmax backward free of cancellation: G_n - S equals
    // (G_n - gref) - sum_k alpha_k (G_k - gref), in which the dominant row's
    // term is exactly zero, so a saturated softmax (alpha_max -> 1) still gets
    // its tiny dlogit to full relative precision instead of G_max - S ~ 0.
    float lg[NR], rr[NR];
    float m = -INFINITY, gref = 0.0f;
    [[maybe_unused]] int top = 0;
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      if (live_row(n)) {
        if constexpr (STATS) {
          lg[n] = scalar(n);
          rr[n] = scalar(kSL + n);
        } else {
          rr[n] = rsqrtf(fmaf(part[2 * NR + n], inv_d, eps));
          lg[n] = part[NR + n] * rr[n];
        }
        if (lg[n] > m) {
          m = lg[n];
          gref = part[n];
          if constexpr (GRAD_STATS) top = n;
        }
      }
    }
    float al[NR];
    float l = 0.0f;
#pragma unroll
    for (int n = 0; n < NR; ++n)
      if (live_row(n)) {
        al[n] = expf(lg[n] - m);
        l += al[n];
      }
    // Afterwards dlogit_n = al[n] * (part[n] - sdev) in both modes.
    float sdev = 0.0f;
    if constexpr (!GRAD_STATS) {
      const float inv_l = 1.0f / l;
#pragma unroll
      for (int n = 0; n < NR; ++n)
        if (live_row(n)) {
          al[n] *= inv_l;
          part[n] -= gref;
          sdev = fmaf(al[n], part[n], sdev);
        }
    } else {
      const float glv = scalar(33), gmv = scalar(32);
      float other = 0.0f;
#pragma unroll
      for (int n = 0; n < NR; ++n)
        if (live_row(n)) {
          part[n] += glv;
          if (n != top) other = fmaf(al[n], part[n], other);
        }
#pragma unroll
      for (int n = 0; n < NR; ++n)
        if (n < rows && n == top) part[n] = gmv - other;
    }

    float gf[VPL][CE];
#pragma unroll
    for (int j = 0; j < VPL; ++j)
#pragma unroll
      for (int e = 0; e < CE; ++e) gf[j][e] = elem<T>(gq[j], e);
    [[maybe_unused]] i32x4_t gk[VPL];  // lean tiles: this token's grad_out, packed
    if constexpr (kLean) {
#pragma unroll
      for (int j = 0; j < VPL; ++j) gk[j] = gq[j];
    }
    if (more) {
      const auto gr = make_rsrc(g + nxt * d, row_bytes);
#pragma unroll
      for (int j = 0; j < VPL; ++j) gq[j] = ld16_stream(gr, lane_off + j * kStep);
    }
    const float dw_on = live ? 1.0f : 0.0f;
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      if (live_row(n)) {
        const float dlogit = al[n] * (part[n] - sdev);
        const float da = dlogit * rr[n];
        const float c = -dlogit * lg[n] * rr[n] * rr[n] * inv_d;
        const float da_w = da * dw_on;
        const auto dr = make_rsrc(row_at<LISTED, S>(dv, n) + tok * d, live ? row_bytes : 0u);
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
          float f[CE];
          if constexpr (kLean) {
            // Lean tiles widen w and grad_out again for every row: opaque
            // copies of the packed words keep the compiler from hoisting the
            // conversions out of the loops, which would rebuild the fp32 copies.
            i32x4_t wj = wq[j], gj = gk[j];
            asm volatile("" : "+v"(wj), "+v"(gj));
#pragma unroll
            for (int e = 0; e < CE; ++e) {
              float xv = elem<T>(x[n][j], e);
              if constexpr (T::code == F16::code) asm volatile("" : "+v"(xv));
              f[e] = fmaf(c, xv, fmaf(da, elem<T>(wj, e), al[n] * elem<T>(gj, e)));
              dwa[j][e] = fmaf(da_w, xv, dwa[j][e]);
            }
          } else {
#pragma unroll
            for (int e = 0; e < CE; ++e) {
              // fp16: an opaque fp32 copy, so that the two FMAs below do not
              // each fold the conversion into a v_fma_mix (which costs the
              // tile register moves: N=9 58.2 vs 56.2 us, N=16 103.1 vs 99.1).
              float xv = elem<T>(x[n][j], e);
              if constexpr (T::code == F16::code) asm volatile("" : "+v"(xv));
              f[e] = fmaf(c, xv, fmaf(da, wf[j][e], al[n] * gf[j][e]));
              dwa[j][e] = fmaf(da_w, xv, dwa[j][e]);
            }
          }
          st16_aux<kDvAux>(dr, lane_off + j * kStep, pack<T>(f));
        }
        if (more) {
          const auto r = make_rsrc(row_at<LISTED, const S>(v, n) + nxt * d, row_bytes);
#pragma unroll
          for (int j = 0; j < VPL; ++j) x[n][j] = ld16_stream(r, lane_off + j * kStep);
        }
      }
    }
  }

  // Fold the TPB slot accumulators: slots [h, 2h) add into [0, h), h halving.
#pragma unroll
  for (int h = TPB / 2; h >= 1; h /= 2) {
    __syncthreads();
    if (slot >= h && slot < 2 * h) {
#pragma unroll
      for (int j = 0; j < VPL; ++j)
#pragma unroll
        for (int e = 0; e < CE; ++e) fold[slot - h][seg][lane][j * CE + e] = dwa[j][e];
    }
    __syncthreads();
    if (slot < h) {
#pragma unroll
      for (int j = 0; j < VPL; ++j)
#pragma unroll
        for (int e = 0; e < CE; ++e) dwa[j][e] += fold[slot][seg][lane][j * CE + e];
    }
  }
  if (slot == 0) {
    const auto pr = make_rsrc(partial + (int64_t)blockIdx.x * d, (uint32_t)d * 4u);
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      // chunk c covers elements [c*CE, c*CE + CE): CE/4 float4 stores
      const uint32_t base = (lane_off / 16u + j * 64u * W) * CE * 4u;
#pragma unroll
      for (int q4 = 0; q4 < CE / 4; ++q4) {
        i32x4_t t;
#pragma unroll
        for (int e = 0; e < 4; ++e) t[e] = __float_as_int(dwa[j][q4 * 4 + e]);
        st16(pr, base + q4 * 16u, t);
      }
    }
  }
}


// ------------------------------------------------ backward, 17 to 64 sources
//
// The operator's gradient with the forward's stats over stacked rows for
// 16 < N <= NR (NR = 32 or 64): k_bwd's algebra, persistence and row-by-row
// refill, with the token's per-row scalars laid out across lanes instead of
// held as uniform values: lane n of one VGPR each carries row n's G_n, logit,
// r, alpha, da and c. The softmax backward is then a few lane-parallel
// operations and three wave reductions, where 32 rows of uniform scalar code
// (as k_bwd writes it) needed ~300 SGPRs and spilled them into VGPR lanes on
// every token. The dv loop broadcasts row n's three coefficients with readlane
// as it reaches the row. Rows n >= N are never loaded; their lanes carry
// logit -inf (weight 0) and zero coefficients. 64 rows of one chunk a lane
// hold 256 tile VGPRs and run one wave per SIMD; their grad dots are summed as
// two 32-row transposed sums.
template <int W, int VPL, int NR>
struct TallGeom {
  static constexpr int kBlock = bwd_block(W, VPL, NR);
  static constexpr int kTpb = kBlock / (64 * W);
};

template <class T, int W, int VPL, int NR>
__global__ void __launch_bounds__((TallGeom<W, VPL, NR>::kBlock))
k_bwd_tall(const RowTable v, const typename T::storage* __restrict__ w,
           const typename T::storage* __restrict__ g, const float* __restrict__ stats,
           const RowTable dv, float* __restrict__ partial, int n_src, int64_t n_tok, int d,
           float inv_d, int n_iter) {
  using S = typename T::storage;
  constexpr int CE = T::ce;
  static_assert(NR == 32 || NR == 64, "tall tiles hold 32 or 64 rows");
  constexpr int TPB = TallGeom<W, VPL, NR>::kTpb;
  constexpr uint32_t kStep = 64u * W * 16u;
  constexpr int kLaneFloats = VPL * CE;
  constexpr int kFH = TPB > 1 ? TPB / 2 : 1;
  constexpr int kFW = TPB > 1 ? W : 1;
  constexpr int kFL = TPB > 1 ? 64 : 1;
  static_assert(W > 1, "a 32-row token spans at least two waves");
  __shared__ float red[2][TPB][W][NR];
  __shared__ float fold[kFH][kFW][kFL][kLaneFloats + 1];

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int slot = wave / W;
  const int seg = wave % W;
  const uint32_t row_bytes = (uint32_t)d * sizeof(S);
  const uint32_t lane_off = (uint32_t)(seg * 64 + lane) * 16u;
  const int64_t slots = (int64_t)gridDim.x * TPB;
  const int64_t first = (int64_t)blockIdx.x * TPB + slot;
  const int rows = n_src;  // host guarantees 16 < n_src <= NR
  const bool row_lane = lane < rows;
  const int iters = n_iter;  // every slot meets the same barriers

  float wf[VPL][CE];
  i32x4_t wq[VPL];
  {
    const auto wr = make_rsrc(w, row_bytes);
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      wq[j] = ld16(wr, lane_off + j * kStep);
#pragma unroll
      for (int e = 0; e < CE; ++e) wf[j][e] = elem<T>(wq[j], e);
    }
  }
  float dwa[VPL][CE];
#pragma unroll
  for (int j = 0; j < VPL; ++j)
#pragma unroll
    for (int e = 0; e < CE; ++e) dwa[j][e] = 0.0f;

  i32x4_t x[NR][VPL];
  i32x4_t gq[VPL];
  const int64_t t0 = first < n_tok ? first : n_tok - 1;
  {
    const S* vrow = static_cast<const S*>(v.p[0]) + t0 * d;
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      if (n < opaque(rows)) {
        asm volatile("" : "+s"(vrow));
        const auto r = make_rsrc(vrow, row_bytes);
#pragma unroll
        for (int j = 0; j < VPL; ++j) x[n][j] = ld16_stream(r, lane_off + j * kStep);
        vrow = reinterpret_cast<const S*>(reinterpret_cast<const char*>(vrow) + v.stride_bytes);
      }
    }
    const auto gr = make_rsrc(g + t0 * d, row_bytes);
#pragma unroll
    for (int j = 0; j < VPL; ++j) gq[j] = ld16_stream(gr, lane_off + j * kStep);
  }
  // Row `lane`'s logit and inverse RMS of token t, one token ahead.
  auto logit_of = [&](int64_t t) { return row_lane ? stats[(int64_t)lane * n_tok + t] : -INFINITY; };
  auto rinv_of = [&](int64_t t) { return row_lane ? stats[(int64_t)(n_src + lane) * n_tok + t] : 0.0f; };
  float lg_next = logit_of(t0), r_next = rinv_of(t0);

  for (int k = 0; k < iters; ++k) {
    const int64_t tok_raw = first + (int64_t)k * slots;
    const bool live = tok_raw < n_tok;
    const int64_t tok = live ? tok_raw : n_tok - 1;
    const bool more = k + 1 < iters;
    const int64_t nxt = tok_raw + slots < n_tok ? tok_raw + slots : n_tok - 1;
    const float lg = lg_next, rr = r_next;
    if (more) {
      lg_next = logit_of(nxt);
      r_next = rinv_of(nxt);
    }

    // G_n = <g, v_n>: this wave's share (transposed sum: row tsum32_row(l) in
    // lane l), then the W shares of the token added in segment order through
    // LDS into lane n.
    float gv = 0.0f;
    {
      float dts[NR];
#pragma unroll
      for (int n = 0; n < NR; ++n) {
        dts[n] = 0.0f;
        if (n < opaque(rows)) {
#pragma unroll
          for (int j = 0; j < VPL; ++j) dts[n] = dot<T>(x[n][j], gq[j], dts[n]);
        }
      }
      if constexpr (NR == 32) {
        const float s = tsum32(dts, lane);
        if ((lane & 2) == 0) red[k & 1][slot][seg][tsum32_row(lane)] = s;
      } else {
        float lo[32], hi[32];
#pragma unroll
        for (int n = 0; n < 32; ++n) {
          lo[n] = dts[n];
          hi[n] = dts[32 + n];
        }
        const float s0 = tsum32(lo, lane), s1 = tsum32(hi, lane);
        if ((lane & 2) == 0) {
          red[k & 1][slot][seg][tsum32_row(lane)] = s0;
          red[k & 1][slot][seg][32 + tsum32_row(lane)] = s1;
        }
      }
    }
    __syncthreads();
    if (lane < NR) {
      float t = red[k & 1][slot][0][lane];
#pragma unroll
      for (int q = 1; q < W; ++q) t += red[k & 1][slot][q][lane];
      gv = t;
    }

    // Softmax backward across lanes, relative to the first row with the
    // largest logit (cancellation-free, as in k_bwd).
    const float m = wave_max(lg);
    const int top = (int)__builtin_ctzll(__builtin_amdgcn_ballot_w64(lg == m));
    const float gref = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gv), top));
    float al = row_lane ? expf(lg - m) : 0.0f;
    al *= 1.0f / wave_sum(al);
    const float dd = row_lane ? gv - gref : 0.0f;
    const float sdev = wave_sum(al * dd);
    const float dlogit = al * (dd - sdev);
    const float da = dlogit * rr;
    const float c = -dlogit * (row_lane ? lg : 0.0f) * rr * rr * inv_d;

    float gf[VPL][CE];
#pragma unroll
    for (int j = 0; j < VPL; ++j)
#pragma unroll
      for (int e = 0; e < CE; ++e) gf[j][e] = elem<T>(gq[j], e);
    if (more) {
      const auto gr = make_rsrc(g + nxt * d, row_bytes);
#pragma unroll
      for (int j = 0; j < VPL; ++j) gq[j] = ld16_stream(gr, lane_off + j * kStep);
    }
    const float dw_on = live ? 1.0f : 0.0f;
    float alv = al, dav = da, cv = c;
    // Row n's addresses walk from row 0 one stride at a time; the empty asm
    // keeps the walk serial, so the 2 x 32 row addresses (and their buffer
    // resources) are never all live at once in SGPRs.
    const S* vrow = static_cast<const S*>(v.p[0]) + nxt * d;
    S* dvrow = static_cast<S*>(dv.p[0]) + tok * d;
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      if (n < opaque(rows)) {
        // Keep the broadcasts at their row: hoisted, the 3 x 32 uniform
        // coefficients would need SGPRs again.
        asm volatile("" : "+v"(alv), "+v"(dav), "+v"(cv), "+s"(vrow), "+s"(dvrow));
        const float aln = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alv), n));
        const float dan = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dav), n));
        const float cn = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cv), n));
        const float da_w = dan * dw_on;
        const auto dr = make_rsrc(dvrow, live ? row_bytes : 0u);
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
          float f[CE];
#pragma unroll
          for (int e = 0; e < CE; ++e) {
            // fp16: converted once into an opaque fp32 copy (see k_bwd; here
            // N=32 247.5 vs 205.4 us).
            float xv = elem<T>(x[n][j], e);
            if constexpr (T::code == F16::code) asm volatile("" : "+v"(xv));
            f[e] = fmaf(cn, xv, fmaf(dan, wf[j][e], aln * gf[j][e]));
            dwa[j][e] = fmaf(da_w, xv, dwa[j][e]);
          }
          // nt plus the device-scope bit (bf16 backward N=32 207.1 -> 201.6 us, N=48
          // 352.7 -> 348.4)
          st16_aux<SY_DV_STORE_AUX>(dr, lane_off + j * kStep, pack<T>(f));
        }
        if (more) {
          const auto r = make_rsrc(vrow, row_bytes);
#pragma unroll
          for (int j = 0; j < VPL; ++j) x[n][j] = ld16_stream(r, lane_off + j * kStep);
        }
        vrow = reinterpret_cast<const S*>(reinterpret_cast<const char*>(vrow) + v.stride_bytes);
        dvrow = reinterpret_cast<S*>(reinterpret_cast<char*>(dvrow) + dv.stride_bytes);
      }
    }
  }

  // Fold the TPB slot accumulators (slots [h, 2h) into [0, h)), then one fp32
  // partial row per workgroup.
#pragma unroll
  for (int h = TPB / 2; h >= 1; h /= 2) {
    __syncthreads();
    if (slot >= h && slot < 2 * h) {
#pragma unroll
      for (int j = 0; j < VPL; ++j)
#pragma unroll
        for (int e = 0; e < CE; ++e) fold[slot - h][seg][lane][j * CE + e] = dwa[j][e];
    }
    __syncthreads();
    if (slot < h) {
#pragma unroll
      for (int j = 0; j < VPL; ++j)
#pragma unroll
        for (int e = 0; e < CE; ++e) dwa[j][e] += fold[slot][seg][lane][j * CE + e];
    }
  }
  if (slot == 0) {
    const auto pr = make_rsrc(partial + (int64_t)blockIdx.x * d, (uint32_t)d * 4u);
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const uint32_t base = (lane_off / 16u + j * 64u * W) * CE * 4u;
#pragma unroll
      for (int q4 = 0; q4 < CE / 4; ++q4) {
        i32x4_t t;
#pragma unroll
        for (int e = 0; e < 4; ++e) t[e] = __float_as_int(dwa[j][q4 * 4 + e]);
        st16(pr, base + q4 * 16u, t);
      }
    }
  }
}


// ------------------------------------------------------- batched backward
//
// Gradient of the batched forward out[s] = AttnRes(v, q_s), s < n_q <= SQ, for
// grad_out g [S][n_tok][D]. The S queries are S operators sharing v, so per
// token (with alpha, logit, r of query s, G_sn = <g_s, v_n>):
//     dlogit_sn = alpha_sn (G_sn - sum_k alpha_sk G_sk)   [relative to the top row]
//     da_sn     = dlogit_sn r_n,   c_n = -sum_s dlogit_sn logit_sn r_n^2 / D
//     dv_n      = sum_s (alpha_sn g_s + da_sn q_s) + c_n v_n
//     dq_s     += sum_n da_sn v_n
// The token's N rows are read once for all queries; dv is accumulated over the
// queries in fp32 registers and rounded once; dq_s is accumulated over the
// workgroup's tokens in LDS (each lane owns its float4 slots, so no barrier
// is needed until the end) and written as one fp32 partial row per query
// ([grid][n_q][D]), reduced afterwards in a fixed order like dw. Registers
// would hold dv's NR x CE and the tile, but not SQ x CE more without spilling.
// One token per W waves with one chunk per lane (VPL = 1), persistent and
// pipelined like k_bwd. Reference: the batched forward is
// src/switchyard/triton_op.py:378-501; it has no backward.
// EXACT: n_src == NR, so every per-row guard is a compile-time constant (with
// a runtime row count each of the ~18 guarded blocks per query becomes a
// branch, and the merges cost register moves).
template <class T, int W, int NR, int SQ, bool EXACT>
__global__ void __launch_bounds__(FwdGeom<W>::kBlock)
k_bwd_batched(const RowTable v, const typename T::storage* __restrict__ q,
              const typename T::storage* __restrict__ g, const RowTable dv,
              float* __restrict__ partial, int n_src, int n_q, int64_t n_tok, int d, float eps,
              float inv_d, int n_iter) {
  using S = typename T::storage;
  constexpr int CE = T::ce;
  constexpr int TPB = FwdGeom<W>::kTpb;
  constexpr int kQ4 = SQ * CE / 4;  // float4 dq accumulators per lane
  // Two ping-pong buffer pairs: red1 for the sums of squares (once per
  // token), red for the per-query dots (`phase` advances per exchange).
  __shared__ float red1[2][TPB][W][NR];
  __shared__ float red[2][TPB][W][2 * NR];
  // dq accumulators, lane-contiguous float4: dql[wave][s*CE/4 + c][lane].
  __shared__ float4 dql[TPB * W][kQ4][64];

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int slot = wave / W;
  const int seg = wave % W;
  const uint32_t row_bytes = (uint32_t)d * sizeof(S);
  const uint32_t lane_off = (uint32_t)(seg * 64 + lane) * 16u;
  const int64_t slots = (int64_t)gridDim.x * TPB;
  const int64_t first = (int64_t)blockIdx.x * TPB + slot;
  const int rows = EXACT ? NR : n_src;  // host guarantees n_src <= NR and n_q <= SQ
  int iters = n_iter;
  if constexpr (W == 1) iters = first < n_tok ? (int)((n_tok - first + slots - 1) / slots) : 0;

#pragma unroll
  for (int c = 0; c < kQ4; ++c) dql[wave][c][lane] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);

  i32x4_t x[NR];
  {
    const int64_t t0 = first < n_tok ? first : n_tok - 1;
#pragma unroll
    for (int n = 0; n < NR; ++n)
      if (n < rows) x[n] = ld16_stream(make_rsrc(row_at<false, const S>(v, n) + t0 * d, row_bytes), lane_off);
  }

  [[maybe_unused]] int phase = 0;
  for (int k = 0; k < iters; ++k) {
    const int64_t tok_raw = first + (int64_t)k * slots;
    const bool live = tok_raw < n_tok;
    const int64_t tok = live ? tok_raw : n_tok - 1;
    const bool more = k + 1 < iters;
    const int64_t nxt = tok_raw + slots < n_tok ? tok_raw + slots : n_tok - 1;

    float rr[NR];
#pragma unroll
    for (int n = 0; n < NR; ++n)
      if (n < rows) rr[n] = wave_sum(dot<T>(x[n], x[n], 0.0f));
    if constexpr (W > 1) cross_wave_sum<W, 1, NR, TPB>(rr, 1, rows, red1[k & 1], slot, seg, lane);
#pragma unroll
    for (int n = 0; n < NR; ++n)
      if (n < rows) rr[n] = rsqrtf(fmaf(rr[n], inv_d, eps));

    float dva[NR][CE];
    float cacc[NR];
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      cacc[n] = 0.0f;
#pragma unroll
      for (int e = 0; e < CE; ++e) dva[n][e] = 0.0f;
    }

    // Queries in a runtime loop; query s+1's rows are loaded while s is used.
    i32x4_t gq = ld16_stream(make_rsrc(g + tok * d, row_bytes), lane_off);
    i32x4_t qq = ld16(make_rsrc(q, row_bytes), lane_off);
#pragma unroll 1
    for (int s = 0; s < n_q; ++s) {
      // Keep the tile opaque to loop-invariant motion: otherwise its fp32
      // conversions are hoisted out of the query loop (NR x CE more VGPRs).
#pragma unroll
      for (int n = 0; n < NR; ++n)
        if (n < rows) asm volatile("" : "+v"(x[n]));
      {
        i32x4_t gn = gq, qn = qq;
        if (s + 1 < n_q) {
          gn = ld16_stream(make_rsrc(g + ((int64_t)(s + 1) * n_tok + tok) * d, row_bytes), lane_off);
          qn = ld16(make_rsrc(q + (int64_t)(s + 1) * d, row_bytes), lane_off);
        }
        float part[2 * NR];
#pragma unroll
        for (int n = 0; n < NR; ++n) {
          if (n < rows) {
            part[n] = wave_sum(dot<T>(x[n], gq, 0.0f));
            part[NR + n] = wave_sum(dot<T>(x[n], qq, 0.0f));
          }
        }
        if constexpr (W > 1) cross_wave_sum<W, 2, NR, TPB>(part, 2, rows, red[phase++ & 1], slot, seg, lane);
        float lg[NR], al[NR];
        float m = -INFINITY, gref = 0.0f;
#pragma unroll
        for (int n = 0; n < NR; ++n) {
          if (n < rows) {
            lg[n] = part[NR + n] * rr[n];
            if (lg[n] > m) {
              m = lg[n];
              gref = part[n];
            }
          }
        }
        float l = 0.0f;
#pragma unroll
        for (int n = 0; n < NR; ++n)
          if (n < rows) {
            al[n] = expf(lg[n] - m);
            l += al[n];
          }
        const float inv_l = 1.0f / l;
        float sdev = 0.0f;
#pragma unroll
        for (int n = 0; n < NR; ++n)
          if (n < rows) {
            al[n] *= inv_l;
            part[n] -= gref;
            sdev = fmaf(al[n], part[n], sdev);
          }
        float u[CE];
#pragma unroll
        for (int e = 0; e < CE; ++e) u[e] = 0.0f;
#pragma unroll
        for (int n = 0; n < NR; ++n) {
          if (n < rows) {
            const float dlogit = al[n] * (part[n] - sdev);
            const float da = dlogit * rr[n];
            cacc[n] = fmaf(-dlogit * lg[n], rr[n] * rr[n] * inv_d, cacc[n]);
#pragma unroll
            for (int e = 0; e < CE; ++e) {
              dva[n][e] = fmaf(al[n], elem<T>(gq, e), fmaf(da, elem<T>(qq, e), dva[n][e]));
              u[e] = fmaf(da, elem<T>(x[n], e), u[e]);
            }
          }
        }
        if (live) {
#pragma unroll
          for (int c = 0; c < CE / 4; ++c) {
            float4 a = dql[wave][s * (CE / 4) + c][lane];
            a.x += u[4 * c];
            a.y += u[4 * c + 1];
            a.z += u[4 * c + 2];
            a.w += u[4 * c + 3];
            dql[wave][s * (CE / 4) + c][lane] = a;
          }
        }
        gq = gn;
        qq = qn;
      }
    }

#pragma unroll
    for (int n = 0; n < NR; ++n) {
      if (n < rows) {
        float f[CE];
#pragma unroll
        for (int e = 0; e < CE; ++e) f[e] = fmaf(cacc[n], elem<T>(x[n], e), dva[n][e]);
        st16_stream(make_rsrc(row_at<false, S>(dv, n) + tok * d, live ? row_bytes : 0u), lane_off, pack<T>(f));
        if (more) x[n] = ld16_stream(make_rsrc(row_at<false, const S>(v, n) + nxt * d, row_bytes), lane_off);
      }
    }
  }

  // Sum the TPB slots' accumulators in slot order, then one fp32 partial row
  // per query: partial[blockIdx][s][:].
  __syncthreads();
  if (slot == 0) {
    const uint32_t base = (lane_off / 16u) * CE * 4u;
#pragma unroll
    for (int s = 0; s < SQ; ++s) {
      if (s < n_q) {
        const auto pr = make_rsrc(partial + ((int64_t)blockIdx.x * n_q + s) * d, (uint32_t)d * 4u);
#pragma unroll
        for (int c = 0; c < CE / 4; ++c) {
          float4 a = dql[seg][s * (CE / 4) + c][lane];
#pragma unroll
          for (int k = 1; k < TPB; ++k) {
            const float4 b = dql[k * W + seg][s * (CE / 4) + c][lane];
            a.x += b.x;
            a.y += b.y;
            a.z += b.z;
            a.w += b.w;
          }
          i32x4_t t;
          t[0] = __float_as_int(a.x);
          t[1] = __float_as_int(a.y);
          t[2] = __float_as_int(a.z);
          t[3] = __float_as_int(a.w);
          st16(pr, base + c * 16u, t);
        }
      }
    }
  }
}

}  // namespace sy
