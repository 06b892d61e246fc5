// Generic kernels for shapes the register-tiled kernels do not cover: rows
// that are not 16-byte aligned (D = 777, D = 63, ...), a query whose dtype
// differs from v's, N beyond the tile budgets, or very wide D. One 256-thread
// workgroup per token, element-wise loads, two passes: the first computes the
// per-row scalars (kept in LDS), the second re-reads v to produce outputs. The
// second read is served from L2 for all but the widest rows. These are
// correctness paths; the vector kernels carry the performance.
//
// Also here: the deterministic dw reduction that finishes every backward, and
// the HBM probes (reference bench/machine.py:41-61).
#include "sy_device.hpp"
#include "sy_launch.hpp"

namespace sy {

namespace {

constexpr int kBlock = 256;

// Block-wide sum / max with a fixed combination order. `scr` holds >= 257
// floats; callers must not reuse it until the next barrier.
__device__ float block_sum(float x, float* scr) {
  const int tid = threadIdx.x;
  scr[tid] = x;
  __syncthreads();
  if (tid < 64) {
    float s = ((scr[tid] + scr[tid + 64]) + scr[tid + 128]) + scr[tid + 192];
    s = wave_sum(s);
    if (tid == 0) scr[256] = s;
  }
  __syncthreads();
  const float r = scr[256];
  __syncthreads();
  return r;
}

__device__ float block_max(float x, float* scr) {
  const int tid = threadIdx.x;
  scr[tid] = x;
  __syncthreads();
  if (tid < 64) {
    float s = fmaxf(fmaxf(scr[tid], scr[tid + 64]), fmaxf(scr[tid + 128], scr[tid + 192]));
    s = wave_max(s);
    if (tid == 0) scr[256] = s;
  }
  __syncthreads();
  const float r = scr[256];
  __syncthreads();
  return r;
}

// Pass 1 for one token: per-row (sum of squares, query dot[, grad dot]) for
// every row, written to ss[], qd[] and gd[] in LDS. Rows go in groups of 8 so
// a thread carries 16-24 partial sums.
__device__ void row_scalars(const RowTable& v, const void* w, const void* g, int n_src,
                            int64_t tok, int d, int vt, int wt, float* ss, float* qd, float* gd,
                            float* scr) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  constexpr int R = 8;
  for (int g0 = 0; g0 < n_src; g0 += R) {
    float a[R], b[R], c[R];
#pragma unroll
    for (int r = 0; r < R; ++r) a[r] = b[r] = c[r] = 0.0f;
    for (int k = tid; k < d; k += kBlock) {
      const float wk = load_elem(w, k, wt);
      const float gk = g ? load_elem(g, tok * d + k, vt) : 0.0f;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (g0 + r < n_src) {
          const float x = load_elem(row_of<const char>(v, g0 + r), tok * d + k, vt);
          a[r] = fmaf(x, x, a[r]);
          b[r] = fmaf(x, wk, b[r]);
          c[r] = fmaf(x, gk, c[r]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      a[r] = wave_sum(a[r]);
      b[r] = wave_sum(b[r]);
      c[r] = wave_sum(c[r]);
    }
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        scr[wave * 3 * R + r] = a[r];
        scr[wave * 3 * R + R + r] = b[r];
        scr[wave * 3 * R + 2 * R + r] = c[r];
      }
    }
    __syncthreads();
    if (tid < R && g0 + tid < n_src) {
      float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f;
      for (int q = 0; q < kBlock / 64; ++q) {
        s0 += scr[q * 3 * R + tid];
        s1 += scr[q * 3 * R + R + tid];
        s2 += scr[q * 3 * R + 2 * R + tid];
      }
      ss[g0 + tid] = s0;
      qd[g0 + tid] = s1;
      if (gd) gd[g0 + tid] = s2;
    }
    __syncthreads();
  }
}

// LDS layout (floats): [0, n) lg, [n, 2n) ss/r, [2n, 3n) gd, then 257 scratch.
__global__ void __launch_bounds__(kBlock)
k_fwd_generic(const RowTable v, const void* __restrict__ w, void* __restrict__ out,
              float* __restrict__ stats, float* __restrict__ m_out, float* __restrict__ l_out,
              int normalize, int n_src, int64_t n_tok, int d, int vt, int wt, float eps,
              float inv_d) {
  extern __shared__ float sh[];
  float* lg = sh;
  float* ss = sh + n_src;
  float* scr = sh + 2 * n_src;
  const int tid = threadIdx.x;
  const int64_t tok = blockIdx.x;
  row_scalars(v, w, nullptr, n_src, tok, d, vt, wt, ss, lg, nullptr, scr);

  float m = -INFINITY;
  for (int n = tid; n < n_src; n += kBlock) {
    const float r = rsqrtf(fmaf(ss[n], inv_d, eps));
    lg[n] *= r;
    ss[n] = r;
    m = fmaxf(m, lg[n]);
  }
  m = block_max(m, scr);
  float l = 0.0f;
  for (int n = tid; n < n_src; n += kBlock) l += expf(lg[n] - m);
  l = block_sum(l, scr);
  const float inv_l = normalize ? 1.0f / l : 1.0f;
  if (m_out != nullptr && tid == 0) {
    m_out[tok] = m;
    l_out[tok] = l;
  }
  if (stats) {
    for (int n = tid; n < n_src; n += kBlock) {
      stats[(int64_t)n * n_tok + tok] = lg[n];
      stats[(int64_t)(n_src + n) * n_tok + tok] = ss[n];
    }
  }
  __syncthreads();
  for (int n = tid; n < n_src; n += kBlock) lg[n] = expf(lg[n] - m) * inv_l;
  __syncthreads();
  for (int k = tid; k < d; k += kBlock) {
    float acc = 0.0f;
    for (int n = 0; n < n_src; ++n)
      acc = fmaf(lg[n], load_elem(row_of<const char>(v, n), tok * d + k, vt), acc);
    store_elem(out, tok * d + k, acc, vt);
  }
}

__global__ void __launch_bounds__(kBlock)
k_sol_generic(const RowTable v, void* __restrict__ out, int n_src, int64_t n_tok, int d, int vt) {
  const int64_t tok = blockIdx.x;
  for (int k = threadIdx.x; k < d; k += kBlock) {
    float acc = 0.0f;
    for (int n = 0; n < n_src; ++n) acc += load_elem(row_of<const char>(v, n), tok * d + k, vt);
    store_elem(out, tok * d + k, acc, vt);
  }
}

// Persistent over tokens; workgroup b accumulates its dw contribution in its
// own fp32 row partial[b][:] (no other workgroup touches it). gm != nullptr
// selects the gradient of the unnormalised (o, m, l) triple, as in k_bwd.
__global__ void __launch_bounds__(kBlock)
k_bwd_generic(const RowTable v, const void* __restrict__ w, const void* __restrict__ g,
              const float* __restrict__ gm, const float* __restrict__ gl, const RowTable dv,
              float* __restrict__ partial, int n_src, int64_t n_tok, int d, int vt, int wt,
              float eps, float inv_d) {
  extern __shared__ float sh[];
  float* al = sh;              // logit, then alpha
  float* da = sh + n_src;      // sum of squares, then r, then da
  float* gc = sh + 2 * n_src;  // grad dot, then c
  float* scr = sh + 3 * n_src;
  const int tid = threadIdx.x;
  float* prow = partial + (int64_t)blockIdx.x * d;
  for (int k = tid; k < d; k += kBlock) prow[k] = 0.0f;

  for (int64_t tok = blockIdx.x; tok < n_tok; tok += gridDim.x) {
    row_scalars(v, w, g, n_src, tok, d, vt, wt, da, al, gc, scr);
    float m = -INFINITY;
    for (int n = tid; n < n_src; n += kBlock) {
      const float r = rsqrtf(fmaf(da[n], inv_d, eps));
      al[n] *= r;
      da[n] = r;
      m = fmaxf(m, al[n]);
    }
    m = block_max(m, scr);
    // gref = grad dot of the first row with the largest logit: the softmax
    // backward is evaluated relative to it (see k_bwd) to avoid cancellation.
    float first = (float)n_src;
    for (int n = tid; n < n_src; n += kBlock)
      if (al[n] == m) first = fminf(first, (float)n);
    first = -block_max(-first, scr);
    const int top = min((int)first, n_src - 1);
    if (gm == nullptr) {
      const float gref = gc[top];
      float l = 0.0f, sp = 0.0f;
      for (int n = tid; n < n_src; n += kBlock) {
        const float p = expf(al[n] - m);
        l += p;
        sp = fmaf(p, gc[n] - gref, sp);
      }
      l = block_sum(l, scr);
      sp = block_sum(sp, scr);
      const float inv_l = 1.0f / l;
      const float sdev = sp * inv_l;
      for (int n = tid; n < n_src; n += kBlock) {
        const float lgn = al[n], r = da[n];
        const float a = expf(lgn - m) * inv_l;
        const float dlogit = a * ((gc[n] - gref) - sdev);
        al[n] = a;
        da[n] = dlogit * r;
        gc[n] = -dlogit * lgn * r * r * inv_d;
      }
    } else {
      const float glv = gl[tok], gmv = gm[tok];
      float other = 0.0f;
      for (int n = tid; n < n_src; n += kBlock)
        if (n != top) other = fmaf(expf(al[n] - m), gc[n] + glv, other);
      other = block_sum(other, scr);
      for (int n = tid; n < n_src; n += kBlock) {
        const float lgn = al[n], r = da[n];
        const float p = expf(lgn - m);
        const float dlogit = n == top ? gmv - other : p * (gc[n] + glv);
        al[n] = p;
        da[n] = dlogit * r;
        gc[n] = -dlogit * lgn * r * r * inv_d;
      }
    }
    __syncthreads();
    for (int k = tid; k < d; k += kBlock) {
      const float gk = load_elem(g, tok * d + k, vt);
      const float wk = load_elem(w, k, wt);
      float dwk = 0.0f;
      for (int n = 0; n < n_src; ++n) {
        const float x = load_elem(row_of<const char>(v, n), tok * d + k, vt);
        store_elem(row_of<char>(dv, n), tok * d + k,
                   fmaf(gc[n], x, fmaf(da[n], wk, al[n] * gk)), vt);
        dwk = fmaf(da[n], x, dwk);
      }
      prow[k] += dwk;
    }
    __syncthreads();
  }
}

// Batched backward for the shapes the register tile does not take (see
// k_bwd_batched for the algebra). Persistent over tokens, one workgroup per
// token; per token and query the row scalars go to LDS, then one pass over D
// writes dv and adds the workgroup's dq contribution to its own fp32 rows
// partial[b][s][:]. LDS floats: al[S*N], da[S*N], c[N], r[N], ss/qd/gd[N]
// and the 257-float reduction scratch (bwd_batched_generic_lds).
__global__ void __launch_bounds__(kBlock)
k_bwd_batched_generic(const RowTable v, const void* __restrict__ q, const void* __restrict__ g,
                      const RowTable dv, float* __restrict__ partial, int n_src, int n_q,
                      int64_t n_tok, int d, int vt, float eps, float inv_d) {
  extern __shared__ float sh[];
  const int nn = n_src, sn = n_q * n_src;
  float* al = sh;
  float* da = sh + sn;
  float* cc = sh + 2 * sn;
  float* rr = cc + nn;
  float* ss = rr + nn;
  float* qd = ss + nn;
  float* gd = qd + nn;
  float* scr = gd + nn;
  const int tid = threadIdx.x;
  const int64_t es = vt == 0 ? 4 : 2;
  float* prow = partial + (int64_t)blockIdx.x * n_q * d;
  for (int64_t k = tid; k < (int64_t)n_q * d; k += kBlock) prow[k] = 0.0f;

  for (int64_t tok = blockIdx.x; tok < n_tok; tok += gridDim.x) {
    for (int n = tid; n < nn; n += kBlock) cc[n] = 0.0f;
    for (int s = 0; s < n_q; ++s) {
      const char* qs = static_cast<const char*>(q) + (int64_t)s * d * es;
      const char* gs = static_cast<const char*>(g) + (int64_t)s * n_tok * d * es;
      row_scalars(v, qs, gs, nn, tok, d, vt, vt, ss, qd, gd, scr);
      float m = -INFINITY;
      for (int n = tid; n < nn; n += kBlock) {
        const float r = rsqrtf(fmaf(ss[n], inv_d, eps));
        rr[n] = r;
        qd[n] *= r;  // logit
        m = fmaxf(m, qd[n]);
      }
      m = block_max(m, scr);
      float first = (float)nn;
      for (int n = tid; n < nn; n += kBlock)
        if (qd[n] == m) first = fminf(first, (float)n);
      first = -block_max(-first, scr);
      const float gref = gd[min((int)first, nn - 1)];
      float l = 0.0f, sp = 0.0f;
      for (int n = tid; n < nn; n += kBlock) {
        const float p = expf(qd[n] - m);
        l += p;
        sp = fmaf(p, gd[n] - gref, sp);
      }
      l = block_sum(l, scr);
      sp = block_sum(sp, scr);
      const float inv_l = 1.0f / l;
      const float sdev = sp * inv_l;
      for (int n = tid; n < nn; n += kBlock) {
        const float a = expf(qd[n] - m) * inv_l;
        const float dlogit = a * ((gd[n] - gref) - sdev);
        al[s * nn + n] = a;
        da[s * nn + n] = dlogit * rr[n];
        cc[n] = fmaf(-dlogit * qd[n], rr[n] * rr[n] * inv_d, cc[n]);
      }
      __syncthreads();
    }
    for (int k = tid; k < d; k += kBlock) {
      for (int n = 0; n < nn; ++n) {
        const float x = load_elem(row_of<const char>(v, n), tok * d + k, vt);
        float acc = cc[n] * x;
        for (int s = 0; s < n_q; ++s) {
          const float gk = load_elem(g, ((int64_t)s * n_tok + tok) * d + k, vt);
          const float qk = load_elem(q, (int64_t)s * d + k, vt);
          acc = fmaf(al[s * nn + n], gk, fmaf(da[s * nn + n], qk, acc));
        }
        store_elem(row_of<char>(dv, n), tok * d + k, acc, vt);
      }
      for (int s = 0; s < n_q; ++s) {
        float u = 0.0f;
        for (int n = 0; n < nn; ++n)
          u = fmaf(da[s * nn + n], load_elem(row_of<const char>(v, n), tok * d + k, vt), u);
        prow[(int64_t)s * d + k] += u;
      }
    }
    __syncthreads();
  }
}

// dw[c] = sum over rows r of partial[r][c] (scalar path: any D, any
// alignment), in a fixed order: wave q of the
// 1024-thread workgroup sums rows [q*rows/16, (q+1)*rows/16) in sequence, then
// the 16 wave sums are added in wave order. Same inputs, same bits.
__global__ void __launch_bounds__(1024)
k_dw_reduce(const float* __restrict__ partial, int rows, int d, void* __restrict__ dw, int wt) {
  __shared__ float sh[16][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = blockIdx.x * 64 + lane;
  float s = 0.0f;
  if (col < d) {
    const int r0 = (int)((int64_t)wave * rows / 16), r1 = (int)((int64_t)(wave + 1) * rows / 16);
    for (int r = r0; r < r1; ++r) s += partial[(int64_t)r * d + col];
  }
  sh[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && col < d) {
    float t = sh[0][lane];
#pragma unroll
    for (int q = 1; q < 16; ++q) t += sh[q][lane];
    store_elem(dw, col, t, wt);
  }
}

// dw[c] = sum over rows of partial[r][c], 16-byte path (D % 4 == 0, rows
// 16-byte aligned). A workgroup owns 64 columns: lane l of wave w is column
// group l % 16 (four columns) and row lane rl = 4w + l / 16, which sums rows
// rl, rl + 64, rl + 128, ... in that order (four loads in flight per step).
// Each wave then adds its four row lanes with two lane swaps (row lane q takes
// q ^ 2, then q ^ 1: permlane32 / permlane16), and after one barrier wave 0
// adds the 16 wave sums in wave order. Same inputs, same bits.
__global__ void __launch_bounds__(1024)
k_dw_reduce4(const float* __restrict__ partial, int rows, int d, void* __restrict__ dw, int wt) {
  __shared__ float4 sh[16][16];
  const int lane = threadIdx.x & 63;
  const int cl = lane & 15;
  const int rl = (threadIdx.x >> 6) * 4 + (lane >> 4);
  const int n4 = d / 4;
  const int c4 = blockIdx.x * 16 + cl;
  const float4* __restrict__ p4 = reinterpret_cast<const float4*>(partial);
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (c4 < n4) {
    int r = rl;
    for (; r + 3 * 64 < rows; r += 4 * 64) {
      const float4 a = p4[(int64_t)r * n4 + c4];
      const float4 b = p4[(int64_t)(r + 64) * n4 + c4];
      const float4 c = p4[(int64_t)(r + 128) * n4 + c4];
      const float4 e = p4[(int64_t)(r + 192) * n4 + c4];
      acc.x += a.x; acc.y += a.y; acc.z += a.z; acc.w += a.w;
      acc.x += b.x; acc.y += b.y; acc.z += b.z; acc.w += b.w;
      acc.x += c.x; acc.y += c.y; acc.z += c.z; acc.w += c.w;
      acc.x += e.x; acc.y += e.y; acc.z += e.z; acc.w += e.w;
    }
    for (; r < rows; r += 64) {
      const float4 a = p4[(int64_t)r * n4 + c4];
      acc.x += a.x; acc.y += a.y; acc.z += a.z; acc.w += a.w;
    }
  }
  // Both halves of a swap end up with (low lanes' value) + (high lanes'), in
  // that order, so the lanes that meet later hold identical bits.
  auto pair = [](float x, bool across32) {
    const uint32_t u = __float_as_uint(x);
    const auto r = across32 ? __builtin_amdgcn_permlane32_swap(u, u, false, false)
                            : __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  };
  acc = make_float4(pair(acc.x, true), pair(acc.y, true), pair(acc.z, true), pair(acc.w, true));
  acc = make_float4(pair(acc.x, false), pair(acc.y, false), pair(acc.z, false), pair(acc.w, false));
  const int wave = threadIdx.x >> 6;
  if (lane < 16) sh[wave][cl] = acc;
  __syncthreads();
  if (wave == 0 && lane < 16 && c4 < n4) {
    float4 t = sh[0][cl];
#pragma unroll
    for (int q = 1; q < 16; ++q) {
      const float4 o = sh[q][cl];
      t.x += o.x; t.y += o.y; t.z += o.z; t.w += o.w;
    }
    store_elem(dw, 4 * (int64_t)c4, t.x, wt);
    store_elem(dw, 4 * (int64_t)c4 + 1, t.y, wt);
    store_elem(dw, 4 * (int64_t)c4 + 2, t.z, wt);
    store_elem(dw, 4 * (int64_t)c4 + 3, t.w, wt);
  }
}

// ------------------------------------------------------------------ probes

__global__ void __launch_bounds__(256)
k_probe_read(const i32x4_t* __restrict__ src, int64_t n16, float* __restrict__ dst) {
  __shared__ int sh[256];
  const int64_t stride = (int64_t)gridDim.x * 256;
  int acc = 0;
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const i32x4_t a = __builtin_nontemporal_load(src + i);
    const i32x4_t b = __builtin_nontemporal_load(src + i + stride);
    const i32x4_t c = __builtin_nontemporal_load(src + i + 2 * stride);
    const i32x4_t e = __builtin_nontemporal_load(src + i + 3 * stride);
    acc ^= (a.x ^ a.y ^ a.z ^ a.w) ^ (b.x ^ b.y ^ b.z ^ b.w) ^ (c.x ^ c.y ^ c.z ^ c.w) ^
           (e.x ^ e.y ^ e.z ^ e.w);
  }
  for (; i < n16; i += stride) {
    const i32x4_t a = src[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  sh[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    int t = 0;
    for (int k = 0; k < 256; ++k) t ^= sh[k];
    dst[blockIdx.x] = (float)t;
  }
}

__global__ void __launch_bounds__(256) k_probe_write(i32x4_t* __restrict__ dst, int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  const i32x4_t z = {0x3f800000, 0x3f800000, 0x3f800000, 0x3f800000};
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride)
    __builtin_nontemporal_store(z, dst + i);
}

// Copy probe: each workgroup moves 16 KiB per step (four 16-byte loads per
// thread, all issued before the stores), streamed both ways like the
// operator's kernels; the buffer resources clip the last step to the buffer.
// On MI355X this reaches ~6.0 TB/s (read + write) on 1 GiB, against ~5.4 TB/s
// for a grid-stride loop with two loads in flight per thread.
__global__ void __launch_bounds__(256)
k_probe_copy(const char* __restrict__ src, char* __restrict__ dst, int64_t bytes) {
  constexpr int64_t kChunk = 256 * 16 * 4;
  for (int64_t base = (int64_t)blockIdx.x * kChunk; base < bytes;
       base += (int64_t)gridDim.x * kChunk) {
    const uint32_t len = (uint32_t)(bytes - base < kChunk ? bytes - base : kChunk);
    const auto r = make_rsrc(src + base, len);
    const auto w = make_rsrc(dst + base, len);
    i32x4_t x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = ld16_stream(r, (threadIdx.x + 256u * u) * 16u);
#pragma unroll
    for (int u = 0; u < 4; ++u) st16_stream(w, (threadIdx.x + 256u * u) * 16u, x[u]);
  }
}

// 9:1 mix probe: each workgroup step reads 36 KiB of one contiguous source
// stretch (nine 4 KiB sub-blocks, each load instruction of a wave 1 KiB
// contiguous, nine loads in flight per thread) and writes 4 KiB: output chunk
// c of the step is the sum of chunk c of the nine sub-blocks. The forward's
// bytes and read:write ratio without its 16 MiB row stride.
__global__ void __launch_bounds__(256)
k_probe_mix(const char* __restrict__ src, char* __restrict__ dst, int64_t out_bytes) {
  constexpr int64_t kOut = 256 * 16;  // output bytes per workgroup step
  for (int64_t base = (int64_t)blockIdx.x * kOut; base < out_bytes; base += (int64_t)gridDim.x * kOut) {
    const uint32_t len = (uint32_t)(out_bytes - base < kOut ? out_bytes - base : kOut);
    const auto r = make_rsrc(src + 9 * base, 9 * len);
    const auto w = make_rsrc(dst + base, len);
    i32x4_t x[9];
#pragma unroll
    for (int u = 0; u < 9; ++u) x[u] = ld16_stream(r, (u * 256u + threadIdx.x) * 16u);
    i32x4_t acc = x[0];
#pragma unroll
    for (int u = 1; u < 9; ++u) acc += x[u];
    st16_stream(w, threadIdx.x * 16u, acc);
  }
}

}  // namespace

hipError_t launch_fwd_generic(const FwdArgs& a, hipStream_t s) {
  const size_t lds = (size_t)(2 * a.n_src + 257) * sizeof(float);
  hipLaunchKernelGGL(k_fwd_generic, dim3((unsigned)a.n_tok), dim3(kBlock), lds, s, a.v, a.w, a.out,
                     a.stats, a.m_out, a.l_out, a.normalize, a.n_src, a.n_tok, a.d, a.v_dtype,
                     a.w_dtype, a.eps, 1.0f / (float)a.d);
  return hipGetLastError();
}

hipError_t launch_sol_generic(const FwdArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(k_sol_generic, dim3((unsigned)a.n_tok), dim3(kBlock), 0, s, a.v, a.out,
                     a.n_src, a.n_tok, a.d, a.v_dtype);
  return hipGetLastError();
}

hipError_t launch_bwd_generic(const BwdArgs& a, int grid, hipStream_t s) {
  const size_t lds = (size_t)(3 * a.n_src + 257) * sizeof(float);
  hipLaunchKernelGGL(k_bwd_generic, dim3(grid), dim3(kBlock), lds, s, a.v, a.w, a.g, a.gm, a.gl,
                     a.dv, a.partial, a.n_src, a.n_tok, a.d, a.v_dtype, a.w_dtype, a.eps,
                     1.0f / (float)a.d);
  return hipGetLastError();
}

hipError_t launch_bwd_batched_generic(const BwdBatchedArgs& a, int grid, hipStream_t s) {
  const size_t lds = (size_t)bwd_batched_generic_lds(a.n_src, a.n_q);
  hipLaunchKernelGGL(k_bwd_batched_generic, dim3(grid), dim3(kBlock), lds, s, a.v, a.q, a.g, a.dv,
                     a.partial, a.n_src, a.n_q, a.n_tok, a.d, a.dtype, a.eps, 1.0f / (float)a.d);
  return hipGetLastError();
}

hipError_t launch_dw_reduce(const float* partial, int rows, int d, void* dw, int w_dtype,
                            hipStream_t s) {
  if (d % 4 == 0 && ((uintptr_t)partial & 15) == 0) {
    hipLaunchKernelGGL(k_dw_reduce4, dim3((unsigned)((d / 4 + 15) / 16)), dim3(1024), 0, s, partial,
                       rows, d, dw, w_dtype);
  } else {
    hipLaunchKernelGGL(k_dw_reduce, dim3((unsigned)((d + 63) / 64)), dim3(1024), 0, s, partial,
                       rows, d, dw, w_dtype);
  }
  return hipGetLastError();
}

hipError_t launch_probe(int kind, const void* src, void* dst, int64_t bytes, int grid,
                        hipStream_t s) {
  const int64_t n16 = bytes / 16;
  if (kind == 0) {
    hipLaunchKernelGGL(k_probe_read, dim3(grid), dim3(256), 0, s, (const i32x4_t*)src, n16,
                       (float*)dst);
  } else if (kind == 1) {
    hipLaunchKernelGGL(k_probe_write, dim3(grid), dim3(256), 0, s, (i32x4_t*)dst, n16);
  } else if (kind == 2) {
    hipLaunchKernelGGL(k_probe_copy, dim3(grid), dim3(256), 0, s, (const char*)src, (char*)dst,
                       bytes);
  } else {
    hipLaunchKernelGGL(k_probe_mix, dim3(grid), dim3(256), 0, s, (const char*)src, (char*)dst,
                       bytes / 9);
  }
  return hipGetLastError();
}

}  // namespace sy
