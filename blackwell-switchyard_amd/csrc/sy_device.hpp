// Device-side building blocks shared by every switchyard kernel (gfx950 only).
//
// Data moves in 16-byte chunks: 8 bf16/fp16 values or 4 fp32 values, one
// buffer_load_dwordx4 per lane. Each lane owns fixed chunks of a row; 64 lanes
// of a wave read 1 KiB of contiguous row memory per instruction.
//
// All arithmetic is fp32. Sums of squares and query dot products of 16-bit
// data use v_dot2_f32_{bf16,f16} (two exact products, fp32 accumulate), which
// halves the VALU count of the reductions; fp32 data uses plain FMAs.
//
// Timings in the comments of these sources are MI355X measurements, bf16
// unless stated. Named shapes: "config 2" is N=9 sources, B=1, T=4096,
// D=2048 (the operator's forward and backward); "config 3" the same sources
// with 8 queries (the batched forward); "config 4" the N / T / D sweeps around
// config 2; "config 5" the 1.3B decoder training step.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sy {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));

// dtype tags. `code` matches sy_dtype in include/switchyard.h.
struct BF16 { using storage = uint16_t; static constexpr int code = 2; static constexpr int ce = 8; };
struct F16  { using storage = uint16_t; static constexpr int code = 1; static constexpr int ce = 8; };
struct F32  { using storage = float;    static constexpr int code = 0; static constexpr int ce = 4; };

// Where the N source rows of a token start (and, for dv, the N gradient rows).
// Row n of token t is at row_of(table, n) + t*D. Rows n < kTableRows come from
// p[n]; rows beyond are p[0] + n*stride_bytes, the stacked [N][n_tok][D]
// layout. A stacked caller fills p[n] = base + n*stride; a caller with one
// tensor per source fills p[0..N) directly and needs N <= kTableRows. The table
// travels in the kernel arguments, so the resident kernels (compile-time n)
// read each row pointer with one scalar load.
constexpr int kTableRows = 16;
struct RowTable {
  void* p[kTableRows];
  int64_t stride_bytes;
};

template <class S>
__host__ __device__ __forceinline__ S* row_of(const RowTable& t, int n) {
  return n < kTableRows ? static_cast<S*>(t.p[n])
                        : reinterpret_cast<S*>(static_cast<char*>(t.p[0]) + (int64_t)n * t.stride_bytes);
}

// Row n with the addressing mode fixed at compile time: LISTED reads p[n]
// (n < kTableRows), otherwise p[0] + n*stride_bytes. Kernels that are short of
// SGPRs use this: the stacked form keeps one pointer and a stride live, where
// per-row pointers would take two SGPRs per row.
template <bool LISTED, class S>
__device__ __forceinline__ S* row_at(const RowTable& t, int n) {
  if constexpr (LISTED) {
    return static_cast<S*>(t.p[n]);
  } else {
    return reinterpret_cast<S*>(static_cast<char*>(t.p[0]) + (int64_t)n * t.stride_bytes);
  }
}

// Threads per backward workgroup (token slots x waves per token), at least one
// token's waves. Two- and one-chunk tiles use SY_BWD_BLOCK (512 measured best on
// MI355X: 128 +9%, 256 equal), i.e. two waves per SIMD at <= 256 VGPRs. Four-chunk
// tiles use 256 threads: one wave per SIMD, so a wave may hold 512 registers
// (256 VGPRs + 256 AGPRs) -- the 144-register tile plus everything else, with
// no spills. The 32-row kernel (k_bwd_tall) runs 512 threads with one chunk a
// lane (two waves per SIMD: a 128-VGPR tile) and 256 with two; its 64-row
// tiles (one chunk a lane, 256 tile VGPRs) run 256. Build-time
// constants so that kernels and the host plan agree.
#ifndef SY_BWD_BLOCK
#define SY_BWD_BLOCK 512
#endif
constexpr int bwd_block_base(int vpl, int nr) {
  return nr > 16 ? (vpl == 1 && nr <= 32 ? 512 : 256) : vpl >= 4 ? 256 : SY_BWD_BLOCK;
}
constexpr int bwd_block(int w, int vpl, int nr = 0) {
  return bwd_block_base(vpl, nr) > 64 * w ? bwd_block_base(vpl, nr) : 64 * w;
}

// Buffer resource word 3 for gfx9-family raw buffers (32-bit dword format).
constexpr int kRsrcFlags = 0x00020000;

// A raw buffer over [p, p + bytes). Loads past `bytes` return 0 and stores
// past it are dropped, which gives free masking of partial rows.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kRsrcFlags);
}

// Cache policy of streamed traffic (v, grad_out in; out, dv out): every byte
// is touched once, so the loads carry the `nt` (non-temporal) hint by default.
// Operands every wave re-reads (w, queries) use the default policy.
#ifndef SY_STREAM_LOAD_AUX
#define SY_STREAM_LOAD_AUX 2
#endif
#ifndef SY_STREAM_STORE_AUX
#define SY_STREAM_STORE_AUX 2
#endif

__device__ __forceinline__ i32x4_t ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
__device__ __forceinline__ i32x4_t ld16_stream(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, SY_STREAM_LOAD_AUX);
}
__device__ __forceinline__ void st16(__amdgpu_buffer_rsrc_t r, uint32_t off, i32x4_t x) {
  __builtin_amdgcn_raw_buffer_store_b128(x, r, off, 0, 0);
}
__device__ __forceinline__ void st16_stream(__amdgpu_buffer_rsrc_t r, uint32_t off, i32x4_t x) {
  __builtin_amdgcn_raw_buffer_store_b128(x, r, off, 0, SY_STREAM_STORE_AUX);
}
// Policy of the dv stores that measured faster with the device-scope bit (sc1 = 16)
// next to nt: the operator backward's 16-bit 9-row tiles whose wave slice spans four
// chunks, and its 32- and 64-row tiles (k_bwd, k_bwd_tall); the other tiles and
// kernels measured slower with it and keep SY_STREAM_STORE_AUX.
#ifndef SY_DV_STORE_AUX
#define SY_DV_STORE_AUX 18
#endif
template <int AUX>
__device__ __forceinline__ void st16_aux(__amdgpu_buffer_rsrc_t r, uint32_t off, i32x4_t x) {
  __builtin_amdgcn_raw_buffer_store_b128(x, r, off, 0, AUX);
}

// ---------------------------------------------------------------- conversion

__device__ __forceinline__ float bf_lo(uint32_t x) { return __uint_as_float(x << 16); }
__device__ __forceinline__ float bf_hi(uint32_t x) { return __uint_as_float(x & 0xffff0000u); }

// Element e of a 16-byte chunk as fp32.
template <class T> __device__ __forceinline__ float elem(const i32x4_t& c, int e);
template <> __device__ __forceinline__ float elem<BF16>(const i32x4_t& c, int e) {
  const uint32_t x = (uint32_t)c[e >> 1];
  return (e & 1) ? bf_hi(x) : bf_lo(x);
}
template <> __device__ __forceinline__ float elem<F16>(const i32x4_t& c, int e) {
  const int word = c[e >> 1];  // copy first: bit_cast of a vector element reads lane 0
  const f16x2_t h = __builtin_bit_cast(f16x2_t, word);
  return (e & 1) ? (float)h.y : (float)h.x;
}
template <> __device__ __forceinline__ float elem<F32>(const i32x4_t& c, int e) {
  return __int_as_float(c[e]);
}

// Round fp32 values to the storage type (round-to-nearest-even) and pack.
template <class T> __device__ __forceinline__ i32x4_t pack(const float* f);
template <> __device__ __forceinline__ i32x4_t pack<BF16>(const float* f) {
  i32x4_t r;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const f32x2_t p = {f[2 * k], f[2 * k + 1]};
    r[k] = __builtin_bit_cast(int, __builtin_convertvector(p, bf16x2_t));
  }
  return r;
}
template <> __device__ __forceinline__ i32x4_t pack<F16>(const float* f) {
  i32x4_t r;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const f32x2_t p = {f[2 * k], f[2 * k + 1]};
    r[k] = __builtin_bit_cast(int, __builtin_convertvector(p, f16x2_t));
  }
  return r;
}
template <> __device__ __forceinline__ i32x4_t pack<F32>(const float* f) {
  i32x4_t r;
#pragma unroll
  for (int k = 0; k < 4; ++k) r[k] = __float_as_int(f[k]);
  return r;
}

// acc + sum_e a[e] * b[e] over one chunk.
template <class T> __device__ __forceinline__ float dot(const i32x4_t& a, const i32x4_t& b, float acc);
template <> __device__ __forceinline__ float dot<BF16>(const i32x4_t& a, const i32x4_t& b, float acc) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    // Copy the dwords out first: __builtin_bit_cast applied directly to an
    // ext_vector element reads element 0 whatever the index.
    const int ak = a[k], bk = b[k];
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, ak),
                                          __builtin_bit_cast(bf16x2_t, bk), acc, false);
  }
  return acc;
}
template <> __device__ __forceinline__ float dot<F16>(const i32x4_t& a, const i32x4_t& b, float acc) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int ak = a[k], bk = b[k];
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, ak), __builtin_bit_cast(f16x2_t, bk),
                                 acc, false);
  }
  return acc;
}
template <> __device__ __forceinline__ float dot<F32>(const i32x4_t& a, const i32x4_t& b, float acc) {
#pragma unroll
  for (int k = 0; k < 4; ++k) acc = fmaf(__int_as_float(a[k]), __int_as_float(b[k]), acc);
  return acc;
}

// Scalar element load/store for the generic (unaligned) path.
__device__ __forceinline__ float load_elem(const void* p, int64_t i, int dtype) {
  if (dtype == 2) return __uint_as_float((uint32_t)((const uint16_t*)p)[i] << 16);
  if (dtype == 1) return (float)((const _Float16*)p)[i];
  return ((const float*)p)[i];
}
__device__ __forceinline__ void store_elem(void* p, int64_t i, float x, int dtype) {
  if (dtype == 2) {
    ((__bf16*)p)[i] = (__bf16)x;
  } else if (dtype == 1) {
    ((_Float16*)p)[i] = (_Float16)x;
  } else {
    ((float*)p)[i] = x;
  }
}

// ---------------------------------------------------------------- reductions

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xf, false));
}

// Sum over the 64 lanes of a wave, returned as a wave-uniform value. Six DPP
// adds leave the total in lane 63 (quad swaps, half-row and row mirrors, then
// the two row broadcasts), and one readlane makes it uniform. The order of the
// adds is fixed, so every wave of a kernel rounds identically.
__device__ __forceinline__ float wave_sum(float x) {
  x += dpp<0xB1>(x);          // quad_perm [1,0,3,2]
  x += dpp<0x4E>(x);          // quad_perm [2,3,0,1]
  x += dpp<0x141>(x);         // row_half_mirror
  x += dpp<0x140>(x);         // row_mirror: every lane holds its row's sum
  x += dpp<0x142, 0xa>(x);    // row_bcast:15 into rows 1 and 3
  x += dpp<0x143, 0xc>(x);    // row_bcast:31 into rows 2 and 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}

// Sums of P per-lane values over the 64 lanes, transposed (P = 2, 4, ..., 32):
// lane l ends up with the total of v[tsum_row<P>(l)]. Each step halves the
// values a lane carries: gfx950's permlane32/permlane16 swaps pair the halves
// across lane bits 5 and 4, then DPP row rotation by 8, the half-row mirror and
// a quad permutation pair lanes across bits 3, 2 and 0, each taking the next
// lower bit of the value index; the lane bits left over are summed out by the
// same DPP steps without a split. So v[n] lands in the lanes l with
// n = b5..b2 of l for P = 16 (l >> 2), l >> 3 for P = 8, and for P = 32 in
// n = b0 + 2*b2 + 4*b3 + 8*b4 + 16*b5 -- 70 VALU instructions for 32 values
// where 32 separate six-step reductions take ~380, 36 for 16. tsum_lane<P>(n)
// is one lane that holds v[n]'s total. The order of the adds is fixed, so the
// result is deterministic; lanes that hold the same total hold the same bits
// within a quad, but may differ by rounding between quads for P <= 8.
template <int P>
__device__ __forceinline__ constexpr int tsum_lane(int n) {
  static_assert(P >= 2 && P <= 32 && (P & (P - 1)) == 0, "P is a power of two in [2, 32]");
  if constexpr (P == 32) return (n & 1) | ((n >> 1) << 2);
  return n << (P == 16 ? 2 : P == 8 ? 3 : P == 4 ? 4 : 5);
}
template <int P>
__device__ __forceinline__ int tsum_row(int lane) {
  if constexpr (P == 32) return (lane & 1) | ((lane >> 1) & ~1);
  return lane >> (P == 16 ? 2 : P == 8 ? 3 : P == 4 ? 4 : 5);
}
template <int P>
__device__ __forceinline__ float tsum(const float (&v)[P], int lane) {
  static_assert(P >= 2 && P <= 32 && (P & (P - 1)) == 0, "P is a power of two in [2, 32]");
  const bool b3 = (lane & 8) != 0, b2 = (lane & 4) != 0, b0 = (lane & 1) != 0;
  float a[P / 2];
#pragma unroll
  for (int i = 0; i < P / 2; ++i) {  // value i + (P/2)*b5
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[i + P / 2]),
                                                    false, false);
    a[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  if constexpr (P == 2) {
    // one value: halve across bit 4 with the swap on itself, then sum bits 3..0
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a[0]), __float_as_uint(a[0]),
                                                    false, false);
    float f = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    f += dpp<0x128>(f);  // row_ror:8
    f += dpp<0x141>(f);  // row_half_mirror
    f += dpp<0xB1>(f);
    return f + dpp<0x4E>(f);
  } else {
    float b[P / 4];
#pragma unroll
    for (int i = 0; i < P / 4; ++i) {  // value i + (P/4)*b4 + (P/2)*b5
      const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a[i]), __float_as_uint(a[i + P / 4]),
                                                      false, false);
      b[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    if constexpr (P == 4) {
      float f = b[0] + dpp<0x128>(b[0]);
      f += dpp<0x141>(f);
      f += dpp<0xB1>(f);
      return f + dpp<0x4E>(f);
    } else {
      float c[P / 8];
#pragma unroll
      for (int i = 0; i < P / 8; ++i)  // row_ror:8 pairs l with l ^ 8
        c[i] = (b3 ? b[i + P / 8] : b[i]) + dpp<0x128>(b3 ? b[i] : b[i + P / 8]);
      if constexpr (P == 8) {
        float f = c[0] + dpp<0x141>(c[0]);
        f += dpp<0xB1>(f);
        return f + dpp<0x4E>(f);
      } else {
        float e[P / 16];
#pragma unroll
        for (int i = 0; i < P / 16; ++i)  // row_half_mirror pairs l with 7 - l in each 8 lanes
          e[i] = (b2 ? c[i + P / 16] : c[i]) + dpp<0x141>(b2 ? c[i] : c[i + P / 16]);
        if constexpr (P == 16) {
          const float f = e[0] + dpp<0xB1>(e[0]);
          return f + dpp<0x4E>(f);
        } else {
          const float f = (b0 ? e[1] : e[0]) + dpp<0xB1>(b0 ? e[0] : e[1]);  // quad_perm [1,0,3,2]
          return f + dpp<0x4E>(f);                                          // quad_perm [2,3,0,1]
        }
      }
    }
  }
}
__device__ __forceinline__ int tsum32_row(int lane) { return tsum_row<32>(lane); }
__device__ __forceinline__ float tsum32(const float (&v)[32], int lane) { return tsum<32>(v, lane); }

// Smallest power of two >= x (x >= 1), for sizing a tsum.
__host__ __device__ constexpr int pow2_at_least(int x) { return x <= 1 ? 1 : 2 * pow2_at_least((x + 1) / 2); }

// Max over the 64 lanes, wave-uniform. Rows that a broadcast skips see -inf
// from the DPP `old` operand, which leaves the max unchanged.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_or_ninf(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp((int)0xff800000, __float_as_int(x), CTRL,
                                                    ROW_MASK, 0xf, false));
}
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp_or_ninf<0xB1>(x));
  x = fmaxf(x, dpp_or_ninf<0x4E>(x));
  x = fmaxf(x, dpp_or_ninf<0x141>(x));
  x = fmaxf(x, dpp_or_ninf<0x140>(x));
  x = fmaxf(x, dpp_or_ninf<0x142, 0xa>(x));
  x = fmaxf(x, dpp_or_ninf<0x143, 0xc>(x));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}

__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

}  // namespace sy
