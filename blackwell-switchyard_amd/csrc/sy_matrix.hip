// Batched forward on the matrix cores (bf16 / fp16 inputs).
//
// With S queries the batched operator does S dot products and S weighted sums
// per source row: 8 queries x 9 rows at D=2048 cost ~7000 VALU instructions a
// token in the register-tiled kernel, which makes it VALU-bound at half the
// HBM rate. Both products are small matrix products per token, so here they run
// on MFMA:
//   logits   L^T[n][s] = sum_d V[n][d] Q[s][d]   v_mfma_f32_16x16x32 (K = d)
//   output   O^T[d][s] = sum_n V[n][d] P[s][n]   v_mfma_f32_16x16x16 (K = n)
// with N <= 16 sources on one MFMA dimension and S <= 16 queries on the other.
// V and Q are exact in the 16-bit operands and every product accumulates in
// fp32. P (the softmax numerators, fp32) is split into a 16-bit high part and
// the 16-bit rounding of its remainder, two MFMAs per output block, so the
// weights carry ~17 significant bits and the output keeps fp32-level error
// before its single rounding.
//
// Work split: a workgroup of WV waves (4; 8 at D=4096) owns one token at a
// time (persistent over tokens); wave w owns the D/WV columns [w*D/WV,
// (w+1)*D/WV), at most 512, so a wave's registers are those of D=2048. Its slice of the
// queries stays in registers for the whole kernel (B operand of the logits),
// its slice of the token's rows goes to LDS, row-major, and is read twice: as
// 16-byte row chunks for the logits and through ds_read_b64_tr_b16 (a 4x4
// transpose of 16-bit elements within each 16-lane group) as the n-packed A
// operand of the output product. Each wave reads back only what it wrote, so V
// needs no barrier; the per-wave logit and sum-of-squares partials are summed
// through LDS once per token (one barrier, double-buffered). The next token's
// rows are loaded into registers while the current one is computed and
// written to LDS when it is done.
//
// Reference: the batched forward of src/switchyard/triton_op.py:378-501 (same
// math as S calls of the single-query operator, one read of v).
#include <algorithm>
#include <cstdlib>

#include "sy_launch.hpp"

namespace sy {

namespace {

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef int i32x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

constexpr int kMxWaves = 4;                               // waves per workgroup, one token
constexpr int kMxRows = (int)kMatrixMaxRows;              // MFMA M of the logits, K of the output
// LDS layouts (32 banks of 4 bytes):
//  * source rows: stride = D*2 + 16 bytes, so the 8 rows one 16-byte read
//    pass of the logits touches (same column, rows qi) fall in 8 different
//    4-bank groups;
//  * transposed reads: within each 64-column block, output MFMA a takes from
//    lane (row r = q/4, piece c = q%4) the 8 bytes at 16a + 8(c%2) + 64(c/2):
//    with the 16-byte row skew, the 16 lanes of a pass cover 16 distinct
//    2-bank pairs;
//  * output staging: SC columns per query row (256 with at most 8 queries,
//    else 128), stride SC*2 + 16 bytes, written 8 bytes a lane (2-way bank
//    conflicts), read back as contiguous 16-byte chunks so that each store
//    instruction writes SC*2-byte segments of 64*16/(SC*2) query rows.
constexpr int kMxPad = 16;  // source-row skew (bytes)

template <class T> struct Mx;
template <> struct Mx<BF16> {
  static __device__ __forceinline__ f32x4_t k32(const i32x4_t& a, const i32x4_t& b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4_t k16(const i32x2_t& a, const i32x2_t& b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4_t, a),
                                                     __builtin_bit_cast(bf16x4_t, b), c, 0, 0, 0);
  }
  // Round two values (x in the low half) and read the halves back as fp32.
  static __device__ __forceinline__ int pack2(float x, float y) {
    const f32x2_t p = {x, y};
    return __builtin_bit_cast(int, __builtin_convertvector(p, bf16x2_t));
  }
  static __device__ __forceinline__ float lo(int w) { return __uint_as_float((uint32_t)w << 16); }
  static __device__ __forceinline__ float hi(int w) {
    return __uint_as_float((uint32_t)w & 0xffff0000u);
  }
};
template <> struct Mx<F16> {
  static __device__ __forceinline__ f32x4_t k32(const i32x4_t& a, const i32x4_t& b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4_t k16(const i32x2_t& a, const i32x2_t& b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, a),
                                                 __builtin_bit_cast(f16x4_t, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ int pack2(float x, float y) {
    const f32x2_t p = {x, y};
    return __builtin_bit_cast(int, __builtin_convertvector(p, f16x2_t));
  }
  static __device__ __forceinline__ float lo(int w) {
    return (float)__builtin_bit_cast(f16x2_t, w).x;
  }
  static __device__ __forceinline__ float hi(int w) {
    return (float)__builtin_bit_cast(f16x2_t, w).y;
  }
};

// Orders this wave's LDS accesses across lanes: rows written by one lane are
// read by others in the same wave, with no workgroup barrier in between.
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// LDS: [n_src + 1][d * 2 + kMxPad] bytes of rows (the extra row is zero and
// stands in for rows n >= n_src), then the exchange buffers. KS = D / (32 WV)
// (32-column steps of a wave), NR >= n_src staged rows. Two tokens are in
// flight per workgroup while a third is computed; the loop is unrolled by two
// so that both staging sets keep compile-time register indices. The loads of a
// staged token are split around the logits of the current one (half before,
// half after the exchange barrier), which spreads them over the token.
//
// Every global load and store in the loop is issued unconditionally (missing
// rows load through a zero-size resource, masked lanes store past the end of
// theirs), so the number of memory operations between a prefetch and its use
// is a compile-time constant and the compiler waits for exactly the prefetch,
// not for everything in flight.
template <class T, int KS, int NR, int SQ, int TP, int WV = kMxWaves>
__global__ void __launch_bounds__(64 * WV * TP, 8 / (WV * TP))
k_batched_mx(const RowTable v, const uint16_t* __restrict__ q, uint16_t* __restrict__ out,
             float* __restrict__ m_out, float* __restrict__ l_out, int normalize, int n_src,
             int n_q, int64_t n_tok, float eps, float inv_d) {
  using M = Mx<T>;
  static_assert(WV * TP <= 8, "one workgroup of at most 8 waves per CU");
  constexpr int d = 32 * KS * WV;
  constexpr uint32_t rs = (uint32_t)d * 2u + kMxPad;  // LDS row stride (bytes)
  constexpr uint32_t row_bytes = (uint32_t)d * 2u;
  constexpr int cpr = 4 * KS;  // 16-byte chunks per row in a wave's slice (<= 64)
  constexpr uint32_t kDrop = 0x80000000u;  // store offset past every resource
  extern __shared__ __align__(16) char vs_all[];
  __shared__ __align__(16) float xl[2][TP][WV][64][4];  // logit partials, C layout
  __shared__ __align__(16) float xs[2][TP][WV][kMxRows];  // sum-of-squares partials
  // Output staging: [query][SC columns] per wave (the MFMA result layout
  // gives each lane 8 bytes of one query).
  // 256-column rounds halve the store count; the 16-row staging leaves no
  // registers for their wider operand window.
  constexpr int SC = SQ <= 8 && KS % 8 == 0 && NR <= 9 ? 256 : 128;  // columns per round
  static_assert((32 * KS) % SC == 0, "store rounds must tile the wave's columns");
  constexpr int kRow = SC * 2 + 16;                   // staging row stride (bytes)
  constexpr int kLpq = SC / 8;                        // lanes per query row
  constexpr int kQpi = 64 / kLpq;                     // query rows per store
  constexpr int kRounds = SQ / kQpi;
  __shared__ __align__(16) char ob[TP][WV][SQ * kRow];

  const int lane = threadIdx.x & 63;
  // TP tokens per workgroup: waves WV*h .. WV*h + WV-1 own token slot h (its
  // own LDS rows and buffers); the slots of a workgroup advance in step (one
  // barrier per token), so no co-resident slot runs ahead of another.
  // Both are the same in every lane of a wave; readfirstlane tells the
  // compiler so. Without it the slot's token index counts as per-lane, and
  // every buffer load and store built from it is wrapped in a waterfall loop
  // (readfirstlane, compare, exec mask, branch) that serialises the memory ops.
  const int half = TP > 1 ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x / (64 * WV))) : 0;
  const int w = __builtin_amdgcn_readfirstlane((int)((threadIdx.x >> 6) % WV));
  char* const vs = vs_all + (size_t)half * (size_t)(n_src + 1) * rs;
  const int qi = lane & 15;  // MFMA column: query (logits, output) / row (A of logits)
  const int g = lane >> 4;   // 16-lane group
  const int cb = w * 32 * KS;  // first column of this wave

  // Query slice, B operand of the logits: Q[s][cb + 32k + 8g .. +7], s = qi
  // (queries past n_q repeat the last one; their columns are never stored).
  i32x4_t qr[KS];
  {
    const int sq = qi < n_q ? qi : n_q - 1;
    const auto r = make_rsrc(q, (uint32_t)n_q * row_bytes);
#pragma unroll
    for (int k = 0; k < KS; ++k) qr[k] = ld16(r, (uint32_t)(sq * d + cb + 32 * k + 8 * g) * 2u);
  }
  // Zero row (index n_src), this wave's slice.
  if (lane < cpr) *(i32x4_t*)(vs + n_src * rs + (cb + 8 * lane) * 2) = i32x4_t{0, 0, 0, 0};

  // Persistent over groups of TP consecutive tokens; slot `half` takes token
  // (group * TP + half), which is past n_tok only in an odd last group (its
  // loads and stores are then dropped).
  const int64_t step = gridDim.x;
  const int64_t first = blockIdx.x;
  const int64_t n_groups = (n_tok + TP - 1) / TP;
  const int iters = first < n_groups ? (int)((n_groups - first + step - 1) / step) : 0;
  if (iters == 0) return;  // uniform over the workgroup
  auto tok_at = [&](int64_t k) { return (first + k * step) * TP + half; };

  // Staging: chunk `lane` of each row of this wave's slice of token t (rows
  // past n_src and tokens past n_tok load zeros through a zero-size resource).
  auto stage_rows = [&](i32x4_t (&st)[NR], int64_t t, int n0, int n1) {
    const bool tok_ok = t < n_tok;
    const int64_t tc = tok_ok ? t : n_tok - 1;
#pragma unroll
    for (int n = n0; n < n1; ++n) {
      const bool real = n < n_src && tok_ok;
      const auto r = make_rsrc(row_of<const uint16_t>(v, n < n_src ? n : 0) + tc * d,
                               real ? row_bytes : 0u);
      st[n] = ld16_stream(r, (uint32_t)(cb + 8 * lane) * 2u);
    }
  };
  auto stage = [&](i32x4_t (&st)[NR], int64_t t) { stage_rows(st, t, 0, NR); };
  constexpr int kLate = NR / 2;  // rows of the next token loaded after the logits
  auto commit = [&](const i32x4_t (&st)[NR]) {
    wave_lds_fence();
    if (lane < cpr) {
#pragma unroll
      for (int n = 0; n < NR; ++n)
        if (n < n_src) *(i32x4_t*)(vs + n * rs + (cb + 8 * lane) * 2) = st[n];
    }
    wave_lds_fence();
  };

  // Row this lane feeds to the logits (A: row qi) and to the output product
  // (A: the 4x4-transposed read supplies row 4g + qi/4); missing rows read the
  // zero row.
  const int ra = qi < n_src ? qi : n_src;
  const int rt = 4 * g + (qi >> 2) < n_src ? 4 * g + (qi >> 2) : n_src;
  const char* abase = vs + ra * rs + (cb + 8 * g) * 2;
  const char* tbase = vs + rt * rs + cb * 2 + 8 * (qi & 1) + 64 * ((qi >> 1) & 1);
  // Statistics: lanes 0..15 of wave 0 own query qi; others store out of range.
  const bool stat_lane = w == 0 && g == 0 && qi < n_q;
  const uint32_t stat_bytes = m_out != nullptr ? (uint32_t)((int64_t)n_q * n_tok * 4) : 0u;
  // Output rounds: lane l stores query 4r + l/16, 16-byte chunk l%16 of the
  // group; rows of a round are n_tok * d apart.
  const uint32_t q_stride = (uint32_t)(n_tok * d * 2);

  // One token whose rows are in LDS; k selects the exchange buffer.
  auto token = [&](int k, int64_t tok, auto&& mid) {
    // Logit and sum-of-squares partials over this wave's columns: row chunks
    // are read kAhead steps ahead of their MFMA, and even and odd steps
    // accumulate in separate chains.
    constexpr int kAhead = 4;
    f32x4_t acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
    float ss0 = 0.0f, ss1 = 0.0f;
    i32x4_t win[kAhead];
#pragma unroll
    for (int kk = 0; kk < kAhead && kk < KS; ++kk) win[kk] = *(const i32x4_t*)(abase + kk * 64);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const i32x4_t a = win[kk % kAhead];
      if (kk + kAhead < KS) win[kk % kAhead] = *(const i32x4_t*)(abase + (kk + kAhead) * 64);
      if (kk % 2 == 0) {
        ss0 = dot<T>(a, a, ss0);
        acc0 = M::k32(a, qr[kk], acc0);
      } else {
        ss1 = dot<T>(a, a, ss1);
        acc1 = M::k32(a, qr[kk], acc1);
      }
    }
    const f32x4_t acc = acc0 + acc1;
    float ss = ss0 + ss1;
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    const int xb = k & 1;
    *(f32x4_t*)&xl[xb][half][w][lane][0] = acc;
    if (lane < kMxRows) xs[xb][half][w][lane] = ss;
    __syncthreads();
    mid();
    // Lane (g, qi) now holds rows n = 4g + j of query column s = qi.
    f32x4_t pl4[WV], ps4[WV];
#pragma unroll
    for (int ww = 0; ww < WV; ++ww) {
      pl4[ww] = *(const f32x4_t*)&xl[xb][half][ww][lane][0];
      ps4[ww] = *(const f32x4_t*)&xs[xb][half][ww][4 * g];
    }
    f32x4_t lt = pl4[0], sq = ps4[0];
#pragma unroll
    for (int ww = 1; ww < WV; ++ww) {
      lt += pl4[ww];
      sq += ps4[ww];
    }

    // Softmax over the rows of each query column (4 rows a lane, 4 lanes).
    float lg[4], p[4];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      lg[j] = 4 * g + j < n_src ? lt[j] * rsqrtf(fmaf(sq[j], inv_d, eps)) : -INFINITY;
      mx = fmaxf(mx, lg[j]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    float ls = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      p[j] = 4 * g + j < n_src ? expf(lg[j] - mx) : 0.0f;
      ls += p[j];
    }
    ls += __shfl_xor(ls, 16);
    ls += __shfl_xor(ls, 32);

    // B operand of the output product: P^T[4g + j][qi], high and low parts.
    const int h01 = M::pack2(p[0], p[1]), h23 = M::pack2(p[2], p[3]);
    const i32x2_t ph = {h01, h23};
    const i32x2_t pl = {M::pack2(p[0] - M::lo(h01), p[1] - M::hi(h01)),
                        M::pack2(p[2] - M::lo(h23), p[3] - M::hi(h23))};

    // Output, 64 columns at a time (4 MFMA pairs, high and low weight parts).
    // Lane (g, qi) of MFMA a holds query qi at local columns
    // 8a + 4(g%2) + 32(g/2) + j, j < 4; it stages them (8 bytes) and every
    // SC columns the wave stores SC*2-byte row segments.
    const float inv_l = normalize ? 1.0f / ls : 1.0f;
    char* obw = ob[half][w];
    constexpr int kBlocks = KS / 2;            // 64-column blocks of this wave
    constexpr int kPerStage = SC / 64;         // blocks per store round
    auto tread = [&](int b, int a) {
      return __builtin_bit_cast(i32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                             (lds_s16x4_t*)(tbase + b * 128 + a * 16)));
    };
    const int ocol = 4 * (g & 1) + 32 * (g >> 1);  // lane's first local column
    i32x2_t tw[kPerStage][4];
#pragma unroll
    for (int j = 0; j < kPerStage; ++j)
#pragma unroll
      for (int a = 0; a < 4; ++a) tw[j][a] = tread(j, a);
#pragma unroll
    for (int b = 0; b < kBlocks; ++b) {
      if (b % kPerStage == 0) wave_lds_fence();
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        f32x4_t c = {0.0f, 0.0f, 0.0f, 0.0f};
        c = M::k16(tw[b % kPerStage][a], pl, c);
        c = M::k16(tw[b % kPerStage][a], ph, c);
        const i32x2_t o = {M::pack2(c[0] * inv_l, c[1] * inv_l),
                           M::pack2(c[2] * inv_l, c[3] * inv_l)};
        if (qi < SQ) *(i32x2_t*)(obw + qi * kRow + ((b % kPerStage) * 64 + 8 * a + ocol) * 2) = o;
      }
      if (b % kPerStage == kPerStage - 1) {
        // Next round's operands go out before the staging round trip.
#pragma unroll
        for (int j = 0; j < kPerStage; ++j)
          if (b + 1 + j < kBlocks)
#pragma unroll
            for (int a = 0; a < 4; ++a) tw[j][a] = tread(b + 1 + j, a);
        wave_lds_fence();
        const int col0 = cb + 64 * (b + 1 - kPerStage);  // first column of the round
        const int chunk = lane % kLpq;  // 16-byte chunk of a query's segment
        i32x4_t vals[kRounds];
#pragma unroll
        for (int rr = 0; rr < kRounds; ++rr)
          vals[rr] = *(const i32x4_t*)(obw + (kQpi * rr + lane / kLpq) * kRow + chunk * 16);
#pragma unroll
        for (int rr = 0; rr < kRounds; ++rr) {
          const int live = tok < n_tok ? n_q - kQpi * rr : 0;  // queries of this round
          const uint32_t bytes =
              live <= 0 ? 0u
                        : (uint32_t)(live > kQpi ? kQpi - 1 : live - 1) * q_stride + row_bytes;
          const auto orr =
              make_rsrc(out + ((int64_t)(live > 0 ? kQpi * rr : 0) * n_tok + tok) * d, bytes);
          const bool ok = kQpi * rr + lane / kLpq < n_q;
          st16_stream(orr,
                      ok ? (uint32_t)(lane / kLpq) * q_stride + (uint32_t)(col0 + 8 * chunk) * 2u
                         : kDrop,
                      vals[rr]);
        }
      }
    }
    const auto mr = make_rsrc(m_out, stat_bytes);
    const auto lr = make_rsrc(l_out, stat_bytes);
    const uint32_t so =
        stat_lane && tok < n_tok ? (uint32_t)(((int64_t)qi * n_tok + tok) * 4) : kDrop;
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(mx), mr, so, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(ls), lr, so, 0, 0);
  };

  // Stores one token issues (output rounds, then m and l).
  constexpr int kTokenStores = (32 * KS / SC) * kRounds + 2;
  // Two staged tokens in flight, except where 16 rows x 2048 columns would
  // not leave the registers for two staging sets.
  constexpr bool kTwoDeep = NR <= 9 || KS < 16;
  i32x4_t sa[NR], sb[kTwoDeep ? NR : 1];
  stage(sa, tok_at(0));
  // Queries and the first token have landed before the loop: the compiler
  // then knows no register of theirs is pending inside it.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  commit(sa);
  if constexpr (kTwoDeep) {
    stage(sb, tok_at(1));
    // As many (dropped) stores as a token issues: entering the loop, the
    // loads of sb are then followed by the same number of memory operations
    // as on every later pass, so the compiler's wait before committing sb
    // counts exactly those loads instead of also draining the previous
    // token's stores. The scheduling barriers keep the stores after the loads.
    __builtin_amdgcn_sched_barrier(0);
    {
      const auto none = make_rsrc(out, 0u);
#pragma unroll
      for (int i = 0; i < kTokenStores; ++i) st16_stream(none, 16u * i, i32x4_t{0, 0, 0, 0});
    }
    __builtin_amdgcn_sched_barrier(0);
    for (int k = 0; k < iters; k += 2) {
      // Token k is in LDS, token k+1 in flight in sb.
      stage_rows(sa, tok_at(k + 2), 0, NR - kLate);
      token(k, tok_at(k), [&] { stage_rows(sa, tok_at(k + 2), NR - kLate, NR); });
      if (k + 1 >= iters) break;
      commit(sb);
      stage_rows(sb, tok_at(k + 3), 0, NR - kLate);
      token(k + 1, tok_at(k + 1), [&] { stage_rows(sb, tok_at(k + 3), NR - kLate, NR); });
      if (k + 2 < iters) commit(sa);
    }
  } else {
    for (int k = 0; k < iters; ++k) {
      stage(sa, tok_at(k + 1));
      token(k, tok_at(k), [] {});
      if (k + 1 < iters) commit(sa);
    }
  }
}

// ------------------------------------------------------------ batched backward
//
// Gradient of the batched forward for grad_out g [S][n_tok][D], S <= 8. Per
// token, with GQ = [g_0 .. g_7 ; q_0 .. q_7] (16 rows, zero past n_q):
//   D[n][c]  = sum_d V[n][d] GQ[c][d]         v_mfma_f32_16x16x32 (K = d)
// gives G_sn = <g_s, v_n> (c = s) and the logit dots <q_s, v_n> (c = 8 + s)
// in one product. Then per (s, n), like the single-query operator,
//   dlogit = alpha (G - sum_k alpha_k G_k),  da = dlogit r_n,
//   c_n    = -sum_s dlogit logit r_n^2 / D,
// and two more products of the token's LDS tile with one A operand,
// A[d][k] = [GQ ; V][k][d] (K = 32: 16 GQ rows, 16 source rows):
//   dV^T[d][n]  = sum_k A[d][k] [alpha ; da ; diag(c)][k][n]
//   dQ^T[d][s] += sum_k A[d][k] [0 ; da^T][k][s]            (over the tokens)
// both v_mfma_f32_16x16x32 (on gfx950 the K = 16 form costs the same issue
// time for half the work). A comes from two 4x4-transposed LDS reads. The fp32
// coefficients are split into high and low 16-bit parts (two MFMAs each), so
// dv keeps fp32-level error before its single rounding and dq accumulates in
// fp32 registers for the whole kernel (one partial row per query and
// workgroup, reduced afterwards in a fixed order).
//
// Layout of the D[n][c] result: lane (g, i) holds rows n = 4g + j of column
// i, so lanes i and i ^ 8 hold G and the logit dot of query i & 7 (one DPP
// row rotation swaps them); the softmax over n runs over j and the four
// 16-lane groups. The B operands need other lane layouts (k = 8g + j, column
// i), which go through two small LDS tables per wave.
//
// Work split as in the forward: W waves per workgroup (4, or 8 = two per
// SIMD), one token at a time, wave w owns D/W columns and reads back only the
// LDS rows it wrote; the logit partials cross the waves through LDS once per
// token. The v and g rows of the token after next are loaded into registers
// a few rows per output block of the current one (a burst of loads would
// stall the wave at issue), and written to LDS when the next one is done; a
// load covers 64 / (chunks of a wave's slice) rows. dv rows leave through LDS
// staging as SC-column row segments, all rows of a store from one buffer
// resource (offsets below 2^31, checked by the host). Every global load and
// store in the loop is unconditional (see k_batched_mx), so the waits are
// exact. The cross-lane sums of the softmax use the gfx950 row swaps
// (v_permlane16/32_swap) instead of LDS-routed shuffles.
//
// Reference: the batched forward is src/switchyard/triton_op.py:378-501; it
// has no backward (the single-query derivation is at :205-214).
// Pair reductions over lanes (l, l ^ 16) and (l, l ^ 32) with the gfx950 row
// swaps (VALU, no LDS round trip). Each swap leaves the even-row (low-half)
// value in one result and the odd-row (high-half) value in the other, so every
// lane combines the same two operands in the same order.
__device__ __forceinline__ f32x2_t swap16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return f32x2_t{__uint_as_float(r[0]), __uint_as_float(r[1])};
}
__device__ __forceinline__ f32x2_t swap32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return f32x2_t{__uint_as_float(r[0]), __uint_as_float(r[1])};
}
__device__ __forceinline__ float sum64(float x) {  // over the four 16-lane groups
  f32x2_t p = swap16(x);
  p = swap32(p[0] + p[1]);
  return p[0] + p[1];
}
__device__ __forceinline__ float max64(float x) {
  f32x2_t p = swap16(x);
  p = swap32(fmaxf(p[0], p[1]));
  return fmaxf(p[0], p[1]);
}

template <class T, int KS, int NR, int W>
__global__ void __launch_bounds__(64 * W, 1)
k_bwd_batched_mx(const RowTable v, const uint16_t* __restrict__ q, const uint16_t* __restrict__ g,
                 const RowTable dv, float* __restrict__ partial, int n_src, int n_q,
                 int64_t n_tok, float eps, float inv_d) {
  using M = Mx<T>;
  constexpr int d = 32 * KS * W;
  constexpr uint32_t rs = (uint32_t)d * 2u + kMxPad;
  constexpr uint32_t row_bytes = (uint32_t)d * 2u;
  constexpr int cpr = 4 * KS;  // 16-byte chunks of a row in a wave's slice
  constexpr uint32_t kDrop = 0x80000000u;
  constexpr int SQ = (int)kBwdMatrixMaxQ;
  static_assert(SQ == 8, "g and q rows take 8 of the 16 MFMA columns each");
  // Staging loads cover kRpl rows each (lane / cpr picks the row) when a
  // wave's slice is narrower than 64 chunks.
  constexpr int kRpl = cpr <= 32 && 64 % cpr == 0 ? 64 / cpr : 1;
  constexpr int kVl = (NR + kRpl - 1) / kRpl;  // source-row loads
  constexpr int kGl = (SQ + kRpl - 1) / kRpl;  // g-row loads
  // dv staging: SC columns per round, stride SC*2 + 16 bytes; a store covers
  // kRpi rows with kLpr lanes each.
  constexpr int SC = bwd_matrix_store_cols(NR, KS, W);
  static_assert((32 * KS) % SC == 0, "store rounds must tile the wave's columns");
  constexpr int kRow = SC * 2 + 16;
  constexpr int kLpr = SC / 8;
  constexpr int kRpi = 64 / kLpr;
  constexpr int kRounds = (NR + kRpi - 1) / kRpi;
  constexpr int kTs = 20;  // coefficient table row stride (floats): [n][k], k = 16 is c_n
  extern __shared__ __align__(16) char lds[];
  char* const gq = lds;            // 16 rows: g of the token, then the queries
  char* const vs = lds + 16 * rs;  // n_src source rows, then a zero row
  __shared__ __align__(16) float xl[2][W][64][4];
  __shared__ __align__(16) float xs[2][W][kMxRows];
  __shared__ __align__(16) float tt[W][16 * kTs];
  __shared__ __align__(16) float ut[W][8 * kTs];
  // Staged rows: the store rounds' rows plus row NR, where lanes of rows
  // past n_src write (unconditional LDS writes, no branches).
  constexpr int kObRows = kRounds * kRpi > NR ? kRounds * kRpi : NR + 1;
  __shared__ __align__(16) char ob[W][kObRows * kRow];

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int qi = lane & 15;
  const int grp = lane >> 4;
  const int cb = w * 32 * KS;
  const uint32_t coff = lane < cpr ? (uint32_t)(cb + 8 * lane) * 2u : kDrop;
  const int loff = (cb + 8 * lane) * 2;  // this lane's chunk (bytes into a row)
  // Staging: this lane's row within a load and its chunk.
  const int lr = kRpl > 1 ? lane / cpr : 0;
  const int lc = kRpl > 1 ? lane % cpr : lane;
  const bool lane_ok = kRpl > 1 || lane < cpr;
  const int soff = (cb + 8 * lc) * 2;
  const uint32_t v_stride = (uint32_t)v.stride_bytes;
  const uint32_t g_stride = (uint32_t)(n_tok * d * 2);

  // Queries (GQ rows 8..15, zero past n_q) and the zero source row; called
  // after the first token's loads are issued, so both arrive in one wait.
  auto queries = [&]() {
    i32x4_t qv[SQ];
#pragma unroll
    for (int s = 0; s < SQ; ++s)
      qv[s] = ld16(make_rsrc(q + (int64_t)(s < n_q ? s : 0) * d, s < n_q ? row_bytes : 0u), coff);
    if (lane < cpr) {
#pragma unroll
      for (int s = 0; s < SQ; ++s) *(i32x4_t*)(gq + (8 + s) * rs + loff) = qv[s];
      *(i32x4_t*)(vs + n_src * rs + loff) = i32x4_t{0, 0, 0, 0};
    }
  };

  f32x4_t qacc[KS / 2][4];
#pragma unroll
  for (int b = 0; b < KS / 2; ++b)
#pragma unroll
    for (int a = 0; a < 4; ++a) qacc[b][a] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  const int64_t step = gridDim.x;
  const int64_t first = blockIdx.x;
  const int iters = first < n_tok ? (int)((n_tok - first + step - 1) / step) : 0;

  // Staging load r of token t: source rows [r*kRpl, +kRpl) (r < kVl), else
  // g rows [(r - kVl)*kRpl, +kRpl), one buffer resource per load (tokens past
  // n_tok and missing rows load zeros without memory traffic).
  constexpr int kLoads = kVl + kGl;
  auto issue = [&](i32x4_t (&sv)[kVl], i32x4_t (&sg)[kGl], int64_t t, int r) {
    const bool tok_ok = t < n_tok;
    const int64_t tc = tok_ok ? t : n_tok - 1;
    if (r < kVl) {
      const int n0 = r * kRpl, n = n0 + lr;
      const int last = (n_src < n0 + kRpl ? n_src : n0 + kRpl) - 1;  // last real row
      const uint32_t bytes = tok_ok && n0 < n_src ? (uint32_t)(last - n0) * v_stride + row_bytes : 0u;
      const auto rr = make_rsrc(row_at<false, const uint16_t>(v, n0 < n_src ? n0 : 0) + tc * d, bytes);
      sv[r] = ld16_stream(rr, lane_ok && n < n_src ? (uint32_t)lr * v_stride + (uint32_t)soff : kDrop);
    } else {
      const int s0 = (r - kVl) * kRpl, s = s0 + lr;
      const int last = (n_q < s0 + kRpl ? n_q : s0 + kRpl) - 1;
      const uint32_t bytes = tok_ok && s0 < n_q ? (uint32_t)(last - s0) * g_stride + row_bytes : 0u;
      const auto rr = make_rsrc(g + ((int64_t)(s0 < n_q ? s0 : 0) * n_tok + tc) * d, bytes);
      sg[r - kVl] = ld16_stream(rr, lane_ok && s < n_q ? (uint32_t)lr * g_stride + (uint32_t)soff : kDrop);
    }
  };
  auto stage = [&](i32x4_t (&sv)[kVl], i32x4_t (&sg)[kGl], int64_t t) {
#pragma unroll
    for (int r = 0; r < kLoads; ++r) issue(sv, sg, t, r);
  };
  // Rows past n_src hold zeros (dropped loads) and go to the zero row.
  auto commit = [&](const i32x4_t (&sv)[kVl], const i32x4_t (&sg)[kGl]) {
    wave_lds_fence();
    if (lane_ok) {
#pragma unroll
      for (int r = 0; r < kVl; ++r) {
        const int n = r * kRpl + lr;
        *(i32x4_t*)(vs + (n < n_src ? n : n_src) * rs + soff) = sv[r];
      }
#pragma unroll
      for (int r = 0; r < kGl; ++r) *(i32x4_t*)(gq + (r * kRpl + lr) * rs + soff) = sg[r];
    }
    wave_lds_fence();
  };

  // Logits A operand: source row qi (zero row past n_src); B: GQ row qi.
  const int ra = qi < n_src ? qi : n_src;
  const char* const abase = vs + ra * rs + (cb + 8 * grp) * 2;
  const char* const bbase = gq + qi * rs + (cb + 8 * grp) * 2;
  // Transposed reads (A of both output products, k = 8*grp + j): lane
  // (grp, 4j + t) reads row k = 8*grp + j (first read) and 8*grp + 4 + j
  // (second read), k < 16 from GQ, else V row k - 16 (the zero row past
  // n_src), at the forward's bank-conflict-free column pieces t.
  const uint32_t toff = (uint32_t)cb * 2u + 8u * (qi & 1) + 64u * ((qi >> 1) & 1);
  auto trow = [&](int k) {
    return k < 16 ? gq + k * rs : vs + (k - 16 < n_src ? k - 16 : n_src) * rs;
  };
  const char* const ta1 = trow(8 * grp + (qi >> 2)) + toff;
  const char* const ta2 = trow(8 * grp + 4 + (qi >> 2)) + toff;
  auto tread = [&](const char* base, int b, int a) {
    return __builtin_bit_cast(i32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                           (lds_s16x4_t*)(base + b * 128 + a * 16)));
  };
  // Output layout of MFMA a of a 64-column block: lane (grp, qi) holds row n = qi
  // (dv) or query s = qi (dq) at local columns 8a + ocol + j, j < 4.
  const int ocol = 4 * (grp & 1) + 32 * (grp >> 1);
  const int wrow = qi < n_src ? qi : NR;  // staging row of this lane's dv values
  float* const tw = tt[w];
  float* const tu = ut[w];
  char* const obw = ob[w];
  const uint32_t dv_stride = (uint32_t)dv.stride_bytes;
  const uint32_t dv_bytes = (uint32_t)(n_src - 1) * dv_stride + row_bytes;
  const bool gl = qi < 8;  // column qi is G (else the logit dot of query qi - 8)

  // Token tok (exchange buffer k & 1); its output loop also issues the loads
  // of token stok into (sv, sg), a few per block, so that no wave stalls on a
  // burst of loads.
  auto token = [&](int k, int64_t tok, i32x4_t (&sv)[kVl], i32x4_t (&sg)[kGl], int64_t stok) {
    // 1. D[n][c] partials over this wave's columns, and the sums of squares.
    constexpr int kAhead = 4;
    f32x4_t acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
    float ss0 = 0.0f, ss1 = 0.0f;
    i32x4_t wa[kAhead], wb[kAhead];
#pragma unroll
    for (int kk = 0; kk < kAhead && kk < KS; ++kk) {
      wa[kk] = *(const i32x4_t*)(abase + kk * 64);
      wb[kk] = *(const i32x4_t*)(bbase + kk * 64);
    }
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const i32x4_t a = wa[kk % kAhead], b = wb[kk % kAhead];
      if (kk + kAhead < KS) {
        wa[kk % kAhead] = *(const i32x4_t*)(abase + (kk + kAhead) * 64);
        wb[kk % kAhead] = *(const i32x4_t*)(bbase + (kk + kAhead) * 64);
      }
      if (kk % 2 == 0) {
        ss0 = dot<T>(a, a, ss0);
        acc0 = M::k32(a, b, acc0);
      } else {
        ss1 = dot<T>(a, a, ss1);
        acc1 = M::k32(a, b, acc1);
      }
      // Keep the read window: at one wave per SIMD the scheduler would
      // otherwise hoist every read of the token.
      __builtin_amdgcn_sched_barrier(0);
    }
    const f32x4_t acc = acc0 + acc1;
    float ss = ss0 + ss1;
    ss = sum64(ss);
    const int xb = k & 1;
    *(f32x4_t*)&xl[xb][w][lane][0] = acc;
    if (lane < kMxRows) xs[xb][w][lane] = ss;
    __syncthreads();
    f32x4_t lt = *(const f32x4_t*)&xl[xb][0][lane][0];
    f32x4_t sq = *(const f32x4_t*)&xs[xb][0][4 * grp];
#pragma unroll
    for (int ww = 1; ww < W; ++ww) {
      lt += *(const f32x4_t*)&xl[xb][ww][lane][0];
      sq += *(const f32x4_t*)&xs[xb][ww][4 * grp];
    }

    // 2. Softmax of query qi & 7 over rows n = 4*grp + j (j, then the groups).
    float G[4], lgr[4], lg[4], r[4];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float o = dpp<0x128>(lt[j]);  // row_ror:8: the lane qi ^ 8 value
      G[j] = gl ? lt[j] : o;
      r[j] = rsqrtf(fmaf(sq[j], inv_d, eps));
      lgr[j] = (gl ? o : lt[j]) * r[j];
      lg[j] = 4 * grp + j < n_src ? lgr[j] : -INFINITY;
      mx = fmaxf(mx, lg[j]);
    }
    mx = max64(mx);
    float p[4];
    int top = 64;  // first row at the maximum
#pragma unroll
    for (int j = 3; j >= 0; --j) {
      const bool real = 4 * grp + j < n_src;
      p[j] = real ? expf(lg[j] - mx) : 0.0f;
      if (real && lg[j] == mx) top = 4 * grp + j;
    }
    float ls = (p[0] + p[1]) + (p[2] + p[3]);
    ls = sum64(ls);
    // (row indices below 64 are exact in fp32)
    top = (int)-max64(-(float)top);
    // G of the top row (lane (top / 4, qi), element top % 4): the dots are
    // taken relative to it, as in the single-query backward.
    const int tj = top & 3;
    const float gsel = tj == 0 ? G[0] : tj == 1 ? G[1] : tj == 2 ? G[2] : G[3];
    const float gref = sum64(grp == ((top >> 2) & 3) ? gsel : 0.0f);
    const float inv_l = 1.0f / ls;
    float al[4], dg[4];
    float sdev = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      al[j] = p[j] * inv_l;
      dg[j] = G[j] - gref;
      sdev = fmaf(al[j], dg[j], sdev);
    }
    sdev = sum64(sdev);
    float da[4], cn4[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float dl = al[j] * (dg[j] - sdev);
      da[j] = dl * r[j];
      // c_n: sum over the 8 queries, lanes qi & 7 (both halves of a row agree)
      float c = -dl * lgr[j] * (r[j] * r[j] * inv_d);
      c += dpp<0xB1>(c);   // quad_perm [1,0,3,2]
      c += dpp<0x4E>(c);   // quad_perm [2,3,0,1]
      c += dpp<0x141>(c);  // row_half_mirror
      cn4[j] = c;
    }

    // 3. B operands of the output products. The A operand of both is
    //    A[d][k] (k < 32) = GQ[k][d] for k < 16, V[k - 16][d] for k >= 16;
    //    lane (grp, i) supplies B[k = 8*grp + j][column i], j < 8.
    //    dv:  B[k][n] = alpha[k][n], da[k - 8][n], then diag(c) (c_n v_n);
    //    dq:  B[k][s] = 0 for the GQ rows, da[s][k - 16] for the V rows.
    //    Tables (this wave's LDS): tw[n][k] = alpha[k][n] (k < 8),
    //    da[k - 8][n] (k < 16), c_n (k = 16); tu[s][n] = da[s][n].
    wave_lds_fence();
#pragma unroll
    for (int j = 0; j < 4; ++j) tw[(4 * grp + j) * kTs + qi] = gl ? al[j] : da[j];
    if (qi == 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j) tw[(4 * grp + j) * kTs + 16] = cn4[j];
    }
    *(f32x4_t*)&tu[(qi & 7) * kTs + 4 * grp] = f32x4_t{da[0], da[1], da[2], da[3]};
    wave_lds_fence();
    const float cn = tw[qi * kTs + 16];
    const f32x4_t w0 = *(const f32x4_t*)&tw[qi * kTs + 8 * (grp & 1)];
    const f32x4_t w1 = *(const f32x4_t*)&tw[qi * kTs + 8 * (grp & 1) + 4];
    const f32x4_t u0 = *(const f32x4_t*)&tu[(qi & 7) * kTs + 8 * (grp & 1)];
    const f32x4_t u1 = *(const f32x4_t*)&tu[(qi & 7) * kTs + 8 * (grp & 1) + 4];
    float bv[8], bq[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float wv = j < 4 ? w0[j] : w1[j - 4];
      const float uv = j < 4 ? u0[j] : u1[j - 4];
      bv[j] = grp < 2 ? wv : (8 * (grp & 1) + j == qi ? cn : 0.0f);
      bq[j] = grp >= 2 && gl ? uv : 0.0f;
    }
    i32x4_t bvh, bvl, bqh, bql;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      bvh[j] = M::pack2(bv[2 * j], bv[2 * j + 1]);
      bvl[j] = M::pack2(bv[2 * j] - M::lo(bvh[j]), bv[2 * j + 1] - M::hi(bvh[j]));
      bqh[j] = M::pack2(bq[2 * j], bq[2 * j + 1]);
      bql[j] = M::pack2(bq[2 * j] - M::lo(bqh[j]), bq[2 * j + 1] - M::hi(bqh[j]));
    }

    // 4. dv (staged, SC columns per store round) and dq, 64 columns a block.
    constexpr int kBlocks = KS / 2;
    constexpr int kPerStage = SC / 64;
    const auto dr = make_rsrc(row_at<false, uint16_t>(dv, 0) + tok * d, dv_bytes);
    // A operands of a block (k = 8*grp + j from two transposed reads), read
    // one block ahead of their MFMAs; scheduling barriers keep that window.
    i32x4_t aa[2][4];
    auto operands = [&](int b, int u) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const i32x2_t lo = tread(ta1, b, a), hi = tread(ta2, b, a);
        aa[u][a] = i32x4_t{lo[0], lo[1], hi[0], hi[1]};
      }
    };
    operands(0, 0);
#pragma unroll
    for (int b = 0; b < kBlocks; ++b) {
      const int u = b & 1;
      if (b % kPerStage == 0) wave_lds_fence();
      if (b + 1 < kBlocks) operands(b + 1, u ^ 1);
#pragma unroll
      for (int r = b * kLoads / kBlocks; r < (b + 1) * kLoads / kBlocks; ++r) issue(sv, sg, stok, r);
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        f32x4_t c = {0.0f, 0.0f, 0.0f, 0.0f};
        c = M::k32(aa[u][a], bvl, c);
        c = M::k32(aa[u][a], bvh, c);
        qacc[b][a] = M::k32(aa[u][a], bql, qacc[b][a]);
        qacc[b][a] = M::k32(aa[u][a], bqh, qacc[b][a]);
        const i32x2_t o = {M::pack2(c[0], c[1]), M::pack2(c[2], c[3])};
        *(i32x2_t*)(obw + wrow * kRow + ((b % kPerStage) * 64 + 8 * a + ocol) * 2) = o;
      }
      if (b % kPerStage == kPerStage - 1) {
        wave_lds_fence();
        const int col0 = cb + 64 * (b + 1 - kPerStage);
        const int chunk = lane % kLpr;
        i32x4_t vals[kRounds];
#pragma unroll
        for (int rr = 0; rr < kRounds; ++rr)
          vals[rr] = *(const i32x4_t*)(obw + (kRpi * rr + lane / kLpr) * kRow + chunk * 16);
#pragma unroll
        for (int rr = 0; rr < kRounds; ++rr) {
          const int row = kRpi * rr + lane / kLpr;
          st16_stream(dr,
                      row < n_src ? (uint32_t)row * dv_stride + (uint32_t)(col0 + 8 * chunk) * 2u
                                  : kDrop,
                      vals[rr]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Two staged tokens in flight while one is computed (one in flight measured
  // the same at config 3: 115.4 vs 116.7 us).
  if (iters > 0) {
    // Stores one token issues.
    constexpr int kTokenStores = (32 * KS / SC) * kRounds;
    i32x4_t sva[kVl], sga[kGl], svb[kVl], sgb[kGl];
    stage(sva, sga, first);
    queries();  // waits for the queries and the first token
    commit(sva, sga);
    stage(svb, sgb, first + step);
    // Dropped stores, so that the loads of the second set are followed by as
    // many memory operations as on every later pass (exact waits).
    __builtin_amdgcn_sched_barrier(0);
    {
      const auto none = make_rsrc(partial, 0u);
#pragma unroll
      for (int i = 0; i < kTokenStores; ++i) st16_stream(none, 16u * i, i32x4_t{0, 0, 0, 0});
    }
    __builtin_amdgcn_sched_barrier(0);
    // Pairs of tokens, then the odd one (a break inside the pair would make
    // the compiler copy the dq accumulators between register files).
    int k = 0;
    for (; k + 1 < iters; k += 2) {
      const int64_t tok = first + (int64_t)k * step;
      token(k, tok, sva, sga, tok + 2 * step);
      commit(svb, sgb);
      token(k + 1, tok + step, svb, sgb, tok + 3 * step);
      if (k + 2 < iters) commit(sva, sga);
    }
    // The odd last token stages nothing (its loads are past n_tok: dropped).
    if (k < iters) token(k, first + (int64_t)k * step, sva, sga, n_tok);
  }

  // dq partial row of each query: partial[blockIdx][s][:].
  if (qi < n_q) {
    float* const pr = partial + ((int64_t)blockIdx.x * n_q + qi) * d + cb + ocol;
#pragma unroll
    for (int b = 0; b < KS / 2; ++b)
#pragma unroll
      for (int a = 0; a < 4; ++a) *(f32x4_t*)(pr + b * 64 + 8 * a) = qacc[b][a];
  }
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

template <class T, int KS, int NR, int SQ, int TP, int WV = kMxWaves>
hipError_t launch_mx(const BatchedArgs& a, hipStream_t s, KernelRes* info) {
  const size_t lds = (size_t)TP * (size_t)(a.n_src + 1) * ((size_t)a.d * 2 + kMxPad);
  auto* kern = k_batched_mx<T, KS, NR, SQ, TP, WV>;
  KernelRes r{0, 0, 1, 0};
  // The attributes of an instantiation do not change: query them once.
  static hipFuncAttributes fa;
  static const hipError_t fa_err =
      hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(kern));
  hipError_t e = fa_err;
  if (e != hipSuccess) return e;
  r.vgprs = fa.numRegs;
  r.lds = (int)(fa.sharedSizeBytes + lds);
  if (r.lds > 160 * 1024) return hipErrorInvalidConfiguration;
  const int alloc = std::max(8, ((fa.numRegs + 7) / 8) * 8);
  const int by_waves = std::max(1, std::min(8, 512 / alloc) / (WV * TP / 4));  // per SIMD
  r.blocks_per_cu = std::max(1, std::min(by_waves, (160 * 1024) / std::max(1, r.lds)));
  int cus = 0;
  if (cu_count(&cus) != hipSuccess || cus < 1) cus = 1;
  r.grid = (int)std::max<int64_t>(
      1, std::min<int64_t>((int64_t)cus * r.blocks_per_cu, (a.n_tok + TP - 1) / TP));
  if (info != nullptr) {
    *info = r;
    return hipSuccess;
  }
  if (lds > 64 * 1024) {
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3(r.grid), dim3(64 * WV * TP), lds, s, a.v,
                     (const uint16_t*)a.q,
                     (uint16_t*)a.out, a.m_out, a.l_out, a.normalize, a.n_src, a.n_q, a.n_tok,
                     a.eps, 1.0f / (float)a.d);
  return hipGetLastError();
}

// Two token slots per workgroup at D = 2048 with N <= 9 (else one slot per
// workgroup, two workgroups per CU). With two workgroups per CU the second one
// to start falls behind (config 3 on MI355X: its workgroups end 9 us later on
// average and the last ones 26 us after the first) and the CU runs half empty
// until it catches up; two slots in step: 61.2 vs 72.8 us at config 3, 112.6 vs
// 118.4 us at T = 8192. At smaller D or with 16 rows they are slower (D = 1024:
// 39.2 vs 36.8 us; N=16 D=1536 S=16: 111.7 vs 85.0; N=5 D=512 S=6: 23.9 vs 19.3).
// Nor below three tokens per CU, where two slots leave CUs idle (N=9, D=2048,
// S=8: T=256 10.9 vs 9.0 us, T=512 11.7 vs 11.5; T=1024 equal, T=2048 33.2 vs
// 36.1).
template <class T, int KS, int NR, int SQ>
hipError_t launch_mx_slots(const BatchedArgs& a, hipStream_t s, KernelRes* info) {
  int cus = 0;
  if (cu_count(&cus) != hipSuccess || cus < 1) cus = 1;
  const bool enough = a.n_tok > 2 * (int64_t)cus;
  int want = KS == 16 && NR <= 9 && enough ? 2 : 1;
  sy_tuning t;  // measurement override: 1 or 2 slots
  if (tuning_snapshot(&t) && t.mx_slots > 0) want = t.mx_slots;
  KernelRes two;
  if (want == 2 && launch_mx<T, KS, NR, SQ, 2>(a, s, &two) == hipSuccess)
    return launch_mx<T, KS, NR, SQ, 2>(a, s, info);
  return launch_mx<T, KS, NR, SQ, 1>(a, s, info);
}

template <class T, int KS>
hipError_t launch_mx_rows(const BatchedArgs& a, hipStream_t s, KernelRes* info) {
  if (a.n_q <= 8)
    return a.n_src <= 9 ? launch_mx_slots<T, KS, 9, 8>(a, s, info)
                        : launch_mx_slots<T, KS, 16, 8>(a, s, info);
  return a.n_src <= 9 ? launch_mx_slots<T, KS, 9, 16>(a, s, info)
                      : launch_mx_slots<T, KS, 16, 16>(a, s, info);
}

template <class T>
hipError_t launch_mx_dtype(const BatchedArgs& a, hipStream_t s, KernelRes* info) {
  switch (a.d / 128) {
    case 4: return launch_mx_rows<T, 4>(a, s, info);
    case 8: return launch_mx_rows<T, 8>(a, s, info);
    case 12: return launch_mx_rows<T, 12>(a, s, info);
    case 16: return launch_mx_rows<T, 16>(a, s, info);
    case 32:
      // D = 4096: eight waves of 512 columns share a token (one workgroup per
      // CU, N <= 9: ten 8 KiB LDS rows plus the exchange and staging buffers).
      if (a.n_src > 9) return hipErrorInvalidConfiguration;
      return a.n_q <= 8 ? launch_mx<T, 16, 9, 8, 1, 8>(a, s, info)
                        : launch_mx<T, 16, 9, 16, 1, 8>(a, s, info);
    default: return hipErrorInvalidConfiguration;
  }
}

template <class T, int KS, int NR, int W>
hipError_t launch_bmx(const BwdBatchedArgs& a, int grid, hipStream_t s, KernelRes* info) {
  const size_t lds = (size_t)bwd_matrix_dynamic_lds(a.n_src, a.d);
  auto* kern = k_bwd_batched_mx<T, KS, NR, W>;
  KernelRes r{0, 0, 1, 0};
  static hipFuncAttributes fa;
  static const hipError_t fa_err =
      hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(kern));
  hipError_t e = fa_err;
  if (e != hipSuccess) return e;
  r.vgprs = fa.numRegs;
  r.lds = (int)(fa.sharedSizeBytes + lds);
  if (r.lds > 160 * 1024) return hipErrorInvalidConfiguration;
  const int alloc = std::max(8, ((fa.numRegs + 7) / 8) * 8);
  const int by_waves = std::max(1, std::min(8, 512 / alloc) / (W / 4));  // waves per SIMD
  r.blocks_per_cu = std::max(1, std::min(by_waves, (160 * 1024) / std::max(1, r.lds)));
  int cus = 0;
  if (cu_count(&cus) != hipSuccess || cus < 1) cus = 1;
  r.grid = (int)std::max<int64_t>(1, std::min<int64_t>((int64_t)cus * r.blocks_per_cu, a.n_tok));
  if (info != nullptr) {
    *info = r;
    return hipSuccess;
  }
  // Every workgroup needs a token: the dq partial rows are the grid's.
  if (grid < 1 || grid > a.n_tok) return hipErrorInvalidConfiguration;
  if (lds > 64 * 1024) {
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * W), lds, s, a.v, (const uint16_t*)a.q,
                     (const uint16_t*)a.g, a.dv, a.partial, a.n_src, a.n_q, a.n_tok, a.eps,
                     1.0f / (float)a.d);
  return hipGetLastError();
}

template <class T, int KS, int W>
hipError_t launch_bmx_rows(const BwdBatchedArgs& a, int grid, hipStream_t s, KernelRes* info) {
  if constexpr (32 * KS * W == 2048) {  // N <= 9 there (the 16-row tile spills)
    return launch_bmx<T, KS, 9, W>(a, grid, s, info);
  } else {
    return a.n_src <= 9 ? launch_bmx<T, KS, 9, W>(a, grid, s, info)
                        : launch_bmx<T, KS, 16, W>(a, grid, s, info);
  }
}

template <class T>
hipError_t launch_bmx_dtype(const BwdBatchedArgs& a, int grid, hipStream_t s, KernelRes* info) {
  int w = bwd_matrix_waves(a.d);
  // Measurement override: four waves per workgroup where that tile exists.
  sy_tuning t;
  if (tuning_snapshot(&t) && t.bmx_waves == 4) w = 4;
  if (w == 8) {
    switch (a.d) {
      case 1024: return launch_bmx_rows<T, 4, 8>(a, grid, s, info);
      case 2048: return launch_bmx_rows<T, 8, 8>(a, grid, s, info);
      default: break;
    }
  }
  switch (a.d) {
    case 512: return launch_bmx_rows<T, 4, 4>(a, grid, s, info);
    case 1024: return launch_bmx_rows<T, 8, 4>(a, grid, s, info);
    case 1536: return launch_bmx_rows<T, 12, 4>(a, grid, s, info);
    case 2048: return launch_bmx_rows<T, 16, 4>(a, grid, s, info);
    default: return hipErrorInvalidConfiguration;
  }
}

}  // namespace

hipError_t launch_bwd_batched_matrix(const BwdBatchedArgs& a, int grid, hipStream_t s,
                                     KernelRes* info) {
  if (!bwd_matrix_fits(a.n_src, a.n_q, a.d, a.dtype)) return hipErrorInvalidConfiguration;
  if (!bwd_matrix_offsets_fit(a.n_src, a.n_tok, a.d, a.v.stride_bytes))
    return hipErrorInvalidConfiguration;
  if (a.n_tok == 0) return hipSuccess;
  return a.dtype == SY_BF16 ? launch_bmx_dtype<BF16>(a, grid, s, info)
                            : launch_bmx_dtype<F16>(a, grid, s, info);
}

hipError_t launch_batched_matrix(const BatchedArgs& a, hipStream_t s, KernelRes* info) {
  if (!matrix_batched_fits(a.n_src, a.n_q, a.d, a.dtype)) return hipErrorInvalidConfiguration;
  if (!matrix_batched_offsets_fit(a.n_q, a.n_tok, a.d)) return hipErrorInvalidConfiguration;
  if (a.n_tok == 0) return hipSuccess;
  return a.dtype == SY_BF16 ? launch_mx_dtype<BF16>(a, s, info) : launch_mx_dtype<F16>(a, s, info);
}

}  // namespace sy
