// Shape -> kernel plan. Pure arithmetic, no device access, so the CPU test
// suite can pin the dispatch rules (the reference pins its own in
// tests/test_triton_op.py:145-148 and :271-288).
//
// Rules, in order:
//  1. Vector kernels need every row start 16-byte aligned, D a multiple of the
//     chunk width, and (forward/backward) w in v's dtype. Otherwise: generic.
//  2. Prefer the fewest waves per token whose chunks-per-lane is 1, 2 or 4
//     (backward: 1 or 2) and whose resident tile (rows_per_tile x
//     chunks_per_lane 16-byte chunks, four VGPRs each) fits the op's budget
//     with rows_per_tile >= N.
//  3. Forward / speed-of-light whose fewest-waves tile has four chunks per
//     lane but no resident fit (N > 9): online-softmax chunks of 4 rows at
//     that wave count, rather than more waves per token (N=16: 49.9 vs 74.9 us
//     for the resident (2,2,16) tile on MI355X). No resident fit at any wave
//     count: online-softmax chunks of the largest tile that fits.
//  4. Backward with 5 <= N <= 16: four chunks per lane on the waves that cover
//     the row (1, 2 or 4 waves for 9 rows, 1 or 2 for 16), one wave per SIMD
//     with up to 512 registers (config 2: 62.2 vs 64.9 us; D=4096: 130.1 vs
//     134.0 us; N=16: 106.3 vs 113.8 us for (2,2,16)). Otherwise the
//     two-waves-per-SIMD tiles under their budget, then generic. The budget
//     admits 16 rows x 2 chunks when the forward's stats are passed (that
//     variant holds no recompute state and fits 256 VGPRs); without stats that
//     tile spills and the thinner one is kept.
//     Rows of 1025-2048 chunks: eight waves of four chunks, two a SIMD, for
//     2 <= N <= 4, and up to 9 rows with the forward's stats.
//     16 < N <= 32 with stats: the 32-row tile, one chunk per lane on the 2 or
//     4 waves that cover the row, or two chunks on 4 (D = 4096 in bf16);
//     32 < N <= 64 with stats: the 64-row tile, one chunk per lane on 2 or 4
//     waves (rows of up to 256 chunks).
//  5. Batched: 16-bit inputs with N <= 16, 4 <= S <= 16 and D in {512, 1024,
//     1536, 2048} run on the matrix cores (config 3: 8 queries x 9 rows is ~7000
//     VALU instructions a token on the register tile); otherwise resident with
//     S <= 16, else one forward launch per query.
//  6. Batched backward: 16-bit inputs with S <= 8, D in {512, 1024, 1536,
//     2048}, N <= 16 (N <= 9 at D = 2048) and the workgroup's LDS within
//     160 KiB run on the matrix cores, unless the caller says its dv offsets
//     do not fit; otherwise one chunk per lane on the fewest waves that cover the row,
//     N <= 9 and S <= 8 (dv and dq accumulators stay in registers); otherwise
//     the generic kernel while its LDS scalars fit.
#include "../../include/switchyard.h"
#include "sy_launch.hpp"

namespace sy {

namespace {

// Resident tile budget in 16-byte chunks per lane (4 VGPRs each). The
// backward also keeps grad_out, w, their fp32 copies and dw accumulators live,
// so it takes a thinner tile (more waves per token) than the forward unless
// one wave per token fits at one wave per SIMD (rule 4). The batched forward
// holds a query and one accumulator next to the tile, like the forward, and
// gains most from one wave per token: no cross-wave exchange per query
// (config 3, 8 queries: 81.8 us at (1,4,9) vs 115.5 us at (2,2,9) on MI355X).
constexpr int kFwdBudget = 36;
constexpr int kBwdBudget = 18;
constexpr int kBwdStatsBudget = 32;
constexpr int kBatchedBudget = 36;
constexpr int kWaves[] = {1, 2, 4, 8};
constexpr int kRows[] = {4, 9, 16};

bool valid_dtype(int t) { return t == SY_F32 || t == SY_F16 || t == SY_BF16; }

int round_vpl(int64_t v) { return v <= 1 ? 1 : (v <= 2 ? 2 : (v <= 4 ? 4 : 0)); }

bool tile_exists(int vpl, int nr) { return !(vpl == 4 && nr == 16); }

void set(sy_plan* p, int family, int w, int vpl, int nr, int ce, int op, int64_t n_src) {
  p->family = family;
  p->waves_per_token = w;
  p->chunks_per_lane = vpl;
  p->rows_per_tile = nr;
  p->elems_per_chunk = ce;
  if (family == SY_FAMILY_GENERIC) {
    p->block_threads = 256;
    p->tokens_per_block = 1;
    p->n_chunks = 1;
    return;
  }
  if (op == SY_OP_BWD) {
    p->block_threads = bwd_block(w, vpl, nr);
    p->tokens_per_block = p->block_threads / (64 * w);
  } else {
    p->block_threads = 64 * w > 256 ? 64 * w : 256;
    p->tokens_per_block = p->block_threads / (64 * w);
  }
  p->n_chunks = (int)((n_src + nr - 1) / nr);
}

// Resident plan with rows_per_tile >= n_src under `budget` and at most
// `max_vpl` chunks per lane; false if none.
bool resident(int64_t n_src, int64_t e, int budget, int max_vpl, int* w_out, int* vpl_out,
              int* nr_out) {
  for (int w : kWaves) {
    const int vpl = round_vpl((e + 64 * w - 1) / (64 * w));
    if (vpl == 0 || vpl > max_vpl) continue;
    for (int nr : kRows) {
      if (!tile_exists(vpl, nr) || nr < n_src || nr * vpl > budget) continue;
      *w_out = w;
      *vpl_out = vpl;
      *nr_out = nr;
      return true;
    }
  }
  return false;
}

}  // namespace

int make_plan(int op, int64_t n_src, int64_t n_q, int64_t d, int v_dtype, int w_dtype,
              int aligned, sy_plan* out, int has_stats, int matrix_ok) {
  if (out == nullptr) return SY_ERR_NULL;
  if (op < SY_OP_FWD || op > SY_OP_BWD_BATCHED) return SY_ERR_OP;
  if (!valid_dtype(v_dtype) || !valid_dtype(w_dtype)) return SY_ERR_DTYPE;
  const bool batched = op == SY_OP_BATCHED || op == SY_OP_BWD_BATCHED;
  if (n_src < 1 || d < 1 || (batched && n_q < 1)) return SY_ERR_SHAPE;
  if (n_src > 0x7fffffff || d > 0x7fffffff / 16 || n_q > 0x7fffffff) return SY_ERR_SHAPE;

  const int ce = v_dtype == SY_F32 ? 4 : 8;
  const bool same_w = op == SY_OP_SOL || batched || v_dtype == w_dtype;
  const bool vec = aligned && (d % ce == 0) && same_w;
  const int64_t e = d / ce;
  int w = 0, vpl = 0, nr = 0;

  if (op == SY_OP_BWD_BATCHED) {
    if (vec && matrix_ok && bwd_matrix_fits(n_src, n_q, d, v_dtype)) {
      out->family = SY_FAMILY_MATRIX;
      out->waves_per_token = 4;
      out->chunks_per_lane = 1;
      out->rows_per_tile = n_src <= 9 ? 9 : 16;
      out->elems_per_chunk = ce;
      out->block_threads = 256;
      out->tokens_per_block = 1;
      out->n_chunks = 1;
      return SY_OK;
    }
    if (vec && n_src <= kBwdBatchedMaxN && n_q <= kBwdBatchedMaxQ) {
      for (int ww : kWaves) {
        if ((int64_t)64 * ww < e) continue;
        set(out, SY_FAMILY_RESIDENT, ww, 1, n_src <= 4 ? 4 : 9, ce, op, n_src);
        return SY_OK;
      }
    }
    if (bwd_batched_generic_lds(n_src, n_q) > kGenericMaxLds) return SY_ERR_SHAPE;
    set(out, SY_FAMILY_GENERIC, 4, 0, 0, 1, op, n_src);
    return SY_OK;
  }

  if (op == SY_OP_BATCHED && vec && matrix_batched_fits(n_src, n_q, d, v_dtype)) {
    out->family = SY_FAMILY_MATRIX;
    out->waves_per_token = d == 4096 ? 8 : 4;  // a wave's slice is at most 512 columns
    out->chunks_per_lane = 1;
    out->rows_per_tile = (int)kMatrixMaxRows;
    out->elems_per_chunk = ce;
    out->block_threads = 64 * out->waves_per_token;
    out->tokens_per_block = 1;
    out->n_chunks = 1;
    return SY_OK;
  }
  // Four chunks per lane at one wave per SIMD pay off from 5 rows on (N=9:
  // 62.2 vs 64.9 us), and from 2 rows on for 16-bit sources (T=4096 bf16,
  // D=2048: N=2 17.4 vs 18.5 us, N=4 28.5 vs 30.2; D=4096: N=4 52.6 vs 56.1;
  // D=8192: N=4 101.1 vs 109.3). With fp32 sources and N <= 4 two chunks on
  // twice the waves stay faster (D=2048, N=4: 52.6 vs 58.1 us). Rows of more
  // than 1024 chunks take eight such waves (below). The 16-row tile holds 256 VGPRs of source
  // rows: its recompute variant (no stats) spills 68 bytes a lane and still
  // beats the thinner tiles (N=16: 119 vs 167 us).
  // 16 < N <= 32 with the forward's stats: 32 rows resident, a token on as
  // few waves as the registers allow -- two waves with one or two chunks a
  // lane, four with two from 512 chunks on (v read once; the generic kernel
  // reads it twice with element-wise loads). At N=32, D=2048 bf16 two waves
  // of two chunks run the backward in 207 us against 237 us for four waves of
  // one (fewer waves share each row's loads and each token's barrier).
  // Without stats the per-row scalars would not fit; that case stays generic.
  if (vec && op == SY_OP_BWD && has_stats && n_src > 16 && n_src <= kTallRows && e > 64) {
    const int ww = e <= 256 ? 2 : 4, vv = e <= 128 ? 1 : 2;
    if (e <= 512) {
      set(out, SY_FAMILY_RESIDENT, ww, vv, kTallRows, ce, op, n_src);
      return SY_OK;
    }
  }
  // 32 < N <= 64 with stats: 64 rows of one chunk a lane on two or four waves
  // (rows of up to 256 chunks: 16-bit D <= 2048, fp32 D <= 1024), one wave per
  // SIMD.
  if (vec && op == SY_OP_BWD && has_stats && n_src > kTallRows && n_src <= kTallerRows && e > 64 &&
      e <= 256) {
    set(out, SY_FAMILY_RESIDENT, e <= 128 ? 2 : 4, 1, kTallerRows, ce, op, n_src);
    return SY_OK;
  }
  if (vec && op == SY_OP_BWD && (n_src > 4 || (n_src >= 2 && ce == 8)) && n_src <= 16) {
    for (int ww : {1, 2, 4}) {
      if (n_src > 9 && ww == 4) break;
      if (e > 64 * 2 * ww && e <= 64 * 4 * ww) {
        set(out, SY_FAMILY_RESIDENT, ww, 4, n_src <= 4 ? 4 : n_src <= 9 ? 9 : 16, ce, op, n_src);
        return SY_OK;
      }
    }
  }
  // Rows of 1025-2048 chunks (fp32 D = 8192, 16-bit D = 16384): only eight
  // waves of four chunks cover them, two waves a SIMD at 256 VGPRs each (16-bit
  // rows keep w and grad_out packed there). The 4-row tile fits (167-225
  // VGPRs); the 9-row one with the forward's stats spills 4 VGPRs in fp32 and
  // 51-72 in 16 bits and still runs the backward 4-6x faster than the generic
  // kernel (bf16 T=2048 D=16384: N=9 313 vs 1842 us, N=5 206 vs 1100; fp32
  // T=4096 D=8192 N=9 447 vs 1696). Its recompute variants (over 100 spilled)
  // and more rows stay generic.
  if (vec && op == SY_OP_BWD && e > 64 * 4 * 4 && e <= 64 * 4 * 8 && n_src >= 2 &&
      (n_src <= 4 || (n_src <= 9 && has_stats))) {
    set(out, SY_FAMILY_RESIDENT, 8, 4, n_src <= 4 ? 4 : 9, ce, op, n_src);
    return SY_OK;
  }
  if (vec && !(op == SY_OP_BATCHED && n_q > kBatchedMaxQ)) {
    const int budget = op == SY_OP_BWD     ? (has_stats ? kBwdStatsBudget : kBwdBudget)
                       : op == SY_OP_BATCHED ? kBatchedBudget
                                             : kFwdBudget;
    // The backward keeps grad_out, w (raw and fp32) and dw accumulators next
    // to the tile: with 4 chunks per lane some of its variants spill.
    const int max_vpl = op == SY_OP_BWD ? 2 : 4;
    if ((op == SY_OP_FWD || op == SY_OP_SOL) && n_src > 9) {
      for (int ww : kWaves) {
        const int v2 = round_vpl((e + 64 * ww - 1) / (64 * ww));
        if (v2 == 0) continue;
        if (v2 == 4) {
          set(out, SY_FAMILY_CHUNKED, ww, 4, 4, ce, op, n_src);
          return SY_OK;
        }
        break;
      }
    }
    if (resident(n_src, e, budget, max_vpl, &w, &vpl, &nr)) {
      set(out, SY_FAMILY_RESIDENT, w, vpl, nr, ce, op, n_src);
      return SY_OK;
    }
    if (op == SY_OP_FWD || op == SY_OP_SOL) {
      for (int ww : kWaves) {
        const int v2 = round_vpl((e + 64 * ww - 1) / (64 * ww));
        if (v2 == 0) continue;
        set(out, SY_FAMILY_CHUNKED, ww, v2, v2 == 4 ? 4 : 16, ce, op, n_src);
        return SY_OK;
      }
    }
  }
  if (op == SY_OP_BATCHED) {
    // Per-query forward launches; report the plan each of them uses.
    const int rc = make_plan(SY_OP_FWD, n_src, 0, d, v_dtype, v_dtype, aligned, out);
    if (rc != SY_OK) return rc;
    out->family = SY_FAMILY_PER_QUERY;
    return SY_OK;
  }
  if ((op == SY_OP_FWD || op == SY_OP_BWD) && n_src > kGenericMaxN) return SY_ERR_SHAPE;
  set(out, SY_FAMILY_GENERIC, 4, 0, 0, 1, op, n_src);
  return SY_OK;
}

bool tile_listed(int op, int w, int vpl, int nr) {
#define X(W_, V_, N_) \
  if (w == W_ && vpl == V_ && nr == N_) return true;
  SY_TILES(X)
  if (op == SY_OP_BWD) {
    SY_BWD_WIDE_TILES(X)
    SY_BWD_TALL_TILES(X)
  }
#undef X
  return false;
}

// Measurement override (sy_tuning_set): a forced "W,VPL,NR" tile replaces the
// tile of a vector plan when that tile is built, covers the row, and
// (backward, batched) holds every row. Anything else leaves the plan untouched.
void apply_tile_override(int op, int64_t n_src, int64_t d, sy_plan* p) {
  const bool tiled = p->family == SY_FAMILY_RESIDENT || p->family == SY_FAMILY_CHUNKED;
  if (!tiled && !(op == SY_OP_BATCHED && p->family == SY_FAMILY_MATRIX)) return;
  sy_tuning t;
  if (!tuning_snapshot(&t)) return;
  const int32_t* f = op == SY_OP_FWD ? t.fwd_tile
                     : op == SY_OP_BWD ? t.bwd_tile
                     : op == SY_OP_BATCHED ? t.batched_tile
                                           : t.sol_tile;
  const int w = f[0], vpl = f[1], nr = f[2];
  if (w == 0 || !tile_listed(op, w, vpl, nr)) return;
  if ((int64_t)64 * w * vpl < d / p->elems_per_chunk) return;
  const bool can_chunk = op == SY_OP_FWD || op == SY_OP_SOL;
  if (nr < n_src && !can_chunk) return;
  set(p, nr >= n_src ? SY_FAMILY_RESIDENT : SY_FAMILY_CHUNKED, w, vpl, nr, p->elems_per_chunk, op,
      n_src);
}

// Token-count rule. With at most two tokens per CU the one-wave tiles leave
// the CUs short of waves, and tiles that spread a token over four waves move
// the same bytes sooner. Measured on MI355X, bf16 D = 2048 (forward and
// forward + backward, us, plan tiles -> this rule):
//   N=9  T=512: 9.41 -> 8.75,  25.0 -> 21.9     N=9  T=256: 8.95 -> 7.57, 23.7 -> 20.0
//   N=4  T=512: 5.65 -> 5.07,  15.7 -> 14.1     N=16 T=512: 14.7 -> 13.6, 36.9 -> 32.7
// At four tokens per CU (T = 1024) the one-wave tiles are faster again. The
// forward takes (4,1) at up to one token per CU, else (2,2); the backward
// (4,1), also at N = 2 (backward main kernel, device time from graph replays:
// T=256 5.20 -> 3.91 us, T=512 5.73 -> 4.73; the forward gains nothing there).
// Rows of two chunks a lane at one wave (16-bit D = 1024): the backward takes
// (4,1) up to two tokens per CU and (2,1) at up to four. (4,1) covers twice the
// row, and its upper two waves' loads, stores and partial-row writes fall
// outside their buffer ranges, but it puts one token in each workgroup where
// (2,1) puts two, so the tokens reach twice the CUs. Backward main kernel, us:
//   N=9  T=128: 9.56 -> 6.94   T=512: 10.39 -> 7.67   T=1024: 10.93 -> 9.38
//   N=16 T=128: 16.62 -> 11.54 T=512: 17.45 -> 12.35  T=1024: 18.23 -> 15.59
//   N=2  T=512: 5.03 -> 3.91   N=4 T=512: 6.42 -> 4.93 (fp16 N=9 T=512: 10.35 -> 7.73)
// and at eight tokens per CU the one-wave tile stays (N=16 T=2048: 26.1 vs 31.6).
// The forward's one-wave tiles at D = 1024 are already the fastest there.
// fp32 rows (four elements a chunk) behave the same in the backward: D = 1024
// (four chunks a lane) N=9 T=128 9.75 -> 7.52, T=512 11.24 -> 9.19, N=16
// T=128 16.65 -> 12.67, N=4 T=256 5.81 -> 4.49 (four tokens per CU: within
// 4% either way, so the plan's tile); D = 512 (two chunks) N=9 T=256
// 8.92 -> 7.25, T=1024 10.70 -> 9.33. The fp32 forward has a branch of its own
// (below).
// The forward over 10-16 rows (16-bit D = 2048, the chunked family) keeps its
// four-row chunks and spreads a token over four waves up to three tokens per
// CU, over two up to six (HIP-graph replays, bf16, us, plan tile -> this rule):
//   N=16 T=256 10.60 -> 10.12, T=512 14.09 -> 12.13, T=768 15.18 -> 14.17,
//        T=1024 17.24 -> 16.23, T=1280 22.58 -> 17.97, T=1536 23.36 -> 20.16
//   N=12 T=512 11.95 -> 9.87, T=1024 13.98 -> 13.08; N=10 T=256 8.38 -> 7.60
// (fp16 the same within 0.2 us); at eight tokens per CU the one-wave chunks
// stay (N=16 T=2048: 26.1 vs 28.1 us on two waves). Where a caller needs a
// resident tile (the fused merge carries its prior as one more row),
// `chunked_ok` false keeps the 16-row resident tiles of the rule below.
void apply_token_rule(int op, int64_t n_src, int64_t n_tok, sy_plan* p, bool chunked_ok) {
  if (op != SY_OP_FWD && op != SY_OP_BWD) return;
  const bool tiled = p->family == SY_FAMILY_RESIDENT || p->family == SY_FAMILY_CHUNKED;
  const bool bwd = op == SY_OP_BWD;
  if (!tiled || n_src < 2 || n_src > 16) return;
  const int span = p->waves_per_token * p->chunks_per_lane;  // one wave's chunks a lane
  if (!bwd && p->elems_per_chunk == 4) {
    // fp32 forward: four waves a token up to one token per CU (rows of four or
    // eight chunks a lane), and for 10-16 rows four-row chunks on four waves up
    // to two (HIP-graph replays, us, plan tile -> this rule: N=9 D=2048 T=256
    // 8.65 -> 7.59, D=1024 6.94 -> 5.99; N=16 D=2048 T=512 18.25 -> 16.18; at
    // two tokens per CU the 9-row plan tiles stay, 10.63 vs 10.90, and from four
    // tokens per CU every plan tile).
    if (n_src < 3 || (span != 4 && span != 8)) return;
    int cus = 0;
    if (cu_count(&cus) != hipSuccess || cus < 1 || n_tok < 1) return;
    const int vv = span / 4;
    if (n_src > 9) {
      if (!chunked_ok || n_tok > 2 * (int64_t)cus || !tile_listed(op, 4, vv, 4)) return;
      set(p, SY_FAMILY_CHUNKED, 4, vv, 4, p->elems_per_chunk, op, n_src);
      return;
    }
    const int nr4 = n_src <= 4 ? 4 : 9;
    if (n_tok > cus || !tile_listed(op, 4, vv, nr4)) return;
    set(p, SY_FAMILY_RESIDENT, 4, vv, nr4, p->elems_per_chunk, op, n_src);
    return;
  }
  if (!bwd && (p->elems_per_chunk != 8 || n_src < 3)) return;  // forward: 16-bit rows, N >= 3
  if (span == 8 && p->elems_per_chunk == 8 && n_src <= 9) {
    // 16-bit rows of eight chunks a lane (D = 4096) up to one token per CU: the
    // forward on four waves of two chunks, the backward on eight of one (HIP-graph
    // replays, bf16, us, plan tile -> this rule: N=9 T=256 forward 9.50 -> 7.88,
    // backward 12.40 -> 10.56; T=128 8.80 -> 6.77, 11.51 -> 8.55; N=4 T=256
    // 5.40 -> 4.47, 7.26 -> 6.29; at two tokens per CU the plan tiles stay,
    // 11.53 vs 11.99 and 15.8 vs 16.4).
    int cus8 = 0;
    if (cu_count(&cus8) != hipSuccess || cus8 < 1 || n_tok < 1 || n_tok > cus8) return;
    const int nr8 = n_src <= 4 ? 4 : 9;
    const int w8 = bwd ? 8 : 4, v8 = bwd ? 1 : 2;
    if (!tile_listed(op, w8, v8, nr8)) return;
    set(p, SY_FAMILY_RESIDENT, w8, v8, nr8, p->elems_per_chunk, op, n_src);
    return;
  }
  if (span != 4 && !(span == 2 && bwd && p->waves_per_token == 1)) return;
  int cus = 0;
  if (cu_count(&cus) != hipSuccess || cus < 1) return;
  if (n_tok < 1) return;
  if (!bwd && n_src > 9 && chunked_ok) {
    if (n_tok > 6 * (int64_t)cus) return;
    const int wc = n_tok <= 3 * (int64_t)cus ? 4 : 2;
    if (!tile_listed(op, wc, 4 / wc, 4)) return;
    set(p, SY_FAMILY_CHUNKED, wc, 4 / wc, 4, p->elems_per_chunk, op, n_src);
    return;
  }
  if (n_tok > (span == 4 ? 2 : 4) * (int64_t)cus) return;
  const int nr = n_src <= 4 ? 4 : n_src <= 9 ? 9 : 16;
  const int w = span == 2 ? (n_tok <= 2 * (int64_t)cus ? 4 : 2) : (bwd || n_tok <= cus ? 4 : 2);
  const int vpl = span == 2 ? 1 : 4 / w;
  if (!tile_listed(op, w, vpl, nr)) return;
  set(p, SY_FAMILY_RESIDENT, w, vpl, nr, p->elems_per_chunk, op, n_src);
}

void apply_tile_rules(int op, int64_t n_src, int64_t n_tok, int64_t d, sy_plan* p, bool chunked_ok) {
  apply_token_rule(op, n_src, n_tok, p, chunked_ok);
  apply_tile_override(op, n_src, d, p);
}

}  // namespace sy
