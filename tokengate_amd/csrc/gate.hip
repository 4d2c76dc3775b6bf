// Gate path for gfx950: scoring head, order-preserving top-K keep list, ragged pack.
//
// Reference (tokengate/e2e_gate/gate_module/gate_forward.py):
//   * score + select, :1384-1433 — per sample: K_c = max(1, min(K, n_art)), topk over the
//     article scores, keep = cat(arange(s), s + sort(topk), arange(e, seq_len)) (:1417-1421,
//     the same list as _keep_indices :77-81);
//   * prune + pack, :1435-1522 — hidden rows and per-layer K/V rows gathered at the kept
//     positions (index_select, :1497-1520), kept positions recorded for RoPE (:1457), the gate
//     bias of kept article rows (build_gate_bias_vectorized :968-1036; RMS-normalised over the
//     article as in E2EGate.forward, e2e_gate_module.py:348-385), zero on prefix/suffix rows.
// This library packs the kept rows of all sequences back to back (varlen / cu_seqlens layout)
// instead of padding to the longest, and breaks score ties by the lower index.
//
// Kernels:
//   gate_score_kernel  — s = w2 . silu(W1 x + b1) + b2 for every row of a packed (rows, 2048)
//                        bf16 matrix (128 or 256 rows per workgroup; W1 x on bf16 MFMA, fp32
//                        epilogue);
//   gate_topk_*kernel  — one workgroup per sequence: order-preserving uint32 keys, 4-pass 8-bit
//                        radix select of the K_c-th largest key (keys held in registers for
//                        articles up to 65536 tokens, else re-read from global memory), then an
//                        index-order compaction (ballot ranks over 64-key blocks) that keeps keys
//                        above the threshold and the lowest-index ties, writing ascending
//                        positions; also the article's sum of squared scores;
//   gate_pack_kernel   — one launch gathers every kept row for any number of row streams (hidden
//                        states, per-layer K and V, head-chunked rows) in 16-byte units, plus the
//                        kept positions and the kept rows' gate bias.
#include <algorithm>
#include <type_traits>
#include <utility>

#include "tg_common.h"
#include "../../include/tokengate_hip.h"

namespace tg {
namespace {

// ---------------------------------------------------------------------------------------------
// Scoring head: s = w2 . silu(W1 x + b1) + b2, x in R^2048 (bf16), W1 (256 x 2048) bf16.
// Workgroup: 8 waves, 256 rows (128 for grids too small to give every CU two 256-row workgroups);
// wave w owns rows 128(w%2)..+127 and hidden units 64(w/2)..+63 (4 x 2 blocks of 32 x 32; 12 KiB of
// X and W fragments per wave per k step for 16 MFMAs; half of that with 128 rows).  Every
// workgroup streams all of W1 (1 MiB, L2-resident) through LDS once, so the rows per workgroup set
// how many W1 bytes each X byte costs: 256 rows make it 2 MiB of X per 1 MiB of W1.  K loop over
// the 2048 inputs in steps of 32 through an LDS ring filled by DMA (256 rows: 4 slots of X tile
// 256 x 32 + W1 tile 256 x 32, 32 KiB per slot; 128 rows: 6 slots of 24 KiB), unrolled so that
// every ring slot index is a compile-time constant, and software-pipelined: a wave reads step
// k+1's fragments from LDS while its MFMAs of step k run, so the LDS reads and the
// matrix cores overlap instead of alternating between the per-step barriers.  Accumulators are
// C^T blocks (hidden unit = MFMA row, token = column): each lane ends with one token's hidden
// units of each block, the SiLU . w2 reduction is in-lane plus one cross-half exchange, and the four
// hidden quarters of a row are added through LDS in a fixed order.
// At 256 FLOP per byte of X the head sits at the ridge of the MFMA and HBM roofs.  Probes at 710k
// rows with 128-row workgroups, each with one piece compiled out, took 0.33x of the full time with
// only the matrix work, 0.49x with X alone and 0.54x with W1 alone.  A form that loaded W1 from
// L2 straight into registers, leaving only X in the LDS ring, was slower at every size.  The limit
// is therefore the per-step chain (barrier, DMA wait, fragment reads), with MFMA busy about half the
// SIMD cycles.  The SiLU takes the hardware reciprocal: the IEEE division it replaced cost about
// one VALU instruction per MFMA in the epilogue, which both waves of a SIMD run at the same time.
// ---------------------------------------------------------------------------------------------
// f(integral_constant<int, J>) for J = 0, 1, ... in order
template <typename F, int... J>
__device__ __forceinline__ void for_each_c(F &&f, std::integer_sequence<int, J...>) {
  (f(std::integral_constant<int, J>()), ...);
}

constexpr int kDin = 2048;
constexpr int kDh = 256;
constexpr int kSRowsMax = 256;
constexpr int kSK = 32;
constexpr int kSThreads = 512;

struct ScoreArgs {
  const bf16_t *x;
  int64_t x_rs;        // row stride (elements)
  int64_t n_rows;
  const bf16_t *w1;    // element (u, k) at w1[u * w_rs + (k / 32) * w_ss / 2 + k % 32]:
  int64_t w_rs;        //   row-major (256, 2048): w_rs = 2048, w_ss = 64 bytes;
  int64_t w_ss;        //   k-step major (64, 256, 32): w_rs = 32, w_ss = 16384 bytes (a step's 16 KiB contiguous)
  const float *b1, *w2;
  float b2;
  float *out;
};

// ROWS rows per workgroup (128 or 256: wave w owns rows (ROWS/2)(w%2) .. +ROWS/2-1, in ROWS/64
// blocks of 32, and hidden units 64(w/2) .. +63), S-deep LDS ring.
template <int ROWS, int S>
__global__ __launch_bounds__(kSThreads, 1) void gate_score_kernel(ScoreArgs a) {
  constexpr int RB = ROWS / 64;            // 32-row blocks per wave
  constexpr int XI = ROWS / 128;           // 1 KiB X DMA issues per wave per step
  constexpr int kXBytes = ROWS * kSK * 2, kWBytes = kDh * kSK * 2;
  static_assert(S >= 4 && S <= 6 && S * (kXBytes + kWBytes) <= 160 * 1024, "ring fits the LDS");
  // X tile: ROWS rows x 64 B, W tile: 256 rows x 64 B; 16-byte chunks, 4 per row, XOR-swizzled.
  // One __shared__ object per ring slot: the compiler separates LDS-DMA writes from LDS reads
  // only across distinct objects, so a slot's DMA does not hold up the reads of the others.
  constexpr int kX5 = S > 4 ? kXBytes : 16, kW5 = S > 4 ? kWBytes : 16;   // unused slots: minimal
  constexpr int kX6 = S > 5 ? kXBytes : 16, kW6 = S > 5 ? kWBytes : 16;
  __shared__ __attribute__((aligned(1024))) char xs0[kXBytes], xs1[kXBytes], xs2[kXBytes], xs3[kXBytes],
      xs4[kX5], xs5[kX6];
  __shared__ __attribute__((aligned(1024))) char ws0[kWBytes], ws1[kWBytes], ws2[kWBytes], ws3[kWBytes],
      ws4[kW5], ws5[kW6];
  auto xsl = [&](auto b) -> char * {
    constexpr int B = decltype(b)::value;
    if constexpr (B == 0) return xs0; else if constexpr (B == 1) return xs1; else if constexpr (B == 2) return xs2;
    else if constexpr (B == 3) return xs3; else if constexpr (B == 4) return xs4; else return xs5;
  };
  auto wsl = [&](auto b) -> char * {
    constexpr int B = decltype(b)::value;
    if constexpr (B == 0) return ws0; else if constexpr (B == 1) return ws1; else if constexpr (B == 2) return ws2;
    else if constexpr (B == 3) return ws3; else if constexpr (B == 4) return ws4; else return ws5;
  };
  const int tid = threadIdx.x, wave = wave_id(), lane = tid & 63, lq = lane & 31, g = lane >> 5;
  const int rg = wave & 1, hq = wave >> 1;   // row half, hidden quarter
  const int64_t r0 = (int64_t)blockIdx.x * ROWS;

  const int64_t rows_here = min((int64_t)ROWS, a.n_rows - r0);
  const brsrc_t xrs = make_rsrc(a.x + r0 * a.x_rs, (uint32_t)(((rows_here - 1) * a.x_rs + kDin) * 2));
  const brsrc_t wrs = make_rsrc(a.w1, (uint32_t)(kDh * kDin * 2));
  // DMA slots: X tile = 4 ROWS chunks (XI 1 KiB issues per wave), W tile = 1024 chunks (two);
  // LDS row r (64 B), physical chunk p holds logical chunk p ^ ((r>>2)&3): the 16 rows that 16
  // lanes read with one chunk index then land on 16 distinct 16-byte bank groups of the 64-bank
  // LDS (rows r and r+1..3 share a 256-byte bank line at different quarters; rows 4 apart get
  // different chunks).  Per-lane source offsets (bytes) within a k step; the step's byte offset is
  // added per issue.
  uint32_t xoff[XI], woff[2];
#pragma unroll
  for (int it = 0; it < XI; ++it) {
    const int slot = (wave * XI + it) * 64 + lane;
    const int r = slot >> 2, p = slot & 3;
    xoff[it] = (uint32_t)((r * a.x_rs + 8 * (p ^ ((r >> 2) & 3))) * 2);
  }
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int slot = (wave * 2 + it) * 64 + lane;        // 0..1023
    const int r = slot >> 2, p = slot & 3;
    woff[it] = (uint32_t)((r * a.w_rs + 8 * (p ^ ((r >> 2) & 3))) * 2);
  }
  auto issue = [&](int kstep, auto buf_c) {
    const uint32_t k0b = (uint32_t)(kstep * kSK * 2), k0w = (uint32_t)(kstep * a.w_ss);
    char *xd = xsl(buf_c), *wd = wsl(buf_c);
#pragma unroll
    for (int it = 0; it < XI; ++it) dma16(xrs, xd + (wave * XI + it) * 1024, xoff[it] + k0b);
#pragma unroll
    for (int it = 0; it < 2; ++it) dma16(wrs, wd + (wave * 2 + it) * 1024, woff[it] + k0w);
  };

  // fragments of one k step: [substep s][block]: X^T columns (B operand, token (ROWS/2)rg + 32t +
  // lq) and W1 rows (A operand, hidden unit 64hq + 32j + lq), k = 16s + 8g .. +7
  struct Frags {
    bf16x8 x[2][RB], w[2][2];
  };
  auto read = [&](auto buf_c, Frags &f) {
    const char *xb_lds = xsl(buf_c), *wb_lds = wsl(buf_c);
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const uint32_t c = (uint32_t)(2 * s2 + g);
#pragma unroll
      for (int b = 0; b < RB; ++b) {
        const int xr = (ROWS / 2) * rg + 32 * b + lq;
        f.x[s2][b] = lds_load16(xb_lds, xr * 64 + ((c ^ ((xr >> 2) & 3)) << 4));
      }
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const int wr = 64 * hq + 32 * b + lq;
        f.w[s2][b] = lds_load16(wb_lds, wr * 64 + ((c ^ ((wr >> 2) & 3)) << 4));
      }
    }
  };

  f32x16 acc[2][RB];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int t = 0; t < RB; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[j][t][v] = 0.f;
  auto mma = [&](const Frags &f) {
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int t = 0; t < RB; ++t) acc[j][t] = mfma32(f.w[s2][j], f.x[s2][t], acc[j][t]);
  };

  constexpr int nk = kDin / kSK;
  constexpr int kOps = XI + 2;   // DMA ops per thread per step
  constexpr int L = S % 2 == 0 ? S : 2 * S;   // unroll: ring slots and the two fragment sets cycle
  static_assert((nk - 4) % L == 0, "the k loop is unrolled L steps at a time, with a four-step tail");
  // Iteration ks (compile-time ring slots): cur holds step ks's fragments (read in the previous
  // iteration).  Wait until step ks+1's DMA of this wave is done (the DMA ops of steps issued after
  // it may stay in flight), barrier (step ks+1 resident for every wave; the slot of step ks-1 is
  // free), refill that slot with step ks+S-1, read step ks+1's fragments into nxt, then run step
  // ks's MFMAs while those reads are in flight.  Steps ks+2 .. ks+S-2 are in flight at the wait.
  auto iter = [&](int ks, Frags &cur, Frags &nxt, auto next_c, auto waitn_c) {
    constexpr int NX = decltype(next_c)::value;                   // slot of step ks+1
    constexpr int FREE = (NX + S - 2) % S;                        // slot of step ks-1
    if (ks + 1 < nk) wait_vm<decltype(waitn_c)::value>();
    ring_barrier();
    if (ks + S - 1 < nk) issue(ks + S - 1, std::integral_constant<int, FREE>());
    if (ks + 1 < nk) read(std::integral_constant<int, NX>(), nxt);
    mma(cur);
  };
  // step j of an unrolled group (j known at compile time; the group starts at a multiple of L)
  auto step = [&](int ks, auto j_c, Frags &fa, Frags &fb, auto waitn_c) {
    constexpr int J = decltype(j_c)::value;
    if constexpr (J % 2 == 0) iter(ks, fa, fb, std::integral_constant<int, (J + 1) % S>(), waitn_c);
    else iter(ks, fb, fa, std::integral_constant<int, (J + 1) % S>(), waitn_c);
  };
  Frags fa, fb;
  for_each_c([&](auto k_c) { issue(decltype(k_c)::value, k_c); }, std::make_integer_sequence<int, S - 1>());
  wait_vm<(S - 2) * kOps>();   // step 0 resident for this wave
  ring_barrier();
  read(std::integral_constant<int, 0>(), fa);
  using Wsteady = std::integral_constant<int, (S - 3) * kOps>;
  int ks = 0;
  for (; ks + L <= nk - 4; ks += L)
    for_each_c([&](auto j_c) { step(ks + decltype(j_c)::value, j_c, fa, fb, Wsteady()); },
               std::make_integer_sequence<int, L>());
  // the last four steps (nk-4 .. nk-1, steps 0..3 of a group): at step ks the steps after ks+1
  // up to min(ks+S-2, nk-1) are in flight, none after the last DMA
  for_each_c([&](auto j_c) {
    constexpr int J = decltype(j_c)::value;
    constexpr int kInFlight = std::max(0, std::min(nk - 4 + J + S - 2, nk - 1) - (nk - 4 + J + 1));
    step(ks + J, j_c, fa, fb, std::integral_constant<int, kInFlight * kOps>());
  }, std::make_integer_sequence<int, 4>());

  // epilogue: lane holds token (ROWS/2)rg + 32t + lq and hidden units 64hq + 32j + 8(v/4) + 4g + v%4
  __shared__ float red[4][ROWS];   // per hidden quarter, per row
#pragma unroll
  for (int t = 0; t < RB; ++t) {
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int u = 64 * hq + 32 * j + 8 * (v >> 2) + 4 * g + (v & 3);
        const float h = acc[j][t][v] + a.b1[u];
        const float sl = h * __builtin_amdgcn_rcpf(1.f + __expf(-h));   // SiLU, reciprocal to 1 ulp
        part = fmaf(sl, a.w2[u], part);
      }
    const float tot = pair_sum(part);
    if (g == 0) red[hq][(ROWS / 2) * rg + 32 * t + lq] = tot;
  }
  __syncthreads();
  if (tid < ROWS) {
    const int64_t row = r0 + tid;
    if (row < a.n_rows) a.out[row] = (((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid]) + a.b2;
  }
}

// ---------------------------------------------------------------------------------------------
// Top-K keep list.  Per sequence b the geometry row (int32 x 6) is
//   [row_start, seq_len, art_start, art_end, k_clamped, kept_start]
// with scores of the sequence's rows at scores[row_start + i]; the kept positions (within the
// sequence, ascending) go to keep[kept_start .. kept_start + art_start + k_clamped + seq_len - art_end).
// ---------------------------------------------------------------------------------------------
constexpr int kTThreads = 1024;
constexpr int kTWaves = kTThreads / 64;

// float -> uint32 whose unsigned order is the float order; -0 == +0; NaN above +inf.  Branch-free
// (selects only) so that it can run over register-resident key arrays.
__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  uint32_t k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  k = (f == 0.f) ? 0x80000000u : k;
  k = (f != f) ? 0xffffffffu : k;
  return k;
}

// The float an order key stands for (inverse of order_key; zero comes back as +0).
__device__ __forceinline__ float key_value(uint32_t k) {
  return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Bin of value v among 256 equal-width bins over [vmin, vmin + 256 / inv]: non-decreasing in v, so
// every bin holds a contiguous range of the key order.
__device__ __forceinline__ int value_bin(float v, float vmin, float inv) {
  return min(255, (int)((v - vmin) * inv));
}

__device__ __forceinline__ int lanes_below(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Wave 0: over the 16 per-wave 256-bin histograms, find the bin d holding the sel[2]-th largest
// element (bins counted from the top); sel[3] = d, sel[4] = its element count, sel[2] = the rank
// within the bin; for key-space bins (width 2^shift from lo) also sel[0..1] = the bin's key range
// (clipped to the current hi).
// NH = number of histograms to sum (16 per-wave ones, or 1 shared one).
template <int NH = kTWaves>
__device__ __forceinline__ void select_bin(int (*h)[256], int lane, uint32_t *sel, uint32_t lo, int shift) {
  // lane l owns bins 255-4l .. 252-4l (descending)
  int c[4], lt = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    int t = 0;
#pragma unroll
    for (int w = 0; w < NH; ++w) t += h[w][255 - 4 * lane - j];
    c[j] = t;
    lt += t;
  }
  int incl = lt;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  const int before = incl - lt;
  const int krem = (int)sel[2];
  if (before < krem && krem <= incl) {
    int acc = before, d = 0, cd = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (acc + c[j] >= krem) { d = 255 - 4 * lane - j; cd = c[j]; break; }
      acc += c[j];
    }
    const uint32_t hi = sel[1];
    const uint32_t nlo = lo + ((uint32_t)d << shift);
    const uint32_t nhi_raw = nlo + ((1u << shift) - 1u);
    sel[0] = nlo;
    sel[1] = (nhi_raw < nlo || nhi_raw > hi) ? hi : nhi_raw;
    sel[2] = (uint32_t)(krem - acc);
    sel[3] = (uint32_t)d;
    sel[4] = (uint32_t)cd;
  }
}

// Register-resident variant for articles of at most 1024 * KPT tokens: thread t holds keys
// t, t + 1024, ... (KPT of them), so every pass is register arithmetic plus LDS histogram
// updates, and the index-order compaction works on 64-key blocks (block b = round r, wave w covers
// positions 1024 r + 64 w .. +63) whose counts are scanned by one wave.
__device__ __noinline__ void topk_stream_body(const float *scores, const int32_t *geom, int64_t *keep,
                                                 float *sumsq);

template <int KPT>
__global__ __launch_bounds__(kTThreads, 1) void gate_topk_reg_kernel(const float *scores, const int32_t *geom,
                                                                     int64_t *keep, float *sumsq) {
  static_assert(KPT % 4 == 0, "bins are cached four per register");
  constexpr int NB = KPT * kTWaves;    // 64-key blocks
  constexpr int kCand = 4096;          // keys of the chosen value bin gathered into LDS
  __shared__ int hist[2][kTWaves][256];   // double-buffered: the next pass's copy is cleared early
  __shared__ int bgt[NB], beq[NB], bkeep0[NB], beq0[NB];
  __shared__ uint32_t cand[kCand];
  __shared__ int wofs[kTWaves];
  __shared__ uint32_t sel[5];             // lo, hi, k_rem, chosen bin, its count
  __shared__ uint32_t wmin[kTWaves], wmax[kTWaves];
  __shared__ float red[kTWaves];

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int32_t *gm = geom + 6 * blockIdx.x;
  const int64_t row_start = gm[0];
  const int seq_len = gm[1], s = gm[2], e = gm[3], kc = gm[4];
  const int64_t kept0 = gm[5];
  const int n = e - s;
  const float *sc = scores + row_start + s;
  // a sequence longer than the register capacity (the caller's max_article_len understated it)
  // takes the streaming path: the result never depends on the hint, only the speed does
  if (n > KPT * kTThreads) {
    topk_stream_body(scores, geom, keep, sumsq);
    return;
  }

  // keys in registers (all loads in flight); 0 marks a position past the article
  const brsrc_t srs = make_rsrc(sc, n > 0 ? (uint32_t)n * 4u : 0u);
  uint32_t key[KPT];
#pragma unroll
  for (int r = 0; r < KPT; ++r)
    key[r] = __builtin_amdgcn_raw_buffer_load_b32(srs, (uint32_t)(r * kTThreads + tid) * 4u, 0, 0);

  for (int i = tid; i < s; i += kTThreads) keep[kept0 + i] = i;
  for (int i = tid; i < seq_len - e; i += kTThreads) keep[kept0 + s + kc + i] = e + i;
  if (n <= 0 || kc <= 0) {
    if (tid == 0 && sumsq) sumsq[blockIdx.x] = 0.f;
    return;
  }
  for (int i = lane; i < 256; i += 64) hist[0][wave][i] = 0;

  float ss = 0.f;
  uint32_t kmin = 0xffffffffu, kmax = 0u;
#pragma unroll
  for (int r = 0; r < KPT; ++r) {
    const bool valid = r * kTThreads + tid < n;
    const float f = __builtin_bit_cast(float, key[r]);
    ss = valid ? fmaf(f, f, ss) : ss;
    key[r] = valid ? order_key(f) : 0u;
    kmin = min(kmin, valid ? key[r] : 0xffffffffu);
    kmax = max(kmax, key[r]);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    ss += __shfl_xor(ss, o);
    kmin = min(kmin, (uint32_t)__shfl_xor((int)kmin, o));
    kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, o));
  }
  if (lane == 0) { red[wave] = ss; wmin[wave] = kmin; wmax[wave] = kmax; }
  __syncthreads();
  if (tid == 0) {
    float t = 0.f;
    uint32_t lo = 0xffffffffu, hi = 0u;
    for (int w = 0; w < kTWaves; ++w) { t += red[w]; lo = min(lo, wmin[w]); hi = max(hi, wmax[w]); }
    if (sumsq) sumsq[blockIdx.x] = t;
    sel[0] = lo; sel[1] = hi; sel[2] = (uint32_t)kc;
  }
  __syncthreads();

  // First pass in value space: 256 equal-width bins over [min, max] of the scores spread typical
  // score distributions evenly (their order keys crowd into a few power-of-two bins, where the
  // histogram atomics of a wave would serialise).  The bin holding the kc-th largest score then
  // narrows the key range to that bin's own [min, max] key for the key-space passes below.
  // Skipped when the range is empty or not finite (infinities, NaN): the key passes alone are exact.
  int pb = 0;
  {
    const uint32_t lo = sel[0], hi = sel[1];
    const float vmin = key_value(lo), vmax = key_value(hi);
    const float inv = 256.f / (vmax - vmin);
    if (lo != hi && __builtin_isfinite(vmin) && __builtin_isfinite(vmax) && __builtin_isfinite(inv) && inv > 0.f) {
      for (int i = lane; i < 256; i += 64) hist[1][wave][i] = 0;
      uint32_t bins[KPT / 4];   // the bins, four per register, for the range pass below
#pragma unroll
      for (int r = 0; r < KPT; ++r) {
        const uint32_t u = key[r];
        // branch-free: a key past the article (0) decodes to NaN, converts to bin 0 and adds 0
        const int bin = value_bin(key_value(u), vmin, inv);
        atomicAdd(&hist[0][wave][bin], u != 0u ? 1 : 0);
        if (r % 4 == 0) bins[r / 4] = 0u;
        bins[r / 4] |= (uint32_t)bin << (8 * (r % 4));
      }
      __syncthreads();
      if (wave == 0) select_bin(hist[0], lane, sel, 0u, 0);
      __syncthreads();
      // the chosen bin: its key range, and (when it holds at most kCand keys) its keys gathered
      // into LDS so that the key-space passes below read a few LDS words instead of every key
      const uint32_t d = sel[3];
      const int nc = (int)sel[4];
      const bool gather = nc <= kCand;     // block-uniform
      auto in_bin = [&](int r) { return key[r] != 0u && ((bins[r / 4] >> (8 * (r % 4))) & 0xffu) == d; };
      int wcnt = 0;
      uint32_t bmin = 0xffffffffu, bmax = 0u;
#pragma unroll
      for (int r = 0; r < KPT; ++r) {
        const bool in = in_bin(r);
        bmin = in ? min(bmin, key[r]) : bmin;
        bmax = in ? max(bmax, key[r]) : bmax;
        if (gather) wcnt += __builtin_popcountll(__builtin_amdgcn_ballot_w64(in));
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        bmin = min(bmin, (uint32_t)__shfl_xor((int)bmin, o));
        bmax = max(bmax, (uint32_t)__shfl_xor((int)bmax, o));
      }
      if (lane == 0) { wmin[wave] = bmin; wmax[wave] = bmax; wofs[wave] = wcnt; }
      __syncthreads();
      if (tid == 0) {
        uint32_t a = 0xffffffffu, z = 0u;
        int o = 0;
        for (int w = 0; w < kTWaves; ++w) {
          a = min(a, wmin[w]);
          z = max(z, wmax[w]);
          const int c = wofs[w];
          wofs[w] = o;
          o += c;
        }
        sel[0] = a; sel[1] = z;
      }
      __syncthreads();
      if (gather) {
        int base = wofs[wave];
#pragma unroll
        for (int r = 0; r < KPT; ++r) {
          const bool in = in_bin(r);
          const uint64_t m = __builtin_amdgcn_ballot_w64(in);
          if (in) cand[base + lanes_below(m)] = key[r];
          base += __builtin_popcountll(m);
        }
        __syncthreads();
        // key-space passes over the gathered keys only, into one shared histogram per pass (few
        // keys: little contention; the bin search then reads 256 counters instead of 16 x 256)
        int cb = 1;
        while (true) {
          const uint32_t lo = sel[0], hi = sel[1];
          if (lo == hi) break;                             // block-uniform
          const uint32_t span = hi - lo;
          const int shift = span < 256u ? 0 : 32 - __builtin_clz(span >> 8);
          if (tid < 256) hist[cb ^ 1][0][tid] = 0;
          for (int i = tid; i < nc; i += kTThreads) {
            const uint32_t u = cand[i];
            if (u >= lo && u <= hi) atomicAdd(&hist[cb][0][(u - lo) >> shift], 1);
          }
          __syncthreads();
          if (wave == 0) select_bin<1>(hist[cb], lane, sel, lo, shift);
          __syncthreads();
          cb ^= 1;
        }
      }
      pb = 1;
    }
  }
  // Radix select of the kc-th largest key over the occupied key range [lo, hi]: each pass splits
  // the current range into at most 256 power-of-two-wide bins.  Windowing each pass to the
  // range still in play keeps the passes few.
  while (true) {
    const uint32_t lo = sel[0], hi = sel[1];
    if (lo == hi) break;                             // block-uniform
    const uint32_t span = hi - lo;
    const int shift = span < 256u ? 0 : 32 - __builtin_clz(span >> 8);   // span >> shift < 256
    for (int i = lane; i < 256; i += 64) hist[pb ^ 1][wave][i] = 0;     // next pass's copy
#pragma unroll
    for (int r = 0; r < KPT; ++r) {
      const uint32_t u = key[r];
      if (u != 0u && u >= lo && u <= hi) atomicAdd(&hist[pb][wave][(u - lo) >> shift], 1);
    }
    __syncthreads();
    if (wave == 0) select_bin(hist[pb], lane, sel, lo, shift);
    __syncthreads();
    pb ^= 1;
  }
  const uint32_t T = sel[0];
  const int k_eq = (int)sel[2];

  // per-block counts (block r*16 + w covers positions 1024 r + 64 w .. + 63: index order)
#pragma unroll
  for (int r = 0; r < KPT; ++r) {
    const uint64_t gtm = __builtin_amdgcn_ballot_w64(key[r] > T);
    const uint64_t eqm = __builtin_amdgcn_ballot_w64(key[r] == T);
    if (lane == 0) { bgt[r * kTWaves + wave] = (int)__builtin_popcountll(gtm); beq[r * kTWaves + wave] = (int)__builtin_popcountll(eqm); }
  }
  __syncthreads();
  if (wave == 0) {
    constexpr int PER = NB / 64;   // consecutive blocks per lane
    int eqv[PER], gtv[PER], ge = 0, gk = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) { eqv[j] = beq[lane * PER + j]; gtv[j] = bgt[lane * PER + j]; ge += eqv[j]; }
    int ie = ge;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) { const int y = __shfl_up(ie, o); if (lane >= o) ie += y; }
    int eb = ie - ge;
    int kl[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int te = min(eqv[j], max(0, k_eq - eb));
      beq0[lane * PER + j] = eb;
      eb += eqv[j];
      kl[j] = gtv[j] + te;
      gk += kl[j];
    }
    int ik = gk;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) { const int y = __shfl_up(ik, o); if (lane >= o) ik += y; }
    int kb = ik - gk;
#pragma unroll
    for (int j = 0; j < PER; ++j) { bkeep0[lane * PER + j] = kb; kb += kl[j]; }
  }
  __syncthreads();
  int e0[KPT], k0[KPT];
#pragma unroll
  for (int r = 0; r < KPT; ++r) { e0[r] = beq0[r * kTWaves + wave]; k0[r] = bkeep0[r * kTWaves + wave]; }
  int64_t *out = keep + kept0 + s;
#pragma unroll
  for (int r = 0; r < KPT; ++r) {
    const uint32_t u = key[r];
    const bool eq = u == T;
    const uint64_t eqm = __builtin_amdgcn_ballot_w64(eq);
    const bool take = u > T || (eq && e0[r] + lanes_below(eqm) < k_eq);
    const uint64_t tm = __builtin_amdgcn_ballot_w64(take);
    if (take) out[k0[r] + lanes_below(tm)] = s + r * kTThreads + tid;
  }
}

// Streaming variant for articles longer than the register-resident limit: the article is
// processed in chunks of 32 * 1024 keys (thread t holds keys c*32768 + 1024 r + t of chunk c, all
// 32 loads in flight), re-read from L2 on every pass — the same windowed radix select and
// 64-key-block compaction as gate_topk_reg_kernel, with the compaction's tie and output counts
// carried from chunk to chunk.
constexpr int kTChunk = 32;                 // keys per thread per chunk
constexpr int kTChunkKeys = kTChunk * kTThreads;

__device__ __noinline__ void topk_stream_body(const float *scores, const int32_t *geom, int64_t *keep,
                                                 float *sumsq) {
  constexpr int NB = kTChunk * kTWaves;   // 64-key blocks per chunk
  __shared__ int hist[2][kTWaves][256];
  __shared__ int bgt[NB], beq[NB], bkeep0[NB], beq0[NB];
  __shared__ uint32_t sel[5];             // lo, hi, k_rem (and the bin fields select_bin writes)
  __shared__ int carry[2];                // ties seen, rows kept: over the chunks before this one
  __shared__ uint32_t wmin[kTWaves], wmax[kTWaves];
  __shared__ float red[kTWaves];

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int32_t *gm = geom + 6 * blockIdx.x;
  const int64_t row_start = gm[0];
  const int seq_len = gm[1], s = gm[2], e = gm[3], kc = gm[4];
  const int64_t kept0 = gm[5];
  const int n = e - s;
  const float *sc = scores + row_start + s;

  for (int i = tid; i < s; i += kTThreads) keep[kept0 + i] = i;
  for (int i = tid; i < seq_len - e; i += kTThreads) keep[kept0 + s + kc + i] = e + i;
  if (n <= 0 || kc <= 0) {
    if (tid == 0 && sumsq) sumsq[blockIdx.x] = 0.f;
    return;
  }
  const int n_chunks = (n + kTChunkKeys - 1) / kTChunkKeys;
  const brsrc_t srs = make_rsrc(sc, (uint32_t)n * 4u);
  uint32_t key[kTChunk];
  // order keys of chunk c (0 past the article)
  auto load_chunk = [&](int c) {
#pragma unroll
    for (int r = 0; r < kTChunk; ++r)
      key[r] = __builtin_amdgcn_raw_buffer_load_b32(srs, (uint32_t)(c * kTChunkKeys + r * kTThreads + tid) * 4u, 0, 0);
#pragma unroll
    for (int r = 0; r < kTChunk; ++r) {
      const bool valid = c * kTChunkKeys + r * kTThreads + tid < n;
      key[r] = valid ? order_key(__builtin_bit_cast(float, key[r])) : 0u;
    }
  };

  float ss = 0.f;
  uint32_t kmin = 0xffffffffu, kmax = 0u;
  for (int c = 0; c < n_chunks; ++c) {
#pragma unroll
    for (int r = 0; r < kTChunk; ++r)
      key[r] = __builtin_amdgcn_raw_buffer_load_b32(srs, (uint32_t)(c * kTChunkKeys + r * kTThreads + tid) * 4u, 0, 0);
#pragma unroll
    for (int r = 0; r < kTChunk; ++r) {
      const bool valid = c * kTChunkKeys + r * kTThreads + tid < n;
      const float f = __builtin_bit_cast(float, key[r]);
      ss = valid ? fmaf(f, f, ss) : ss;
      const uint32_t u = valid ? order_key(f) : 0u;
      kmin = min(kmin, valid ? u : 0xffffffffu);
      kmax = max(kmax, u);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    ss += __shfl_xor(ss, o);
    kmin = min(kmin, (uint32_t)__shfl_xor((int)kmin, o));
    kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, o));
  }
  if (lane == 0) { red[wave] = ss; wmin[wave] = kmin; wmax[wave] = kmax; }
  for (int i = lane; i < 256; i += 64) hist[0][wave][i] = 0;
  __syncthreads();
  if (tid == 0) {
    float t = 0.f;
    uint32_t lo = 0xffffffffu, hi = 0u;
    for (int w = 0; w < kTWaves; ++w) { t += red[w]; lo = min(lo, wmin[w]); hi = max(hi, wmax[w]); }
    if (sumsq) sumsq[blockIdx.x] = t;
    sel[0] = lo; sel[1] = hi; sel[2] = (uint32_t)kc;
    carry[0] = 0; carry[1] = 0;
  }
  __syncthreads();

  int pb = 0;
  while (true) {
    const uint32_t lo = sel[0], hi = sel[1];
    if (lo == hi) break;                             // block-uniform
    const uint32_t span = hi - lo;
    const int shift = span < 256u ? 0 : 32 - __builtin_clz(span >> 8);
    for (int i = lane; i < 256; i += 64) hist[pb ^ 1][wave][i] = 0;
    for (int c = 0; c < n_chunks; ++c) {
      load_chunk(c);
#pragma unroll
      for (int r = 0; r < kTChunk; ++r) {
        const uint32_t u = key[r];
        if (u != 0u && u >= lo && u <= hi) atomicAdd(&hist[pb][wave][(u - lo) >> shift], 1);
      }
    }
    __syncthreads();
    if (wave == 0) {
      int c4[4], lt = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        int t = 0;
#pragma unroll
        for (int w = 0; w < kTWaves; ++w) t += hist[pb][w][255 - 4 * lane - j];
        c4[j] = t;
        lt += t;
      }
      int incl = lt;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o);
        if (lane >= o) incl += y;
      }
      const int before = incl - lt;
      const int krem = (int)sel[2];
      if (before < krem && krem <= incl) {
        int acc = before, d = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (acc + c4[j] >= krem) { d = 255 - 4 * lane - j; break; }
          acc += c4[j];
        }
        const uint32_t nlo = lo + ((uint32_t)d << shift);
        const uint32_t nhi_raw = nlo + ((1u << shift) - 1u);
        sel[0] = nlo;
        sel[1] = (nhi_raw < nlo || nhi_raw > hi) ? hi : nhi_raw;
        sel[2] = (uint32_t)(krem - acc);
      }
    }
    __syncthreads();
    pb ^= 1;
  }
  const uint32_t T = sel[0];
  const int k_eq = (int)sel[2];

  int64_t *out = keep + kept0 + s;
  for (int c = 0; c < n_chunks; ++c) {
    load_chunk(c);
#pragma unroll
    for (int r = 0; r < kTChunk; ++r) {
      const uint64_t gtm = __builtin_amdgcn_ballot_w64(key[r] > T);
      const uint64_t eqm = __builtin_amdgcn_ballot_w64(key[r] == T);
      if (lane == 0) { bgt[r * kTWaves + wave] = (int)__builtin_popcountll(gtm); beq[r * kTWaves + wave] = (int)__builtin_popcountll(eqm); }
    }
    __syncthreads();
    if (wave == 0) {
      constexpr int PER = NB / 64;
      const int ceq = carry[0], ckeep = carry[1];
      int eqv[PER], gtv[PER], ge = 0, gk = 0;
#pragma unroll
      for (int j = 0; j < PER; ++j) { eqv[j] = beq[lane * PER + j]; gtv[j] = bgt[lane * PER + j]; ge += eqv[j]; }
      int ie = ge;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) { const int y = __shfl_up(ie, o); if (lane >= o) ie += y; }
      int eb = ceq + ie - ge;
      int kl[PER];
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int te = min(eqv[j], max(0, k_eq - eb));
        beq0[lane * PER + j] = eb;
        eb += eqv[j];
        kl[j] = gtv[j] + te;
        gk += kl[j];
      }
      int ik = gk;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) { const int y = __shfl_up(ik, o); if (lane >= o) ik += y; }
      int kb = ckeep + ik - gk;
#pragma unroll
      for (int j = 0; j < PER; ++j) { bkeep0[lane * PER + j] = kb; kb += kl[j]; }
      if (lane == 63) { carry[0] = eb; carry[1] = kb; }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kTChunk; ++r) {
      const uint32_t u = key[r];
      const bool eq = u == T;
      const uint64_t eqm = __builtin_amdgcn_ballot_w64(eq);
      const int e0 = beq0[r * kTWaves + wave], k0 = bkeep0[r * kTWaves + wave];
      const bool take = u > T || (eq && e0 + lanes_below(eqm) < k_eq);
      const uint64_t tm = __builtin_amdgcn_ballot_w64(take);
      if (take) out[k0 + lanes_below(tm)] = s + c * kTChunkKeys + r * kTThreads + tid;
    }
    __syncthreads();   // the block tables are rewritten by the next chunk
  }
}

__global__ __launch_bounds__(kTThreads, 1) void gate_topk_stream_kernel(const float *scores, const int32_t *geom,
                                                                      int64_t *keep, float *sumsq) {
  topk_stream_body(scores, geom, keep, sumsq);
}

// ---------------------------------------------------------------------------------------------
// Pack.  Kept row j (0 <= j < total_kept) of sequence b reads source row
// row_start[b] + keep[j] of every stream and writes destination row j.
// ---------------------------------------------------------------------------------------------
constexpr int kPThreads = 256;
constexpr int kMaxStreams = 16;

struct PackArgs {
  tg_pack_stream st[kMaxStreams];
  int n_streams;
  const int64_t *keep;
  const int32_t *geom;    // (nseq, 6) as for top-K
  int nseq;
  int64_t total_kept;
  int64_t *pos_out;       // optional: kept positions (int64)
  const float *bias_src;  // optional: per-row score at row_start + pos (fp32)
  const float *sumsq;     // optional: per-sequence article sum of squares -> RMS normalisation
  float eps;
  float *bias_out;        // optional: gate bias of kept rows (0 on prefix / suffix rows)
  uint32_t *err;          // optional: set to kPackBadPosition when a kept position lies outside its sequence
};
constexpr uint32_t kPackBadPosition = 3u;

// ROWS kept rows per workgroup: 4 for large packs, 1 when there are too few rows to give every CU
// several workgroups (small K: the copy is latency-bound and wants as many rows in flight as possible)
// NT_LOAD: nontemporal loads (a gather far larger than the caches, whose source lines are not read
// again); otherwise nontemporal stores (the destination is written once, and keeping the source
// lines a smaller gather may find in the caches).  Either form moved a plain 430 MB copy faster
// than ordinary loads and stores; both at once did not.
template <int ROWS, bool NT_LOAD>
__global__ __launch_bounds__(kPThreads) void gate_pack_kernel(PackArgs a) {
  constexpr int kPRows = ROWS;
  __shared__ int64_t src_row[kPRows];
  __shared__ int64_t s_pos[kPRows];
  __shared__ int s_seq[kPRows];
  const int tid = threadIdx.x;
  const int64_t j0 = (int64_t)blockIdx.x * kPRows;
  if (tid < kPRows) {
    const int64_t j = j0 + tid;
    int64_t srow = -1, pos = 0;
    int sb = 0;
    if (j < a.total_kept) {
      int lo = 0, hi = a.nseq - 1;   // last sequence with kept_start <= j
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if ((int64_t)a.geom[6 * mid + 5] <= j) lo = mid; else hi = mid - 1;
      }
      sb = lo;
      pos = a.keep[j];
      // a position outside its sequence (a keep list that was never written) gathers nothing: the
      // row is skipped and the error word raised, instead of reading another sequence's rows or
      // past the source
      if (pos >= 0 && pos < (int64_t)a.geom[6 * lo + 1]) {
        srow = (int64_t)a.geom[6 * lo] + pos;
      } else if (a.err) {
        __hip_atomic_store(a.err, kPackBadPosition, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    src_row[tid] = srow;
    s_pos[tid] = pos;
    s_seq[tid] = sb;
  }
  // stream descriptors in LDS (indexed per lane below) and each stream's first 16-byte unit
  // within a row's units, all streams back to back
  __shared__ tg_pack_stream sst[kMaxStreams];
  __shared__ int upre[kMaxStreams + 1];
  if (tid < a.n_streams) sst[tid] = a.st[tid];
  if (tid == 0) {
    int acc = 0;
    for (int si = 0; si < a.n_streams; ++si) {
      upre[si] = acc;
      acc += (a.st[si].chunk_bytes >> 4) * a.st[si].n_chunks;
    }
    upre[a.n_streams] = acc;
  }
  __syncthreads();
  // every 16-byte unit of every stream of the workgroup's rows, flattened; each thread issues the
  // loads of up to kPBatch units before their stores, so that a row's streams are in flight
  // together instead of one stream's latency after another.  Six per thread measured best: a
  // hidden row and two layers' K/V (768 units) make 4-row workgroups two full rounds of 1536 (with
  // 8, a full round and a half-empty one) and keep fewer registers live (ragged8 select + pack 105
  // -> 101 us, 32k K=2000 24.9 -> 24.5 us; 3, 4 and 12 measured slower)
  constexpr int kPBatch = 6;
  const int U = upre[a.n_streams];
  const int total = U * kPRows;
  for (int w0 = tid; w0 < total; w0 += kPBatch * kPThreads) {
    u32x4 v[kPBatch];
    char *dst[kPBatch];
#pragma unroll
    for (int k = 0; k < kPBatch; ++k) {
      const int w = w0 + k * kPThreads;
      dst[k] = nullptr;
      if (w < total) {
        const int rr = w / U, uu = w % U;
        const int64_t srow = src_row[rr];
        if (srow >= 0) {
          int si = 0;
          while (uu >= upre[si + 1]) ++si;
          const tg_pack_stream &st = sst[si];
          const int upc = st.chunk_bytes >> 4;
          const int u = uu - upre[si];
          const int ch = u / upc, cu = u % upc;
          const char *src = static_cast<const char *>(st.src) + srow * st.src_row_stride +
                            (int64_t)ch * st.src_chunk_stride + 16 * cu;
          if constexpr (NT_LOAD)
            v[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(src));
          else
            v[k] = *reinterpret_cast<const u32x4 *>(src);
          const int64_t drow = j0 + rr + (int64_t)s_seq[rr] * st.dst_seq_gap;
          dst[k] = static_cast<char *>(st.dst) + drow * st.dst_row_stride + (int64_t)ch * st.chunk_bytes + 16 * cu;
        }
      }
    }
#pragma unroll
    for (int k = 0; k < kPBatch; ++k)
      if (dst[k]) {
        if constexpr (NT_LOAD)
          *reinterpret_cast<u32x4 *>(dst[k]) = v[k];
        else
          __builtin_nontemporal_store(v[k], reinterpret_cast<u32x4 *>(dst[k]));
      }
  }
  // positions and gate bias of the rows (after this thread's share of the copy is issued)
  if (tid >= kPThreads - kPRows) {
    const int r = tid - (kPThreads - kPRows);
    const int64_t j = j0 + r, srow = src_row[r], pos = s_pos[r];
    if (srow >= 0) {
      if (a.pos_out) a.pos_out[j] = pos;
      if (a.bias_out) {
        const int lo = s_seq[r];
        const int s = a.geom[6 * lo + 2], e = a.geom[6 * lo + 3];
        float bv = 0.f;
        if (pos >= s && pos < e && a.bias_src) {
          bv = a.bias_src[srow];
          if (a.sumsq) bv *= rsqrtf(a.sumsq[lo] / (float)(e - s) + a.eps);
        }
        a.bias_out[j] = bv;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Threshold selection (the reference's _select_threshold, gate_forward.py:102-125, on the selection
// value of aggregate, e2e_gate_module.py:387-399).  One workgroup per sequence:
//   1. the state span's mean square in fp64, rounded once to fp32 (the correctly rounded mean),
//      inv = fp32(1 / sqrt(fp32(mean + eps))) (fp64 square root and division, rounded once);
//   2. agg_j = sum over heads, in head order, of fp32(fp32(bn_j * sp_h) * w) with
//      bn_j = fp32(gain * fp32(raw_j * inv)), w = fp32(1 / H) (agg_j = bn_j * sp_0 when H = 1):
//      every step a separately rounded fp32 operation, as the reference's tensor ops are;
//      a token passes when agg_j >= b_star (the caller's exact fp32 form of sigmoid(agg_j) >= tau,
//      NaN never passes); count = passing tokens;
//   3. sel_j = passing ? 1 : 0 when count > 0, else agg_j: the top-count (top-1) selection over sel
//      is then exactly the passing set (the argmax fallback, ties and NaN ranked as top-K ranks them).
// ---------------------------------------------------------------------------------------------
constexpr int kThThreads = 512;
constexpr int kThMaxHeads = 64;

struct ThArgs {
  const float *scores;
  const int32_t *geom;
  float sp[kThMaxHeads];   // softplus(gate_scale[0, h]) of the first Phase-2 layer
  int n_heads;
  float gain, eps, b_star;
  float *agg, *sel;
  int32_t *counts;
  float *sumsq;
};

__device__ __forceinline__ float th_agg(const ThArgs &a, float raw, float inv, float w) {
  const float bn = __fmul_rn(a.gain, __fmul_rn(raw, inv));
  if (a.n_heads == 1) return __fmul_rn(bn, a.sp[0]);
  float acc = 0.f;
  for (int h = 0; h < a.n_heads; ++h) acc = __fadd_rn(acc, __fmul_rn(__fmul_rn(bn, a.sp[h]), w));
  return acc;
}

__global__ __launch_bounds__(kThThreads) void gate_threshold_kernel(ThArgs a) {
  __shared__ double s_d[kThThreads / 64];
  __shared__ int s_c[kThThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int *gm = a.geom + 6 * blockIdx.x;
  const int64_t r0 = (int64_t)gm[0] + gm[2];
  const int n = gm[3] - gm[2];
  const float *x = a.scores + r0;
  double ss = 0.0;
  for (int i = tid; i < n; i += kThThreads) {
    const double v = x[i];
    ss += v * v;
  }
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  if (lane == 0) s_d[wv] = ss;
  __syncthreads();
  double tot = 0.0;
  for (int w = 0; w < kThThreads / 64; ++w) tot += s_d[w];
  const float mean = n > 0 ? (float)(tot / (double)n) : 0.f;
  const float inv = (float)(1.0 / sqrt((double)__fadd_rn(mean, a.eps)));
  const float w = (float)(1.0 / (double)a.n_heads);
  int cnt = 0;
  for (int i = tid; i < n; i += kThThreads) {
    const float g = th_agg(a, x[i], inv, w);
    a.agg[r0 + i] = g;
    cnt += g >= a.b_star ? 1 : 0;
  }
  for (int o = 32; o > 0; o >>= 1) cnt += __shfl_xor(cnt, o);
  if (lane == 0) s_c[wv] = cnt;
  __syncthreads();
  int count = 0;
  for (int k = 0; k < kThThreads / 64; ++k) count += s_c[k];
  for (int i = tid; i < n; i += kThThreads) {
    const float g = th_agg(a, x[i], inv, w);
    a.sel[r0 + i] = count > 0 ? (g >= a.b_star ? 1.f : 0.f) : g;
  }
  if (tid == 0) {
    a.counts[blockIdx.x] = count;
    if (a.sumsq) a.sumsq[blockIdx.x] = (float)tot;
  }
}

}  // namespace
}  // namespace tg

using namespace tg;

namespace tg {
namespace {
int score_launch(const void *x, int64_t n_rows, int64_t x_row_stride, int32_t d_in, int32_t d_hidden, const void *w1,
                 int64_t w_rs, int64_t w_ss, const float *b1, const float *w2, float b2, float *scores,
                 hipStream_t stream) {
  TG_CHECK(d_in == kDin && d_hidden == kDh, "the scoring head is Linear(2048->256) -> SiLU -> Linear(256->1) "
                                            "(got %d -> %d)", d_in, d_hidden);
  TG_CHECK(x && w1 && b1 && w2 && scores, "null pointer");
  TG_CHECK((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(w1) & 15) == 0 &&
               x_row_stride % 8 == 0,
           "x and w1 must be 16-byte aligned with a row stride that is a multiple of 8");
  TG_CHECK(n_rows >= 0, "negative size");
  if (n_rows == 0) return 0;
  TG_CHECK((int64_t)(kSRowsMax + 1) * x_row_stride * 2 < (1ll << 32) - 1024,
           "a 256-row block of x must span less than 4 GiB");
  ScoreArgs a{static_cast<const bf16_t *>(x), x_row_stride, n_rows, static_cast<const bf16_t *>(w1), w_rs, w_ss,
              b1, w2, b2, scores};
  // 256-row workgroups (each W1 byte streamed through LDS serves twice the rows) once they still
  // give every CU two of them; 128-row ones below that, where a grid of the larger ones would
  // leave CUs idle
  const bool wide = (n_rows + 255) / 256 >= 2 * (int64_t)device_cus();
  const int rows = wide ? 256 : 128;
  const int64_t nb = (n_rows + rows - 1) / rows;
  TG_CHECK(nb < (1ll << 31), "grid too large");
  if (wide)
    hipLaunchKernelGGL((gate_score_kernel<256, 4>), dim3((unsigned)nb), dim3(kSThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((gate_score_kernel<128, 6>), dim3((unsigned)nb), dim3(kSThreads), 0, stream, a);
  TG_HIP_CHECK(hipPeekAtLastError());
  return 0;
}
}  // namespace
}  // namespace tg

extern "C" int tg_gate_score_mlp(const void *x, int64_t n_rows, int64_t x_row_stride, int32_t d_in,
                                 int32_t d_hidden, const void *w1, const float *b1, const float *w2, float b2,
                                 float *scores, hipStream_t stream) {
  clear_error();
  return score_launch(x, n_rows, x_row_stride, d_in, d_hidden, w1, kDin, kSK * 2, b1, w2, b2, scores, stream);
}

extern "C" int tg_gate_score_mlp_ktiled(const void *x, int64_t n_rows, int64_t x_row_stride, int32_t d_in,
                                        int32_t d_hidden, const void *w1_ktiled, const float *b1, const float *w2,
                                        float b2, float *scores, hipStream_t stream) {
  clear_error();
  return score_launch(x, n_rows, x_row_stride, d_in, d_hidden, w1_ktiled, kSK, (int64_t)kDh * kSK * 2, b1, w2, b2,
                      scores, stream);
}

extern "C" int tg_gate_topk_keep(const float *scores, const int32_t *geom, int32_t num_seqs,
                                 int32_t max_article_len, int64_t *keep, float *sumsq, hipStream_t stream) {
  clear_error();
  TG_CHECK(scores && geom && keep, "null pointer");
  TG_CHECK(num_seqs >= 0 && max_article_len >= 0, "negative size");
  if (num_seqs == 0) return 0;
  const dim3 grid(num_seqs), block(kTThreads);
  if (max_article_len <= 32 * kTThreads)
    hipLaunchKernelGGL(gate_topk_reg_kernel<32>, grid, block, 0, stream, scores, geom, keep, sumsq);
  else if (max_article_len <= 64 * kTThreads)
    hipLaunchKernelGGL(gate_topk_reg_kernel<64>, grid, block, 0, stream, scores, geom, keep, sumsq);
  else
    hipLaunchKernelGGL(gate_topk_stream_kernel, grid, block, 0, stream, scores, geom, keep, sumsq);
  TG_HIP_CHECK(hipPeekAtLastError());
  return 0;
}

namespace tg {
// The pack behind tg_gate_pack and tg_gate_select_pack (err: the selection's error word, or NULL).
int gate_pack_launch(const tg_pack_stream *streams, int32_t n_streams, const int64_t *keep, const int32_t *geom,
                     int32_t num_seqs, int64_t total_kept, int64_t *positions_out, const float *bias_src,
                     const float *sumsq, float rms_eps, float *bias_out, uint32_t *err, hipStream_t stream) {
  TG_CHECK(n_streams >= 0 && n_streams <= kMaxStreams, "at most %d streams", kMaxStreams);
  TG_CHECK(n_streams == 0 || streams != nullptr, "null streams");
  TG_CHECK(keep && geom, "null pointer");
  TG_CHECK(num_seqs >= 0 && total_kept >= 0, "negative size");
  if (num_seqs == 0 || total_kept == 0) return 0;
  PackArgs a{};
  for (int i = 0; i < n_streams; ++i) {
    const tg_pack_stream &s = streams[i];
    TG_CHECK(s.src && s.dst, "stream %d: null pointer", i);
    TG_CHECK(s.chunk_bytes > 0 && s.chunk_bytes % 16 == 0 && s.n_chunks > 0,
             "stream %d: chunks must be positive multiples of 16 bytes", i);
    TG_CHECK(((reinterpret_cast<uintptr_t>(s.src) | reinterpret_cast<uintptr_t>(s.dst) | s.src_row_stride |
               s.dst_row_stride | s.src_chunk_stride) & 15) == 0,
             "stream %d: pointers and strides must be 16-byte aligned", i);
    TG_CHECK(s.dst_row_stride >= (int64_t)s.chunk_bytes * s.n_chunks, "stream %d: destination rows overlap", i);
    TG_CHECK(s.dst_seq_gap >= 0, "stream %d: negative destination gap", i);
    a.st[i] = s;
  }
  a.n_streams = n_streams;
  a.keep = keep;
  a.geom = geom;
  a.nseq = num_seqs;
  a.total_kept = total_kept;
  a.pos_out = positions_out;
  a.bias_src = bias_src;
  a.sumsq = sumsq;
  a.eps = rms_eps;
  a.bias_out = bias_out;
  a.err = err;
  TG_CHECK(total_kept < (1ll << 31), "grid too large");
  int64_t row_bytes = 0;
  for (int i = 0; i < n_streams; ++i) row_bytes += (int64_t)streams[i].chunk_bytes * streams[i].n_chunks;
  // nontemporal loads once the gather outgrows a quarter of the 256 MB last-level cache (the
  // ragged 8 x 16k-128k batch: 214 MB, -11 % against ordinary loads); nontemporal stores below
  // (32k at K=2000: 29 MB, -3.5 %, where nontemporal loads were 9 % slower)
  const bool nt_load = total_kept * row_bytes >= (64ll << 20);
  if (total_kept < 16 * 256) {
    if (nt_load)
      hipLaunchKernelGGL((gate_pack_kernel<1, true>), dim3((unsigned)total_kept), dim3(kPThreads), 0, stream, a);
    else
      hipLaunchKernelGGL((gate_pack_kernel<1, false>), dim3((unsigned)total_kept), dim3(kPThreads), 0, stream, a);
  } else {
    const dim3 grid((unsigned)((total_kept + 3) / 4));
    if (nt_load)
      hipLaunchKernelGGL((gate_pack_kernel<4, true>), grid, dim3(kPThreads), 0, stream, a);
    else
      hipLaunchKernelGGL((gate_pack_kernel<4, false>), grid, dim3(kPThreads), 0, stream, a);
  }
  TG_HIP_CHECK(hipPeekAtLastError());
  return 0;
}
}  // namespace tg

extern "C" int tg_gate_pack(const tg_pack_stream *streams, int32_t n_streams, const int64_t *keep,
                            const int32_t *geom, int32_t num_seqs, int64_t total_kept, int64_t *positions_out,
                            const float *bias_src, const float *sumsq, float rms_eps, float *bias_out,
                            hipStream_t stream) {
  clear_error();
  return gate_pack_launch(streams, n_streams, keep, geom, num_seqs, total_kept, positions_out, bias_src, sumsq,
                          rms_eps, bias_out, nullptr, stream);
}

extern "C" int tg_gate_threshold_select(const float *scores, const int32_t *geom, int32_t num_seqs,
                                        const float *head_scale, int32_t n_heads, float gain, float rms_eps,
                                        float b_star, float *agg_out, float *select_out, int32_t *counts,
                                        float *sumsq, hipStream_t stream) {
  clear_error();
  TG_CHECK(scores && geom && head_scale && agg_out && select_out && counts, "null pointer");
  TG_CHECK(num_seqs >= 0, "negative size");
  TG_CHECK(n_heads >= 1 && n_heads <= kThMaxHeads, "n_heads must be 1 .. %d (got %d)", kThMaxHeads, n_heads);
  if (num_seqs == 0) return 0;
  ThArgs a{};
  a.scores = scores;
  a.geom = geom;
  for (int h = 0; h < n_heads; ++h) a.sp[h] = head_scale[h];
  a.n_heads = n_heads;
  a.gain = gain;
  a.eps = rms_eps;
  a.b_star = b_star;
  a.agg = agg_out;
  a.sel = select_out;
  a.counts = counts;
  a.sumsq = sumsq;
  hipLaunchKernelGGL(gate_threshold_kernel, dim3(num_seqs), dim3(kThThreads), 0, stream, a);
  TG_HIP_CHECK(hipPeekAtLastError());
  return 0;
}
