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
// This build packs the kept rows of all sequences back to back (varlen / cu_seqlens layout)
// instead of padding to the longest, and breaks score ties by the lower index.
//
// Kernels:
//   gate_score_kernel  — s = w2 . silu(W1 x + b1) + b2 for every row of a packed (rows, 2048)
//                        bf16 matrix (128 rows per workgroup; W1 x on bf16 MFMA, fp32 epilogue);
//   gate_topk_kernel   — one workgroup per sequence: order-preserving uint32 keys, 4-pass 8-bit
//                        radix select of the K_c-th largest key (keys LDS-resident when the article
//                        fits, 32768 keys), then an index-order compaction (block scans) that keeps
//                        keys above the threshold and the lowest-index ties, writing ascending
//                        positions; also the article's sum of squared scores;
//   gate_pack_kernel   — one launch gathers every kept row for any number of row streams (hidden
//                        states, per-layer K and V, head-chunked rows) in 16-byte units, plus the
//                        kept positions and the kept rows' gate bias.
#include "tg_common.h"
#include "../../include/tokengate_hip.h"

namespace tg {
namespace {

// ---------------------------------------------------------------------------------------------
// Scoring head: s = w2 . silu(W1 x + b1) + b2, x in R^2048 (bf16), W1 (256 x 2048) bf16.
// Workgroup: 4 waves, 128 rows; wave w owns rows 32w..32w+31 and all 256 hidden units
// (8 column blocks of 32).  K loop over the 2048 inputs in steps of 32, double-buffered through
// LDS: X tile 128 x 32 (8 KiB), W1 tile 256 x 32 (16 KiB).  Accumulators are C^T blocks
// (hidden unit = MFMA row, token = column) so each lane ends with one token's 16 hidden units
// per block and the SiLU . w2 reduction is in-lane plus one cross-half exchange.
// ---------------------------------------------------------------------------------------------
constexpr int kDin = 2048;
constexpr int kDh = 256;
constexpr int kSRows = 128;
constexpr int kSK = 32;
constexpr int kSThreads = 256;

struct ScoreArgs {
  const bf16_t *x;
  int64_t x_rs;        // row stride (elements)
  int64_t n_rows;
  const bf16_t *w1;    // (256, 2048) row-major
  const float *b1, *w2;
  float b2;
  float *out;
};

__global__ __launch_bounds__(kSThreads, 1) void gate_score_kernel(ScoreArgs a) {
  // X tile: 128 rows x 64 B, W tile: 256 rows x 64 B; 16-byte chunks, 4 per row, XOR-swizzled
  __shared__ __attribute__((aligned(1024))) char xs[2][kSRows * kSK * 2];
  __shared__ __attribute__((aligned(1024))) char ws[2][kDh * kSK * 2];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lq = lane & 31, g = lane >> 5;
  const int64_t r0 = (int64_t)blockIdx.x * kSRows;

  const int64_t rows_here = min((int64_t)kSRows, a.n_rows - r0);
  const brsrc_t xrs = make_rsrc(a.x + r0 * a.x_rs, (uint32_t)(((rows_here - 1) * a.x_rs + kDin) * 2));
  const brsrc_t wrs = make_rsrc(a.w1, (uint32_t)(kDh * kDin * 2));
  // DMA slots: X tile = 512 chunks (2 per thread... 256 threads x 16 B = 4 KiB per issue): 2 issues;
  // W tile = 1024 chunks: 4 issues.  LDS row r, physical chunk p holds logical chunk p ^ ((r>>1)&3).
  auto issue = [&](int kstep, int buf) {
    const int k0 = kstep * kSK;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int slot = (wave * 2 + it) * 64 + lane;        // 0..511
      const int r = slot >> 2, p = slot & 3;
      const int c = p ^ ((r >> 1) & 3);
      dma16(xrs, xs[buf] + (wave * 2 + it) * 1024, (uint32_t)((r * a.x_rs + k0 + 8 * c) * 2));
    }
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int slot = (wave * 4 + it) * 64 + lane;        // 0..1023
      const int r = slot >> 2, p = slot & 3;
      const int c = p ^ ((r >> 1) & 3);
      dma16(wrs, ws[buf] + (wave * 4 + it) * 1024, (uint32_t)((r * kDin + k0 + 8 * c) * 2));
    }
  };

  f32x16 acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[j][v] = 0.f;

  constexpr int nk = kDin / kSK;
  issue(0, 0);
  for (int ks = 0; ks < nk; ++ks) {
    const int buf = ks & 1;
    wait_all_mem();
    __syncthreads();
    if (ks + 1 < nk) issue(ks + 1, buf ^ 1);
    // B operand: X^T column (token) = lane's row 32*wave + lq; k = 16*s + 8g + j
    const int xr = 32 * wave + lq;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int c = 2 * s + g;
      const bf16x8 xb = lds_load16(xs[buf], xr * 64 + (((uint32_t)c ^ ((xr >> 1) & 3)) << 4));
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int wr = 32 * j + lq;   // A operand: W1 row (hidden unit)
        const bf16x8 wa = lds_load16(ws[buf], wr * 64 + (((uint32_t)c ^ ((wr >> 1) & 3)) << 4));
        acc[j] = mfma32(wa, xb, acc[j]);
      }
    }
  }
  // epilogue: lane holds token (32*wave + lq), hidden units 32j + 8(v/4) + 4g + v%4
  float part = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int u = 32 * j + 8 * (v >> 2) + 4 * g + (v & 3);
      const float h = acc[j][v] + a.b1[u];
      const float sl = h / (1.f + __expf(-h));
      part = fmaf(sl, a.w2[u], part);
    }
  const float tot = pair_sum(part);
  const int64_t row = r0 + 32 * wave + lq;
  if (g == 0 && row < a.n_rows) a.out[row] = tot + a.b2;
}

// ---------------------------------------------------------------------------------------------
// Top-K keep list.  Per sequence b the geometry row (int32 x 6) is
//   [row_start, seq_len, art_start, art_end, k_clamped, kept_start]
// with scores of the sequence's rows at scores[row_start + i]; the kept positions (within the
// sequence, ascending) go to keep[kept_start .. kept_start + art_start + k_clamped + seq_len - art_end).
// ---------------------------------------------------------------------------------------------
constexpr int kTThreads = 1024;
constexpr int kTWaves = kTThreads / 64;
constexpr int kTLdsKeys = 32768;

// float -> uint32 whose unsigned order is the float order; -0 == +0; NaN above +inf.
__device__ __forceinline__ uint32_t order_key(float f) {
  if (f != f) return 0xffffffffu;
  if (f == 0.f) f = 0.f;
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Block-wide exclusive scan of one int per thread; returns the exclusive prefix, total in *tot.
__device__ int block_exclusive_scan(int x, int *scratch, int *tot) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int incl = x;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  if (lane == 63) scratch[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    int w = lane < kTWaves ? scratch[lane] : 0;
    int wi = w;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(wi, o);
      if (lane >= o) wi += y;
    }
    if (lane < kTWaves) scratch[32 + lane] = wi - w;
    if (lane == kTWaves - 1) scratch[64] = wi;
  }
  __syncthreads();
  const int res = scratch[32 + wave] + incl - x;
  *tot = scratch[64];
  __syncthreads();
  return res;
}

template <bool IN_LDS>
__global__ __launch_bounds__(kTThreads, 1) void gate_topk_kernel(const float *scores, const int32_t *geom,
                                                                 int64_t *keep, float *sumsq) {
  __shared__ uint32_t keys_lds[IN_LDS ? kTLdsKeys : 1];
  __shared__ int hist[kTWaves][256];
  __shared__ int htot[256];
  __shared__ int scratch[96];
  __shared__ uint32_t sel[4];   // prefix, k_rem
  __shared__ float red[kTWaves];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int32_t *gm = geom + 6 * blockIdx.x;
  const int64_t row_start = gm[0];
  const int seq_len = gm[1], s = gm[2], e = gm[3], kc = gm[4];
  const int64_t kept0 = gm[5];
  const int n = e - s;
  const float *sc = scores + row_start + s;

  // prefix and suffix positions
  for (int i = tid; i < s; i += kTThreads) keep[kept0 + i] = i;
  for (int i = tid; i < seq_len - e; i += kTThreads) keep[kept0 + s + kc + i] = e + i;
  if (n <= 0 || kc <= 0) {
    if (tid == 0 && sumsq) sumsq[blockIdx.x] = 0.f;
    return;
  }

  // keys (and the article's sum of squares)
  float ss = 0.f;
  if constexpr (IN_LDS) {
    for (int i = tid; i < n; i += kTThreads) {
      const float f = sc[i];
      ss = fmaf(f, f, ss);
      keys_lds[i] = order_key(f);
    }
  } else {
    for (int i = tid; i < n; i += kTThreads) {
      const float f = sc[i];
      ss = fmaf(f, f, ss);
    }
  }
  auto key_at = [&](int i) -> uint32_t {
    if constexpr (IN_LDS) return keys_lds[i];
    else return order_key(sc[i]);
  };
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  if (lane == 0) red[wave] = ss;
  if (tid == 0) { sel[0] = 0u; sel[1] = (uint32_t)kc; }
  __syncthreads();
  if (tid == 0 && sumsq) {
    float t = 0.f;
    for (int w = 0; w < kTWaves; ++w) t += red[w];
    sumsq[blockIdx.x] = t;
  }

  // radix select of the kc-th largest key, 8 bits per pass from the top
  uint32_t mask = 0u;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = lane; i < 256; i += 64) hist[wave][i] = 0;
    __syncthreads();
    const uint32_t prefix = sel[0];
    for (int i = tid; i < n; i += kTThreads) {
      const uint32_t u = key_at(i);
      if ((u & mask) == prefix) atomicAdd(&hist[wave][(u >> shift) & 255u], 1);
    }
    __syncthreads();
    if (tid < 256) {
      int t = 0;
      for (int w = 0; w < kTWaves; ++w) t += hist[w][tid];
      htot[tid] = t;
    }
    __syncthreads();
    if (wave == 0) {
      // lane l owns digits 255-4l .. 252-4l (descending)
      int c[4], lt = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) { c[j] = htot[255 - 4 * lane - j]; lt += c[j]; }
      int incl = lt;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o);
        if (lane >= o) incl += y;
      }
      const int before = incl - lt;
      const int krem = (int)sel[1];
      if (before < krem && krem <= incl) {
        int acc = before, d = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (acc + c[j] >= krem) { d = 255 - 4 * lane - j; break; }
          acc += c[j];
        }
        sel[0] = prefix | ((uint32_t)d << shift);
        sel[1] = (uint32_t)(krem - acc);
      }
    }
    mask |= 255u << shift;
    __syncthreads();
  }
  const uint32_t T = sel[0];
  const int k_eq = (int)sel[1];   // ties at T to keep (lowest indices first)

  // index-order compaction: each thread owns a contiguous segment
  const int seg = (n + kTThreads - 1) / kTThreads;
  const int i0 = min(n, tid * seg), i1 = min(n, i0 + seg);
  int n_eq = 0;
  for (int i = i0; i < i1; ++i) n_eq += key_at(i) == T;
  int tot;
  const int eq_before = block_exclusive_scan(n_eq, scratch, &tot);
  int n_keep = 0, r = eq_before;
  for (int i = i0; i < i1; ++i) {
    const uint32_t u = key_at(i);
    if (u > T) ++n_keep;
    else if (u == T) { n_keep += r < k_eq; ++r; }
  }
  const int pos0 = block_exclusive_scan(n_keep, scratch, &tot);
  int64_t *out = keep + kept0 + s;
  int p = pos0;
  r = eq_before;
  for (int i = i0; i < i1; ++i) {
    const uint32_t u = key_at(i);
    bool take = u > T;
    if (u == T) { take = r < k_eq; ++r; }
    if (take) out[p++] = s + i;
  }
}

// ---------------------------------------------------------------------------------------------
// Pack.  Kept row j (0 <= j < total_kept) of sequence b reads source row
// row_start[b] + keep[j] of every stream and writes destination row j.
// ---------------------------------------------------------------------------------------------
constexpr int kPThreads = 256;
constexpr int kPRows = 8;     // kept rows per workgroup
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
};

__global__ __launch_bounds__(kPThreads) void gate_pack_kernel(PackArgs a) {
  __shared__ int64_t src_row[kPRows];
  __shared__ int s_seq[kPRows];
  const int tid = threadIdx.x;
  const int64_t j0 = (int64_t)blockIdx.x * kPRows;
  if (tid < kPRows) {
    const int64_t j = j0 + tid;
    int64_t srow = -1;
    int sb = 0;
    if (j < a.total_kept) {
      int lo = 0, hi = a.nseq - 1;   // last sequence with kept_start <= j
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if ((int64_t)a.geom[6 * mid + 5] <= j) lo = mid; else hi = mid - 1;
      }
      sb = lo;
      const int64_t pos = a.keep[j];
      srow = (int64_t)a.geom[6 * lo] + pos;
      if (a.pos_out) a.pos_out[j] = pos;
      if (a.bias_out) {
        const int s = a.geom[6 * lo + 2], e = a.geom[6 * lo + 3];
        float bv = 0.f;
        if (pos >= s && pos < e && a.bias_src) {
          bv = a.bias_src[srow];
          if (a.sumsq) bv *= rsqrtf(a.sumsq[lo] / (float)(e - s) + a.eps);
        }
        a.bias_out[j] = bv;
      }
    }
    src_row[tid] = srow;
    s_seq[tid] = sb;
  }
  __syncthreads();
  for (int si = 0; si < a.n_streams; ++si) {
    const tg_pack_stream st = a.st[si];
    const int units_per_chunk = st.chunk_bytes >> 4;
    const int units = units_per_chunk * st.n_chunks;
    for (int w = tid; w < units * kPRows; w += kPThreads) {
      const int rr = w / units, u = w % units;
      const int64_t srow = src_row[rr];
      if (srow < 0) continue;
      const int ch = u / units_per_chunk, cu = u % units_per_chunk;
      const char *src = static_cast<const char *>(st.src) + srow * st.src_row_stride +
                        (int64_t)ch * st.src_chunk_stride + 16 * cu;
      char *dst = static_cast<char *>(st.dst) + (j0 + rr) * st.dst_row_stride +
                  (int64_t)ch * st.chunk_bytes + 16 * cu;
      *reinterpret_cast<u32x4 *>(dst) = *reinterpret_cast<const u32x4 *>(src);
    }
  }
}

}  // namespace
}  // namespace tg

using namespace tg;

extern "C" int tg_gate_score_mlp(const void *x, int64_t n_rows, int64_t x_row_stride, int32_t d_in,
                                 int32_t d_hidden, const void *w1, const float *b1, const float *w2, float b2,
                                 float *scores, hipStream_t stream) {
  clear_error();
  TG_CHECK(d_in == kDin && d_hidden == kDh, "the scoring head is Linear(2048->256) -> SiLU -> Linear(256->1) "
                                            "(got %d -> %d)", d_in, d_hidden);
  TG_CHECK(x && w1 && b1 && w2 && scores, "null pointer");
  TG_CHECK((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(w1) & 15) == 0 &&
               x_row_stride % 8 == 0,
           "x and w1 must be 16-byte aligned with a row stride that is a multiple of 8");
  TG_CHECK(n_rows >= 0, "negative size");
  if (n_rows == 0) return 0;
  TG_CHECK((int64_t)(kSRows + 1) * x_row_stride * 2 < (1ll << 32) - 1024,
           "a 128-row block of x must span less than 4 GiB");
  ScoreArgs a{static_cast<const bf16_t *>(x), x_row_stride, n_rows, static_cast<const bf16_t *>(w1), b1, w2, b2,
              scores};
  const int64_t nb = (n_rows + kSRows - 1) / kSRows;
  TG_CHECK(nb < (1ll << 31), "grid too large");
  hipLaunchKernelGGL(gate_score_kernel, dim3((unsigned)nb), dim3(kSThreads), 0, stream, a);
  TG_HIP_CHECK(hipPeekAtLastError());
  return 0;
}

extern "C" int tg_gate_topk_keep(const float *scores, const int32_t *geom, int32_t num_seqs,
                                 int32_t max_article_len, int64_t *keep, float *sumsq, hipStream_t stream) {
  clear_error();
  TG_CHECK(scores && geom && keep, "null pointer");
  TG_CHECK(num_seqs >= 0 && max_article_len >= 0, "negative size");
  if (num_seqs == 0) return 0;
  if (max_article_len <= kTLdsKeys)
    hipLaunchKernelGGL(gate_topk_kernel<true>, dim3(num_seqs), dim3(kTThreads), 0, stream, scores, geom, keep, sumsq);
  else
    hipLaunchKernelGGL(gate_topk_kernel<false>, dim3(num_seqs), dim3(kTThreads), 0, stream, scores, geom, keep,
                       sumsq);
  TG_HIP_CHECK(hipPeekAtLastError());
  return 0;
}

extern "C" int tg_gate_pack(const tg_pack_stream *streams, int32_t n_streams, const int64_t *keep,
                            const int32_t *geom, int32_t num_seqs, int64_t total_kept, int64_t *positions_out,
                            const float *bias_src, const float *sumsq, float rms_eps, float *bias_out,
                            hipStream_t stream) {
  clear_error();
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
  const int64_t nb = (total_kept + kPRows - 1) / kPRows;
  TG_CHECK(nb < (1ll << 31), "grid too large");
  hipLaunchKernelGGL(gate_pack_kernel, dim3((unsigned)nb), dim3(kPThreads), 0, stream, a);
  TG_HIP_CHECK(hipPeekAtLastError());
  return 0;
}
