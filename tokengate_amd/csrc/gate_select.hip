// Gate path for gfx950: the order-preserving top-K keep lists of a ragged batch selected by many
// workgroups per sequence (then the rows gathered by the pack kernel of gate.hip).
//
// Reference (tokengate/e2e_gate/gate_module/gate_forward.py): per sample K_c = max(1, min(K, n_art))
// (:1409-1410); keep = cat(arange(s), s + sort(topk(scores, K_c)), arange(e, seq_len)) (:1417-1421);
// kept positions (:1457) and the kept rows' gate bias — the score RMS-normalised over the state
// span (E2EGate.forward, e2e_gate_module.py:342-385, eps 1e-6), 0 on prefix / suffix rows
// (build_gate_bias_vectorized :968-1036).  Ties between equal scores go to the lower position;
// -0 equals +0; NaN ranks above +inf.
//
// Sequence b's state span of n_b scores is cut into chunks of CHUNK = 512 * KPT keys; thread t of
// a chunk's workgroup holds KPT consecutive keys (order-preserving uint32 of the scores).  The
// K_c-th largest key T is found digit by digit (bits 31..20, 19..9, 8..0); the kept keys are those
// above T and, among the keys equal to T, the lowest positions up to the count still needed.
//   select1  per chunk: histogram of the top 12 bits and the sum of squares, published.  The
//            chunk that arrives last at its sequence's counter (no workgroup waits for another)
//            sums the sequence's histograms: digit B1, the rank still needed inside it, the RMS
//            normaliser.
//   select2  per chunk: histogram of bits 19..9 of the keys whose top bits are B1, and those keys
//            (with positions) appended to the sequence's candidate buffer.  The last chunk to
//            arrive sums the histograms (digit B2), takes the candidates of prefix B1.B2 (or, if
//            the buffer overflowed, scans the whole span for them), finds the last digit with a
//            512-bin histogram, hence T and the ties still needed, and each chunk's quota of ties
//            (lowest positions first, chunk by chunk).
//   compact  workgroups take tickets in start order.  The first n_select tickets compact one
//            chunk each: its keys above T plus its quota of ties, published at once; its output
//            offset is the sum of the sequence's earlier chunks' counts (a look-back over lower
//            tickets, which started first and publish without waiting, so the launch completes
//            whatever the scheduling); then kept positions ascending, int64 positions and gate
//            bias.  The other workgroups write the prefix / suffix rows' entries.  The last
//            workgroup to finish zeroes the counters, so a zeroed workspace stays zeroed.
// Only the last arrival of a sequence reads the others' published data, so the cross-XCD
// exchanges are one release (L2 write-back) per chunk and one acquire per sequence and pass.
#include <type_traits>

#include "tg_common.h"
#include "../../include/tokengate_hip.h"

namespace tg {
// gate.hip: the row gather, here with this workspace's error word (a kept position outside its
// sequence, i.e. a keep list left unwritten after a failed wait, is skipped and reported)
int gate_pack_launch(const tg_pack_stream *streams, int32_t n_streams, const int64_t *keep, const int32_t *geom,
                     int32_t num_seqs, int64_t total_kept, int64_t *positions_out, const float *bias_src,
                     const float *sumsq, float rms_eps, float *bias_out, uint32_t *err, hipStream_t stream);
namespace {

constexpr int kQThreads = 512;
constexpr int kQWaves = kQThreads / 64;
constexpr int kQBins1 = 4096;          // bits 31..20
constexpr int kQBins2 = 2048;          // bits 19..9
constexpr int kQBins3 = 512;           // bits 8..0
constexpr int kQMaxChunks = 64;        // chunks per sequence
constexpr int kQCap = 16384;           // candidate buffer per sequence (key, position)
constexpr int kQMaxStreams = 16;
constexpr int kQSeqWords = 16;         // per-sequence record
constexpr int kQChunkWords = 8;        // per-chunk record

// per-sequence record words
enum { SQ_CNT1 = 0, SQ_CNT2, SQ_CAND, SQ_B1, SQ_R1, SQ_T, SQ_RNORM };
// per-chunk record words
enum { CK_SUMSQ = 0, CK_QUOTA, CK_AGG };   // CK_AGG: zero, or kept count | 1 << 31 once published
// global words
enum { GL_TICKET = 0, GL_EXIT, GL_ERROR };

__device__ __forceinline__ uint32_t qkey(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  uint32_t k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  k = (f == 0.f) ? 0x80000000u : k;
  k = (f != f) ? 0xffffffffu : k;
  return k;
}
__device__ __forceinline__ float qval(uint32_t k) {
  return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

struct SelArgs {
  const float *scores;
  const int32_t *geom;       // (nseq, 6): row_start, seq_len, art_start, art_end, k_clamped, kept_start
  const int32_t *wg_start;   // (nseq + 1): sequence b's chunks are [wg_start[b], wg_start[b+1])
  int nseq;
  int n_sel;                 // chunks (wg_start[nseq])
  int64_t total_kept;
  int64_t *keep;             // (total_kept,) int64 positions, ascending per sequence
  int64_t *pos_out;          // optional copy of keep (the RoPE positions)
  float *bias_out;           // optional gate bias of the kept rows
  float eps;
  uint32_t *seq;             // (nseq, kQSeqWords)
  uint32_t *chunk;           // (n_sel, kQChunkWords)
  uint32_t *glob;            // 64 words
  uint32_t *hist1;           // (n_sel, kQBins1)
  uint32_t *hist2;           // (n_sel, kQBins2)
  uint32_t *cand;            // (nseq, kQCap, 2)
  int spin_limit;
};

// Chunk gc's sequence, its first chunk and chunk count.
__device__ __forceinline__ int seq_of_chunk(const SelArgs &a, int gc, int &g0, int &G) {
  int lo = 0, hi = a.nseq - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a.wg_start[mid] <= gc) lo = mid; else hi = mid - 1;
  }
  g0 = a.wg_start[lo];
  G = a.wg_start[lo + 1] - g0;
  return lo;
}

// Order keys of this thread's KPT consecutive scores of the chunk (article index t0 .. t0+KPT-1;
// invalid ones past n are left out of `valid`) and their sum of squares.
template <int KPT>
__device__ __forceinline__ void load_keys(const float *art, int n, int t0, uint32_t (&key)[KPT], uint32_t &valid,
                                          float &ssq) {
  ssq = 0.f;
  const float *src = art + t0;
  if (((reinterpret_cast<uintptr_t>(art) & 15) == 0) && t0 + KPT <= n) {
#pragma unroll
    for (int i = 0; i < KPT; i += 4) {
      const f32x4 f = *reinterpret_cast<const f32x4 *>(src + i);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        key[i + j] = qkey(f[j]);
        ssq = fmaf(f[j], f[j], ssq);
      }
    }
    valid = KPT >= 32 ? 0xffffffffu : ((1u << KPT) - 1u);
  } else {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const bool v = t0 + i < n;
      const float f = v ? src[i] : 0.f;
      key[i] = qkey(f);
      ssq = v ? fmaf(f, f, ssq) : ssq;
    }
    const int nv = max(0, min(KPT, n - t0));
    valid = nv >= 32 ? 0xffffffffu : ((1u << nv) - 1u);
  }
}

// Block-wide exclusive prefix sum of one int per thread (thread order), and the total.
__device__ __forceinline__ int q_scan(int v, int *s_w, int &total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  __syncthreads();
  if (lane == 63) s_w[w] = incl;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kQWaves; ++i) {
    const int x = s_w[i];
    before += i < w ? x : 0;
    tot += x;
  }
  total = tot;
  return before + incl - v;
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Every wave's global stores have completed (reached L2) before the workgroup barrier, so that
// the one agent-scope release issued after it (which writes L2 back for the other XCDs) covers
// them.
__device__ __forceinline__ void stores_done_barrier() {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

// Publish this workgroup's global writes and count its arrival; true in every thread of the
// workgroup that arrived last (which then sees every other arrival's writes).
__device__ bool arrive_last(uint32_t *ctr, int G, int *s_flag) {
  stores_done_barrier();
  if (threadIdx.x == 0) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const uint32_t old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old == (uint32_t)(G - 1);
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    *s_flag = last ? 1 : 0;
  }
  __syncthreads();
  return *s_flag != 0;
}

// Descending digit search over NB bins (thread t owns NB/512 consecutive bins at the top end minus
// t): totals in tv (per owned bin, ascending bin order), krem = rank sought from the top.  The
// owning thread writes the digit, its count and the count above it.
template <int PER>
__device__ __forceinline__ void find_digit(const uint32_t (&tv)[PER], int bin0, int krem, int *s_w, int *s_d,
                                           int *s_cnt, int *s_above) {
  int lt = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) lt += (int)tv[j];
  int tot;
  const int before = q_scan(lt, s_w, tot);
  if (before < krem && krem <= before + lt) {
    int acc = before, d = -1, cd = 0;
#pragma unroll
    for (int j = PER - 1; j >= 0; --j)
      if (d < 0) {
        if (acc + (int)tv[j] >= krem) { d = bin0 + j; cd = (int)tv[j]; }
        else acc += (int)tv[j];
      }
    *s_d = d;
    *s_cnt = cd;
    *s_above = acc;
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------------------------
template <int KPT>
__global__ __launch_bounds__(kQThreads) void gate_select1_kernel(SelArgs a) {
  constexpr int CHUNK = KPT * kQThreads;
  constexpr int PER = kQBins1 / kQThreads;   // 8 bins per thread
  __shared__ uint32_t s_hist[kQBins1];
  __shared__ int s_w[kQWaves], s_flag, s_d, s_cnt, s_above_d;
  __shared__ float s_r2[kQWaves], s_r2c[kQMaxChunks];
  const int tid = threadIdx.x, gc = blockIdx.x;
  int g0, G;
  const int b = seq_of_chunk(a, gc, g0, G);
  const int *gm = a.geom + 6 * b;
  const int s = gm[2], e = gm[3], kc = gm[4];
  const int n = e - s;
  const int t0 = (gc - g0) * CHUNK + tid * KPT;
  const float *art = a.scores + (int64_t)gm[0] + s;
  uint32_t key[KPT], valid;
  float ssq;
  load_keys<KPT>(art, n, t0, key, valid, ssq);
  for (int i = tid; i < kQBins1; i += kQThreads) s_hist[i] = 0u;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < KPT; ++i)
    if (valid >> i & 1u) atomicAdd(&s_hist[key[i] >> 20], 1u);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ssq += __shfl_xor(ssq, o);
  if ((tid & 63) == 0) s_r2[tid >> 6] = ssq;
  __syncthreads();
  u32x4 *gh = reinterpret_cast<u32x4 *>(a.hist1 + (int64_t)gc * kQBins1);
  gh[tid] = reinterpret_cast<const u32x4 *>(s_hist)[tid];
  gh[tid + kQThreads] = reinterpret_cast<const u32x4 *>(s_hist)[tid + kQThreads];
  if (tid == 0) {
    float sq = 0.f;
    for (int i = 0; i < kQWaves; ++i) sq += s_r2[i];
    a.chunk[(int64_t)gc * kQChunkWords + CK_SUMSQ] = __builtin_bit_cast(uint32_t, sq);
  }
  uint32_t *sq_rec = a.seq + (int64_t)b * kQSeqWords;
  if (!arrive_last(sq_rec + SQ_CNT1, G, &s_flag)) return;

  // ---- the sequence's last chunk: digit B1, the rank still needed inside it, the normaliser ----
  const int bin0 = kQBins1 - PER * (tid + 1);     // this thread's bins bin0 .. bin0+PER-1 (descending threads)
  uint32_t tv[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) tv[j] = 0u;
  {
    const uint32_t *hb = a.hist1 + (int64_t)g0 * kQBins1 + bin0;
    int w = 0;
    for (; w + 4 <= G; w += 4) {      // four chunks' loads in flight at once
      u32x4 x[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        x[2 * q] = reinterpret_cast<const u32x4 *>(hb + (int64_t)(w + q) * kQBins1)[0];
        x[2 * q + 1] = reinterpret_cast<const u32x4 *>(hb + (int64_t)(w + q) * kQBins1)[1];
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          tv[j] += x[2 * q][j];
          tv[4 + j] += x[2 * q + 1][j];
        }
    }
    for (; w < G; ++w) {
      const u32x4 x0 = reinterpret_cast<const u32x4 *>(hb + (int64_t)w * kQBins1)[0];
      const u32x4 x1 = reinterpret_cast<const u32x4 *>(hb + (int64_t)w * kQBins1)[1];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        tv[j] += x0[j];
        tv[4 + j] += x1[j];
      }
    }
  }
  // the chunks' sums of squares, one per lane, added in chunk order
  if (tid < G) s_r2c[tid] = __builtin_bit_cast(float, a.chunk[(int64_t)(g0 + tid) * kQChunkWords + CK_SUMSQ]);
  find_digit<PER>(tv, bin0, kc, s_w, &s_d, &s_cnt, &s_above_d);
  if (tid == 0) {
    float sq = 0.f;
    for (int w = 0; w < G; ++w) sq += s_r2c[w];
    sq_rec[SQ_B1] = (uint32_t)s_d;
    sq_rec[SQ_R1] = (uint32_t)(kc - s_above_d);
    sq_rec[SQ_RNORM] = __builtin_bit_cast(uint32_t, rsqrtf(sq / (float)n + a.eps));
    sq_rec[SQ_CNT1] = 0u;           // every chunk has arrived: reset for the next call
  }
}

// ---------------------------------------------------------------------------------------------
template <int KPT>
__global__ __launch_bounds__(kQThreads) void gate_select2_kernel(SelArgs a) {
  constexpr int CHUNK = KPT * kQThreads;
  constexpr int PER = kQBins2 / kQThreads;   // 4 bins per thread
  __shared__ uint32_t s_hist[kQBins2];
  __shared__ int s_w[kQWaves], s_flag, s_d, s_cnt, s_above_d, s_base;
  __shared__ int s_tie[kQMaxChunks];
  const int tid = threadIdx.x, gc = blockIdx.x;
  int g0, G;
  const int b = seq_of_chunk(a, gc, g0, G);
  const int *gm = a.geom + 6 * b;
  const int s = gm[2], e = gm[3];
  const int n = e - s;
  const int t0 = (gc - g0) * CHUNK + tid * KPT;
  const float *art = a.scores + (int64_t)gm[0] + s;
  uint32_t *sq_rec = a.seq + (int64_t)b * kQSeqWords;
  const uint32_t B1 = sq_rec[SQ_B1];
  const int r1 = (int)sq_rec[SQ_R1];
  uint32_t key[KPT], valid;
  float ssq;
  load_keys<KPT>(art, n, t0, key, valid, ssq);
  for (int i = tid; i < kQBins2; i += kQThreads) s_hist[i] = 0u;
  __syncthreads();
  uint32_t inplay = 0u;
#pragma unroll
  for (int i = 0; i < KPT; ++i)
    if ((valid >> i & 1u) && (key[i] >> 20) == B1) {
      inplay |= 1u << i;
      atomicAdd(&s_hist[(key[i] >> 9) & (kQBins2 - 1)], 1u);
    }
  // candidates: this chunk's keys of digit B1, appended to the sequence's buffer
  int nin_tot;
  const int in_off = q_scan(__builtin_popcount(inplay), s_w, nin_tot);
  if (tid == 0)
    s_base = nin_tot ? (int)__hip_atomic_fetch_add(sq_rec + SQ_CAND, (uint32_t)nin_tot, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT)
                     : 0;
  __syncthreads();
  {
    uint32_t *cb = a.cand + (int64_t)b * kQCap * 2;
    int o = s_base + in_off;
#pragma unroll
    for (int i = 0; i < KPT; ++i)
      if (inplay >> i & 1u) {
        if (o < kQCap) {
          cb[2 * o] = key[i];
          cb[2 * o + 1] = (uint32_t)(t0 + i);
        }
        ++o;
      }
  }
  reinterpret_cast<u32x4 *>(a.hist2 + (int64_t)gc * kQBins2)[tid] = reinterpret_cast<const u32x4 *>(s_hist)[tid];
  if (!arrive_last(sq_rec + SQ_CNT2, G, &s_flag)) return;

  // ---- the sequence's last chunk: digit B2, then T and the ties still needed from the candidates,
  // then each chunk's quota of ties (lowest positions first) ----
  const int bin0 = kQBins2 - PER * (tid + 1);
  uint32_t tv[PER] = {0u, 0u, 0u, 0u};
  {
    const uint32_t *hb = a.hist2 + (int64_t)g0 * kQBins2 + bin0;
    int w = 0;
    for (; w + 8 <= G; w += 8) {      // eight chunks' loads in flight at once
      u32x4 x[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) x[q] = *reinterpret_cast<const u32x4 *>(hb + (int64_t)(w + q) * kQBins2);
#pragma unroll
      for (int q = 0; q < 8; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j) tv[j] += x[q][j];
    }
    for (; w < G; ++w) {
      const u32x4 x = *reinterpret_cast<const u32x4 *>(hb + (int64_t)w * kQBins2);
#pragma unroll
      for (int j = 0; j < 4; ++j) tv[j] += x[j];
    }
  }
  find_digit<PER>(tv, bin0, r1, s_w, &s_d, &s_cnt, &s_above_d);
  const uint32_t B2 = (uint32_t)s_d;
  const int r2 = r1 - s_above_d;
  if (tid < G) s_tie[tid] = 0;
  // keys of prefix B1.B2 (23 bits): from the candidate buffer, or the whole span if it overflowed
  const uint32_t pre = (B1 << 11) | B2;
  const int ncand = (int)sq_rec[SQ_CAND];
  const bool from_buf = ncand <= kQCap;
  const uint32_t *cb = a.cand + (int64_t)b * kQCap * 2;
  const int nscan = from_buf ? ncand : n;
  for (int i = tid; i < kQBins3; i += kQThreads) s_hist[i] = 0u;
  __syncthreads();
  for (int i = tid; i < nscan; i += kQThreads) {
    const uint32_t k = from_buf ? cb[2 * i] : qkey(art[i]);
    if ((k >> 9) == pre) atomicAdd(&s_hist[k & (kQBins3 - 1)], 1u);
  }
  __syncthreads();
  const uint32_t t3 = s_hist[kQBins3 - 1 - tid];        // thread t owns bin 511 - t
  uint32_t tv3[1] = {t3};
  find_digit<1>(tv3, kQBins3 - 1 - tid, r2, s_w, &s_d, &s_cnt, &s_above_d);
  const uint32_t T = (pre << 9) | (uint32_t)s_d;
  const int rT = r2 - s_above_d;                       // ties of T still needed
  for (int i = tid; i < nscan; i += kQThreads) {
    const uint32_t k = from_buf ? cb[2 * i] : qkey(art[i]);
    if (k == T) atomicAdd(&s_tie[(from_buf ? (int)cb[2 * i + 1] : i) / CHUNK], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int tb = 0;
    for (int w = 0; w < G; ++w) {       // chunks in position order
      const int q = max(0, min(s_tie[w], rT - tb));
      tb += s_tie[w];
      a.chunk[(int64_t)(g0 + w) * kQChunkWords + CK_QUOTA] = (uint32_t)q;
    }
    sq_rec[SQ_T] = T;
    sq_rec[SQ_CNT2] = 0u;
    sq_rec[SQ_CAND] = 0u;
  }
}

// ---------------------------------------------------------------------------------------------
template <int KPT>
__global__ __launch_bounds__(kQThreads) void gate_compact_kernel(SelArgs a) {
  constexpr int CHUNK = KPT * kQThreads;
  __shared__ int s_w[kQWaves], s_flag;
  const int tid = threadIdx.x;
  if (tid == 0)
    s_flag = (int)__hip_atomic_fetch_add(a.glob + GL_TICKET, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  const int ticket = s_flag;

  if (ticket < a.n_sel) {
    // ---- compaction of chunk `ticket` ----
    const int gc = ticket;
    int g0, G;
    const int b = seq_of_chunk(a, gc, g0, G);
    const int *gm = a.geom + 6 * b;
    const int s = gm[2], e = gm[3], kstart = gm[5];
    const int n = e - s;
    const int t0 = (gc - g0) * CHUNK + tid * KPT;
    const float *art = a.scores + (int64_t)gm[0] + s;
    const uint32_t *sq_rec = a.seq + (int64_t)b * kQSeqWords;
    const uint32_t T = sq_rec[SQ_T];
    const float rn = __builtin_bit_cast(float, sq_rec[SQ_RNORM]);
    const int quota = (int)a.chunk[(int64_t)gc * kQChunkWords + CK_QUOTA];
    uint32_t key[KPT], valid;
    float ssq;
    load_keys<KPT>(art, n, t0, key, valid, ssq);
    uint32_t gtm = 0u, tiem = 0u;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const bool v = valid >> i & 1u;
      gtm |= (v && key[i] > T) ? 1u << i : 0u;
      tiem |= (v && key[i] == T) ? 1u << i : 0u;
    }
    int ntie, ngt;
    int tr = q_scan(__builtin_popcount(tiem), s_w, ntie);   // ties of T before this thread's
    q_scan(__builtin_popcount(gtm), s_w, ngt);
    // publish this chunk's kept count, then add those of the sequence's earlier chunks (their
    // workgroups hold lower tickets: they started first and publish without waiting)
    if (tid == 0)
      __hip_atomic_store(a.chunk + (int64_t)gc * kQChunkWords + CK_AGG,
                         0x80000000u | (uint32_t)(ngt + min(quota, ntie)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid < 64) {
      const int wl = gc - g0;
      int add = 0;
      if (tid < wl) {
        const uint32_t *ag = a.chunk + (int64_t)(g0 + tid) * kQChunkWords + CK_AGG;
        uint32_t v = 0u;
        int it = 0;
        while (!((v = __hip_atomic_load(ag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) & 0x80000000u)) {
          if (++it > a.spin_limit) {
            __hip_atomic_store(a.glob + GL_ERROR, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
        add = (int)(v & 0x7fffffffu);
      }
      add = wave_sum_i(add);
      if (tid == 0) s_flag = add;
    }
    __syncthreads();
    const int off = s_flag;
    uint32_t keepm = gtm;
#pragma unroll
    for (int i = 0; i < KPT; ++i)
      if (tiem >> i & 1u) {
        if (tr < quota) keepm |= 1u << i;
        ++tr;
      }
    int nk;
    const int koff = q_scan(__builtin_popcount(keepm), s_w, nk);
    int64_t j = (int64_t)kstart + s + off + koff;
    const int64_t j_end = (int64_t)kstart + s + gm[4];      // this sequence's state rows end here
#pragma unroll
    for (int i = 0; i < KPT; ++i)
      if (keepm >> i & 1u) {
        const int64_t pos = s + t0 + i;
        if (j < j_end) {
          a.keep[j] = pos;
          if (a.pos_out) a.pos_out[j] = pos;
          if (a.bias_out) a.bias_out[j] = qval(key[i]) * rn;
        } else {
          __hip_atomic_store(a.glob + GL_ERROR, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        ++j;
      }
  } else {
    // ---- prefix / suffix rows of 512 packed rows: positions need no selection ----
    const int64_t jr = (int64_t)(ticket - a.n_sel) * kQThreads + tid;
    if (jr < a.total_kept) {
      int lo = 0, hi = a.nseq - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if ((int64_t)a.geom[6 * mid + 5] <= jr) lo = mid; else hi = mid - 1;
      }
      const int *gm = a.geom + 6 * lo;
      const int64_t t = jr - gm[5];
      const int s = gm[2], e = gm[3], kc = gm[4];
      const int64_t pos = t < s ? t : (t >= (int64_t)s + kc ? e + (t - s - kc) : -1);
      if (pos >= 0) {
        a.keep[jr] = pos;
        if (a.pos_out) a.pos_out[jr] = pos;
        if (a.bias_out) a.bias_out[jr] = 0.f;
      }
    }
  }

  // ---- exit: the last workgroup resets the counters ----
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(a.glob + GL_EXIT, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    s_flag = prev == gridDim.x - 1 ? 1 : 0;
  }
  __syncthreads();
  if (s_flag) {
    for (int i = tid; i < a.n_sel; i += kQThreads) a.chunk[(int64_t)i * kQChunkWords + CK_AGG] = 0u;
    if (tid == 0) {
      a.glob[GL_TICKET] = 0u;
      a.glob[GL_EXIT] = 0u;
    }
  }
}

// Workspace layout for up to seq_cap sequences and chunk_cap chunks.  The counters that must be
// zero when a call starts (global words, per-sequence records) come first at offsets that depend
// only on the capacities, so calls of any size within them find the counters the previous call
// left zeroed.
int64_t ws_layout(int32_t seq_cap, int32_t chunk_cap, int64_t off[6]) {
  int64_t o = 0;
  auto take = [&](int64_t bytes) { const int64_t r = o; o += (bytes + 255) / 256 * 256; return r; };
  off[0] = take(64 * 4);                                       // global words
  off[1] = take((int64_t)seq_cap * kQSeqWords * 4);            // sequence records
  off[2] = take((int64_t)chunk_cap * kQChunkWords * 4);        // chunk records
  off[3] = take((int64_t)chunk_cap * kQBins1 * 4);             // hist1
  off[4] = take((int64_t)chunk_cap * kQBins2 * 4);             // hist2
  off[5] = take((int64_t)seq_cap * kQCap * 8);                 // candidates
  return o;
}

template <int KPT>
void launch_select(const SelArgs &a, int grid, hipStream_t stream) {
  hipLaunchKernelGGL(gate_select1_kernel<KPT>, dim3(a.n_sel), dim3(kQThreads), 0, stream, a);
  hipLaunchKernelGGL(gate_select2_kernel<KPT>, dim3(a.n_sel), dim3(kQThreads), 0, stream, a);
  hipLaunchKernelGGL(gate_compact_kernel<KPT>, dim3(grid), dim3(kQThreads), 0, stream, a);
}

}  // namespace
}  // namespace tg

using namespace tg;

extern "C" int64_t tg_gate_select_pack_workspace_size(int32_t seq_capacity, int32_t chunk_capacity) {
  if (seq_capacity <= 0 || chunk_capacity < 0) return 0;
  int64_t off[6];
  return ws_layout(seq_capacity, chunk_capacity, off);
}

extern "C" int tg_gate_select_pack(const float *scores, const int32_t *geom, const int32_t *wg_start,
                                   int32_t num_seqs, int32_t n_select_wgs, int32_t keys_per_thread,
                                   const tg_pack_stream *streams, int32_t n_streams, int64_t total_kept,
                                   int64_t *keep, int64_t *positions_out, float *bias_out, float rms_eps,
                                   void *workspace, int32_t seq_capacity, int32_t chunk_capacity,
                                   hipStream_t stream) {
  clear_error();
  TG_CHECK(scores && geom && wg_start && keep && workspace, "null pointer");
  TG_CHECK(num_seqs >= 0 && n_select_wgs >= 0 && total_kept >= 0, "negative size");
  TG_CHECK(n_streams >= 0 && n_streams <= kQMaxStreams, "at most %d streams", kQMaxStreams);
  TG_CHECK(n_streams == 0 || streams != nullptr, "null streams");
  TG_CHECK(keys_per_thread == 8 || keys_per_thread == 16 || keys_per_thread == 32,
           "keys_per_thread must be 8, 16 or 32");
  if (num_seqs == 0 || total_kept == 0) return 0;
  TG_CHECK(num_seqs <= seq_capacity && n_select_wgs <= chunk_capacity,
           "workspace capacity (%d sequences, %d chunks) below this call's (%d, %d)", seq_capacity, chunk_capacity,
           num_seqs, n_select_wgs);
  TG_CHECK((reinterpret_cast<uintptr_t>(workspace) & 255) == 0, "workspace must be 256-byte aligned");
  const int64_t meta_wgs = (total_kept + kQThreads - 1) / kQThreads;   // prefix / suffix rows, 512 per workgroup
  TG_CHECK((int64_t)n_select_wgs + meta_wgs < (1ll << 31), "grid too large");
  int64_t off[6];
  ws_layout(seq_capacity, chunk_capacity, off);
  SelArgs a{};
  a.scores = scores;
  a.geom = geom;
  a.wg_start = wg_start;
  a.nseq = num_seqs;
  a.n_sel = n_select_wgs;
  a.total_kept = total_kept;
  a.keep = keep;
  a.pos_out = positions_out;
  a.bias_out = bias_out;
  a.eps = rms_eps;
  char *w = static_cast<char *>(workspace);
  a.glob = reinterpret_cast<uint32_t *>(w + off[0]);
  a.seq = reinterpret_cast<uint32_t *>(w + off[1]);
  a.chunk = reinterpret_cast<uint32_t *>(w + off[2]);
  a.hist1 = reinterpret_cast<uint32_t *>(w + off[3]);
  a.hist2 = reinterpret_cast<uint32_t *>(w + off[4]);
  a.cand = reinterpret_cast<uint32_t *>(w + off[5]);
  a.spin_limit = 1 << 22;
  const int grid = (int)(n_select_wgs + meta_wgs);
  if (n_select_wgs == 0) {
    hipLaunchKernelGGL(gate_compact_kernel<8>, dim3(grid), dim3(kQThreads), 0, stream, a);
  } else {
    switch (keys_per_thread) {
      case 8: launch_select<8>(a, grid, stream); break;
      case 16: launch_select<16>(a, grid, stream); break;
      default: launch_select<32>(a, grid, stream); break;
    }
  }
  TG_HIP_CHECK(hipPeekAtLastError());
  // the rows themselves: the pack over the keep lists just written (positions and bias are done)
  if (n_streams > 0)
    return gate_pack_launch(streams, n_streams, keep, geom, num_seqs, total_kept, nullptr, nullptr, nullptr, rms_eps,
                            nullptr, a.glob + GL_ERROR, stream);
  return 0;
}
