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
constexpr int kQLdsCand = 4096;        // digit-B1 keys the one-launch form resolves in LDS
constexpr int kQFusedMaxChunks = 512;  // chunk workgroups of the one-launch form (at most one per CU)
constexpr int kQMaxChunkKeys = 32 * kQThreads;
constexpr int kQGroups = kQBins1 / 16;   // one-launch form: coarse groups of 16 top-digit bins
constexpr int kQMaxStreams = 16;
constexpr int kQSeqWords = 16;         // per-sequence record
constexpr int kQChunkWords = 8;        // per-chunk record

// per-sequence record words
enum { SQ_CNT1 = 0, SQ_CNT2, SQ_CAND, SQ_B1, SQ_R1, SQ_T, SQ_RNORM, SQ_FLAG, SQ_DONE };   // SQ_FLAG, SQ_DONE: one-launch form
// per-chunk record words
enum { CK_SUMSQ = 0, CK_QUOTA, CK_AGG, CK_OFF };   // CK_AGG: zero, or kept count | 1 << 31 once published;
                                                 // CK_OFF: output offset (one-launch form, resolved in LDS)
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
  uint32_t *sorted;          // one-launch form: (n_sel, 512 * KPT) each chunk's keys by top digit, descending
  uint32_t *coarse;          // one-launch form: (n_sel, kQGroups) each chunk's keys above each group of 16 bins
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

// Inclusive prefix sum over the 64 lanes of a wave on the DPP network: shifts by 1, 2, 4, 8 inside
// each row of 16 lanes (lanes without a source add 0), then the last lane of row 0 broadcast into
// row 1 and that of row 2 into row 3, then lane 31 into rows 2 and 3.
__device__ __forceinline__ int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);    // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);    // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);    // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);    // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);   // row_bcast:15 into rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);   // row_bcast:31 into rows 2, 3
  return v;
}

// Block-wide exclusive prefix sum of one int per thread (thread order), and the total.
__device__ __forceinline__ int q_scan(int v, int *s_w, int &total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int incl = wave_incl_scan(v);
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

__device__ __forceinline__ int wave_sum_i(int v) { return __builtin_amdgcn_readlane(wave_incl_scan(v), 63); }

// Sum over the 64 lanes of a wave (the same DPP network as wave_incl_scan; lane 63 ends with it).
template <int CTRL, int ROWS, bool BOUND>
__device__ __forceinline__ float dpp_add_f(float x) {
  return x + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, ROWS, 0xf, BOUND));
}
__device__ __forceinline__ float wave_sum_f(float v) {
  v = dpp_add_f<0x111, 0xf, true>(v);    // row_shr:1
  v = dpp_add_f<0x112, 0xf, true>(v);    // row_shr:2
  v = dpp_add_f<0x114, 0xf, true>(v);    // row_shr:4
  v = dpp_add_f<0x118, 0xf, true>(v);    // row_shr:8
  v = dpp_add_f<0x142, 0xa, false>(v);   // row_bcast:15 into rows 1, 3
  v = dpp_add_f<0x143, 0xc, false>(v);   // row_bcast:31 into rows 2, 3
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Maximum over the 64 lanes of a wave of non-negative ints (the same DPP network as wave_incl_scan).
__device__ __forceinline__ int wave_max_nonneg(int v) {
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true));
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true));
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true));
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true));
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false));
  return __builtin_amdgcn_readlane(v, 63);
}

// Every wave's global stores have completed (reached L2) before the workgroup barrier, so that
// the one agent-scope release issued after it (which writes L2 back for the other XCDs) covers
// them.
__device__ __forceinline__ void stores_done_barrier() {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

// Agent-scope release and acquire whose cache operations have completed when they return.  The
// release writes this XCD's L2 back (buffer_wbl2) and the acquire invalidates it (buffer_inv);
// both are vector-memory operations, but the compiler does not count them as outstanding, so
// after an earlier s_waitcnt it emits no wait for them: a flag or counter stored right after the
// write-back could reach the other XCDs ahead of the data it publishes, and the workgroup's other
// waves, released by the barrier after the invalidate, could read lines it had not yet dropped.
// The explicit waits (inline assembly, which the compiler's wait insertion leaves in place) close
// both windows.  The chunks waiting on a sequence's phase flag take no acquire at all: the few
// words the flag publishes to them are read with agent-coherent loads (ld_agent), which read
// through this XCD's L2, so no invalidate (whose completion takes microseconds) is needed there.
__device__ __forceinline__ void release_agent() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}
__device__ __forceinline__ void acquire_agent() {
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}
__device__ __forceinline__ uint32_t ld_agent(const uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Publish this workgroup's global writes and count its arrival; true in every thread of the
// workgroup that arrived last (which then sees every other arrival's writes).
__device__ bool arrive_last(uint32_t *ctr, int G, int *s_flag) {
  stores_done_barrier();
  if (threadIdx.x == 0) {
    release_agent();
    const uint32_t old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old == (uint32_t)(G - 1);
    if (last) acquire_agent();
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
// The selection's phases, composed into three launches (select1, select2, compact) or one
// (gate_select_fused_kernel).  Per chunk workgroup: its sequence, geometry and keys.
template <int KPT>
struct Chunk {
  static constexpr int CHUNK = KPT * kQThreads;
  int gc, b, g0, G, s, e, n, kc, kstart, t0;
  const int *gm;
  const float *art;
  uint32_t *sq_rec;
  uint32_t key[KPT], valid;
  float ssq;
  __device__ __forceinline__ void init(const SelArgs &a, int gc_) {
    gc = gc_;
    b = seq_of_chunk(a, gc, g0, G);
    gm = a.geom + 6 * b;
    s = gm[2];
    e = gm[3];
    kc = gm[4];
    kstart = gm[5];
    n = e - s;
    t0 = (gc - g0) * CHUNK + (int)threadIdx.x * KPT;
    art = a.scores + (int64_t)gm[0] + s;
    sq_rec = a.seq + (int64_t)b * kQSeqWords;
    load_keys<KPT>(art, n, t0, key, valid, ssq);
  }
};

struct SelShared {
  uint32_t hist[kQBins1];
  int w[kQWaves], flag, d, cnt, above, base;
  float r2[kQWaves], r2c[kQMaxChunks];
  int tie[kQMaxChunks];
  int coff[kQMaxChunks], clo[kQMaxChunks], ctot;   // one-launch form: digit-B1 key ranges per chunk
  int gt[kQMaxChunks];                             // ... and their keys above T
};

// Pass 1, every chunk: the histogram of the keys' top 12 bits and the chunk's sum of squares,
// published for the sequence's last arrival.
template <int KPT>
__device__ __forceinline__ void pass1_chunk(const SelArgs &a, Chunk<KPT> &c, SelShared &sh) {
  const int tid = threadIdx.x;
  for (int i = tid; i < kQBins1; i += kQThreads) sh.hist[i] = 0u;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < KPT; ++i)
    if (c.valid >> i & 1u) atomicAdd(&sh.hist[c.key[i] >> 20], 1u);
  float ssq = c.ssq;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ssq += __shfl_xor(ssq, o);
  if ((tid & 63) == 0) sh.r2[tid >> 6] = ssq;
  __syncthreads();
  u32x4 *gh = reinterpret_cast<u32x4 *>(a.hist1 + (int64_t)c.gc * kQBins1);
  gh[tid] = reinterpret_cast<const u32x4 *>(sh.hist)[tid];
  gh[tid + kQThreads] = reinterpret_cast<const u32x4 *>(sh.hist)[tid + kQThreads];
  if (tid == 0) {
    float sq = 0.f;
    for (int i = 0; i < kQWaves; ++i) sq += sh.r2[i];
    a.chunk[(int64_t)c.gc * kQChunkWords + CK_SUMSQ] = __builtin_bit_cast(uint32_t, sq);
  }
}

// Pass 1, the sequence's last arrival: digit B1, the rank still needed inside it, the normaliser.
template <int KPT>
__device__ __forceinline__ void pass1_last(const SelArgs &a, const Chunk<KPT> &c, SelShared &sh) {
  constexpr int PER = kQBins1 / kQThreads;   // 8 bins per thread
  const int tid = threadIdx.x;
  const int bin0 = kQBins1 - PER * (tid + 1);     // this thread's bins bin0 .. bin0+PER-1 (descending threads)
  uint32_t tv[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) tv[j] = 0u;
  {
    const uint32_t *hb = a.hist1 + (int64_t)c.g0 * kQBins1 + bin0;
    int w = 0;
    for (; w + 4 <= c.G; w += 4) {      // four chunks' loads in flight at once
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
    for (; w < c.G; ++w) {
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
  if (tid < c.G) sh.r2c[tid] = __builtin_bit_cast(float, a.chunk[(int64_t)(c.g0 + tid) * kQChunkWords + CK_SUMSQ]);
  find_digit<PER>(tv, bin0, c.kc, sh.w, &sh.d, &sh.cnt, &sh.above);
  if (tid == 0) {
    float sq = 0.f;
    for (int w = 0; w < c.G; ++w) sq += sh.r2c[w];
    c.sq_rec[SQ_B1] = (uint32_t)sh.d;
    c.sq_rec[SQ_R1] = (uint32_t)(c.kc - sh.above);
    c.sq_rec[SQ_RNORM] = __builtin_bit_cast(uint32_t, rsqrtf(sq / (float)c.n + a.eps));
    c.sq_rec[SQ_CNT1] = 0u;           // every chunk has arrived: reset for the next call
  }
}

// Pass 2, every chunk: the histogram of bits 19..9 of the keys of digit B1, and those keys (with
// positions) appended to the sequence's candidate buffer.
template <int KPT>
__device__ __forceinline__ void pass2_chunk(const SelArgs &a, const Chunk<KPT> &c, SelShared &sh) {
  const int tid = threadIdx.x;
  const uint32_t B1 = ld_agent(c.sq_rec + SQ_B1);   // published with the phase flag
  for (int i = tid; i < kQBins2; i += kQThreads) sh.hist[i] = 0u;
  __syncthreads();
  uint32_t inplay = 0u;
#pragma unroll
  for (int i = 0; i < KPT; ++i)
    if ((c.valid >> i & 1u) && (c.key[i] >> 20) == B1) {
      inplay |= 1u << i;
      atomicAdd(&sh.hist[(c.key[i] >> 9) & (kQBins2 - 1)], 1u);
    }
  int nin_tot;
  const int in_off = q_scan(__builtin_popcount(inplay), sh.w, nin_tot);
  if (tid == 0)
    sh.base = nin_tot ? (int)__hip_atomic_fetch_add(c.sq_rec + SQ_CAND, (uint32_t)nin_tot, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT)
                      : 0;
  __syncthreads();
  {
    uint32_t *cb = a.cand + (int64_t)c.b * kQCap * 2;
    int o = sh.base + in_off;
#pragma unroll
    for (int i = 0; i < KPT; ++i)
      if (inplay >> i & 1u) {
        if (o < kQCap) {
          cb[2 * o] = c.key[i];
          cb[2 * o + 1] = (uint32_t)(c.t0 + i);
        }
        ++o;
      }
  }
  reinterpret_cast<u32x4 *>(a.hist2 + (int64_t)c.gc * kQBins2)[tid] = reinterpret_cast<const u32x4 *>(sh.hist)[tid];
}

// Pass 2, the sequence's last arrival: digit B2, then T and the ties still needed from the
// candidates, then each chunk's quota of ties (lowest positions first).
template <int KPT>
__device__ __forceinline__ void pass2_last(const SelArgs &a, const Chunk<KPT> &c, SelShared &sh) {
  constexpr int PER = kQBins2 / kQThreads;   // 4 bins per thread
  constexpr int CHUNK = Chunk<KPT>::CHUNK;
  const int tid = threadIdx.x;
  const uint32_t B1 = c.sq_rec[SQ_B1];
  const int r1 = (int)c.sq_rec[SQ_R1];
  const int bin0 = kQBins2 - PER * (tid + 1);
  uint32_t tv[PER] = {0u, 0u, 0u, 0u};
  {
    const uint32_t *hb = a.hist2 + (int64_t)c.g0 * kQBins2 + bin0;
    int w = 0;
    for (; w + 8 <= c.G; w += 8) {      // eight chunks' loads in flight at once
      u32x4 x[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) x[q] = *reinterpret_cast<const u32x4 *>(hb + (int64_t)(w + q) * kQBins2);
#pragma unroll
      for (int q = 0; q < 8; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j) tv[j] += x[q][j];
    }
    for (; w < c.G; ++w) {
      const u32x4 x = *reinterpret_cast<const u32x4 *>(hb + (int64_t)w * kQBins2);
#pragma unroll
      for (int j = 0; j < 4; ++j) tv[j] += x[j];
    }
  }
  find_digit<PER>(tv, bin0, r1, sh.w, &sh.d, &sh.cnt, &sh.above);
  const uint32_t B2 = (uint32_t)sh.d;
  const int r2 = r1 - sh.above;
  if (tid < c.G) sh.tie[tid] = 0;
  // keys of prefix B1.B2 (23 bits): from the candidate buffer, or the whole span if it overflowed
  const uint32_t pre = (B1 << 11) | B2;
  const int ncand = (int)c.sq_rec[SQ_CAND];
  const bool from_buf = ncand <= kQCap;
  const uint32_t *cb = a.cand + (int64_t)c.b * kQCap * 2;
  const int nscan = from_buf ? ncand : c.n;
  for (int i = tid; i < kQBins3; i += kQThreads) sh.hist[i] = 0u;
  __syncthreads();
  for (int i = tid; i < nscan; i += kQThreads) {
    const uint32_t k = from_buf ? cb[2 * i] : qkey(c.art[i]);
    if ((k >> 9) == pre) atomicAdd(&sh.hist[k & (kQBins3 - 1)], 1u);
  }
  __syncthreads();
  const uint32_t t3 = sh.hist[kQBins3 - 1 - tid];        // thread t owns bin 511 - t
  uint32_t tv3[1] = {t3};
  find_digit<1>(tv3, kQBins3 - 1 - tid, r2, sh.w, &sh.d, &sh.cnt, &sh.above);
  const uint32_t T = (pre << 9) | (uint32_t)sh.d;
  const int rT = r2 - sh.above;                       // ties of T still needed
  for (int i = tid; i < nscan; i += kQThreads) {
    const uint32_t k = from_buf ? cb[2 * i] : qkey(c.art[i]);
    if (k == T) atomicAdd(&sh.tie[(from_buf ? (int)cb[2 * i + 1] : i) / CHUNK], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int tb = 0;
    for (int w = 0; w < c.G; ++w) {       // chunks in position order
      const int q = max(0, min(sh.tie[w], rT - tb));
      tb += sh.tie[w];
      a.chunk[(int64_t)(c.g0 + w) * kQChunkWords + CK_QUOTA] = (uint32_t)q;
    }
    c.sq_rec[SQ_T] = T;
    c.sq_rec[SQ_CNT2] = 0u;
    c.sq_rec[SQ_CAND] = 0u;
  }
}

// Compaction of one chunk: its keys above T plus its quota of ties, published at once; its output
// offset is the sum of the sequence's earlier chunks' counts (a look-back over chunks that publish
// without waiting); then kept positions ascending, int64 positions and gate bias.
template <int KPT>
__device__ __forceinline__ void compact_chunk(const SelArgs &a, const Chunk<KPT> &c, SelShared &sh, bool known_off) {
  const int tid = threadIdx.x;
  // published with the phase flag (or by the previous launch)
  const uint32_t T = ld_agent(c.sq_rec + SQ_T);
  const float rn = __builtin_bit_cast(float, ld_agent(c.sq_rec + SQ_RNORM));
  const int quota = (int)ld_agent(a.chunk + (int64_t)c.gc * kQChunkWords + CK_QUOTA);
  uint32_t gtm = 0u, tiem = 0u;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const bool v = c.valid >> i & 1u;
    gtm |= (v && c.key[i] > T) ? 1u << i : 0u;
    tiem |= (v && c.key[i] == T) ? 1u << i : 0u;
  }
  // one scan of both counts (keys above T in the high half, ties in the low; a chunk holds at most
  // 16384 keys, so the low half never carries)
  int both;
  const int before = q_scan((__builtin_popcount(gtm) << 16) | __builtin_popcount(tiem), sh.w, both);
  const int tie_before = before & 0xffff, gt_before = before >> 16;
  int off;
  if (known_off) {
    off = (int)ld_agent(a.chunk + (int64_t)c.gc * kQChunkWords + CK_OFF);
  } else {
    if (tid == 0)
      __hip_atomic_store(a.chunk + (int64_t)c.gc * kQChunkWords + CK_AGG,
                         0x80000000u | (uint32_t)((both >> 16) + min(quota, both & 0xffff)), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    if (tid < 64) {
      const int wl = c.gc - c.g0;
      int add = 0;
      if (tid < wl) {
        const uint32_t *ag = a.chunk + (int64_t)(c.g0 + tid) * kQChunkWords + CK_AGG;
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
      if (tid == 0) sh.flag = add;
    }
    __syncthreads();
    off = sh.flag;
  }
  // the quota's ties are the chunk's first ones in position order
  uint32_t keepm = gtm;
  int tr = tie_before;
#pragma unroll
  for (int i = 0; i < KPT; ++i)
    if (tiem >> i & 1u) {
      if (tr < quota) keepm |= 1u << i;
      ++tr;
    }
  const int koff = gt_before + min(tie_before, quota);
  int64_t j = (int64_t)c.kstart + c.s + off + koff;
  const int64_t j_end = (int64_t)c.kstart + c.s + c.kc;      // this sequence's state rows end here
#pragma unroll
  for (int i = 0; i < KPT; ++i)
    if (keepm >> i & 1u) {
      const int64_t pos = c.s + c.t0 + i;
      if (j < j_end) {
        a.keep[j] = pos;
        if (a.pos_out) a.pos_out[j] = pos;
        if (a.bias_out) a.bias_out[j] = qval(c.key[i]) * rn;
      } else {
        __hip_atomic_store(a.glob + GL_ERROR, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      ++j;
    }
}

// Prefix / suffix rows of 512 packed rows (workgroup `mw` of them): positions need no selection.
__device__ __forceinline__ void write_meta_rows(const SelArgs &a, int64_t mw) {
  const int64_t jr = mw * kQThreads + threadIdx.x;
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

// Compaction launch: the workgroup that finishes last zeroes the tickets and the look-back words,
// so that a zeroed workspace stays zeroed.
__device__ __forceinline__ void exit_reset(const SelArgs &a, SelShared &sh) {
  __syncthreads();
  if (threadIdx.x == 0) {
    release_agent();
    const uint32_t prev = __hip_atomic_fetch_add(a.glob + GL_EXIT, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == gridDim.x - 1) acquire_agent();
    sh.flag = prev == gridDim.x - 1 ? 1 : 0;
  }
  __syncthreads();
  if (sh.flag) {
    for (int i = threadIdx.x; i < a.n_sel; i += kQThreads) a.chunk[(int64_t)i * kQChunkWords + CK_AGG] = 0u;
    if (threadIdx.x == 0) {
      a.glob[GL_TICKET] = 0u;
      a.glob[GL_EXIT] = 0u;
    }
  }
}

// One-launch form: the chunk of a sequence that finishes last (its own counter) zeroes the
// sequence's phase flag and its chunks' look-back words, so that a zeroed workspace stays zeroed.
// Every chunk's reads of those words are complete here (their values were used), and the last
// arrival of each pass finishes after raising the flag.
__device__ __forceinline__ void seq_done(const SelArgs &a, uint32_t *sq_rec, int g0, int G, SelShared &sh) {
  __syncthreads();
  if (threadIdx.x == 0)
    sh.flag = __hip_atomic_fetch_add(sq_rec + SQ_DONE, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
              (uint32_t)(G - 1);
  __syncthreads();
  if (sh.flag) {
    for (int i = threadIdx.x; i < G; i += kQThreads) a.chunk[(int64_t)(g0 + i) * kQChunkWords + CK_AGG] = 0u;
    if (threadIdx.x == 0) {
      sq_rec[SQ_FLAG] = 0u;
      sq_rec[SQ_DONE] = 0u;
    }
  }
}

// ---------------------------------------------------------------------------------------------
template <int KPT>
__global__ __launch_bounds__(kQThreads) void gate_select1_kernel(SelArgs a) {
  __shared__ SelShared sh;
  Chunk<KPT> c;
  c.init(a, blockIdx.x);
  pass1_chunk<KPT>(a, c, sh);
  if (arrive_last(c.sq_rec + SQ_CNT1, c.G, &sh.flag)) pass1_last<KPT>(a, c, sh);
}

template <int KPT>
__global__ __launch_bounds__(kQThreads) void gate_select2_kernel(SelArgs a) {
  __shared__ SelShared sh;
  Chunk<KPT> c;
  c.init(a, blockIdx.x);
  pass2_chunk<KPT>(a, c, sh);
  if (arrive_last(c.sq_rec + SQ_CNT2, c.G, &sh.flag)) pass2_last<KPT>(a, c, sh);
}

// Workgroups take tickets in start order: the first n_sel tickets compact one chunk each (their
// look-back only waits for lower tickets, which started first and publish without waiting), the
// rest write the prefix / suffix rows.
template <int KPT>
__global__ __launch_bounds__(kQThreads) void gate_compact_kernel(SelArgs a) {
  __shared__ SelShared sh;
  if (threadIdx.x == 0)
    sh.flag = (int)__hip_atomic_fetch_add(a.glob + GL_TICKET, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  const int ticket = sh.flag;
  if (ticket < a.n_sel) {
    Chunk<KPT> c;
    c.init(a, ticket);
    compact_chunk<KPT>(a, c, sh, false);
  } else {
    write_meta_rows(a, ticket - a.n_sel);
  }
  exit_reset(a, sh);
}

// One launch for batches whose chunk workgroups all fit the chip at once (n_sel at most the CU
// count; the host checks): workgroups 0 .. n_sel-1 are the chunks, in sequence order, the rest
// write the prefix / suffix rows and wait for nothing.  A chunk keeps its keys in registers
// through the phases; between phases the chunks of a sequence wait for the phase flag that the
// sequence's last arrival raises after writing its results (a bounded spin: on expiry the error
// word is set and the chunk goes on, so every workgroup finishes whatever happens).  The pass-1
// last arrival resolves T, the quotas and every chunk's output offset itself when digit B1 holds
// at most kQLdsCand keys and raises the flag straight to 3: the chunks then skip pass 2 and compact
// without the look-back.
__device__ __forceinline__ uint32_t wait_flag(const SelArgs &a, const uint32_t *flag, uint32_t want, int *s_val) {
  if (threadIdx.x == 0) {
    int it = 0;
    uint32_t v;
    while ((v = __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) < want) {
      if (++it > a.spin_limit) {
        __hip_atomic_store(a.glob + GL_ERROR, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        v = want;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    // no acquire: what the flag publishes is read with ld_agent
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    *s_val = (int)v;
  }
  __syncthreads();
  return (uint32_t)*s_val;
}

// Publish the last arrival's results (stores of this workgroup, complete before the barrier) and
// raise the sequence's phase flag.
__device__ __forceinline__ void raise_flag(uint32_t *flag, uint32_t value) {
  stores_done_barrier();
  if (threadIdx.x == 0) {
    release_agent();
    __hip_atomic_store(flag, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Pass 1 of the one-launch form, every chunk: the histogram of its keys' top 12 bits published as
// descending cumulative counts (cex[b]: keys of the chunk in bins above b), and its keys ordered by
// that digit, descending (bin b's keys at cex[b] .. cex[b-1] - 1), for the sequence's last arrival.
// Only the bins with cex[b] < K_c are written: T is at least the chunk's own K_c-th largest key
// (the chunk alone holds K_c keys at or above it), so digit B1 is at least that key's bin, the
// lowest such bin.
template <int KPT>
__device__ __forceinline__ void pass1_chunk_sorted(const SelArgs &a, const Chunk<KPT> &c, SelShared &sh,
                                                   uint32_t *stage) {
  constexpr int PER = kQBins1 / kQThreads;   // 8 bins per thread
  constexpr int CHUNK = Chunk<KPT>::CHUNK;
  const int tid = threadIdx.x;
  // (sh.hist and sh.base were zeroed, and the workgroup synchronised, before the keys were loaded)
  uint32_t rank[KPT];                        // each key's place among the chunk's keys of its bin
#pragma unroll
  for (int i = 0; i < KPT; ++i) rank[i] = (c.valid >> i & 1u) ? atomicAdd(&sh.hist[c.key[i] >> 20], 1u) : 0u;
  const float wsq = wave_sum_f(c.ssq);       // read by thread 0 after the barriers below
  if ((tid & 63) == 0) sh.r2[tid >> 6] = wsq;
  __syncthreads();
  const int bin0 = kQBins1 - PER * (tid + 1);     // this thread's bins bin0 .. bin0+PER-1 (descending threads)
  uint32_t h[PER];
  int mine = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    h[j] = sh.hist[bin0 + j];
    mine += (int)h[j];
  }
  int nvalid;
  uint32_t run = (uint32_t)q_scan(mine, sh.w, nvalid);   // keys in the bins of lower threads (higher bins)
  uint32_t cx[PER];
#pragma unroll
  for (int j = PER - 1; j >= 0; --j) {
    cx[j] = run;
    run += h[j];
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) sh.hist[bin0 + j] = cx[j];
  u32x4 *gh = reinterpret_cast<u32x4 *>(a.hist1 + (int64_t)c.gc * kQBins1 + bin0);
  gh[0] = u32x4{cx[0], cx[1], cx[2], cx[3]};
  gh[1] = u32x4{cx[4], cx[5], cx[6], cx[7]};
  // the even threads own the top bin of a group of 16: keys above that group
  if ((tid & 1) == 0) a.coarse[(int64_t)c.gc * kQGroups + (kQGroups - 1 - (tid >> 1))] = cx[PER - 1];
  __syncthreads();
  int nwrite = 0;                            // the written prefix: keys of the bins with cex < K_c
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const uint32_t first = sh.hist[c.key[i] >> 20];
    if ((c.valid >> i & 1u) && first < (uint32_t)c.kc) {
      stage[first + rank[i]] = c.key[i];
      nwrite = max(nwrite, (int)(first + rank[i]) + 1);
    }
  }
  nwrite = wave_max_nonneg(nwrite);
  if ((tid & 63) == 0 && nwrite) atomicMax(&sh.base, nwrite);
  __syncthreads();
  nwrite = sh.base;
  uint32_t *dst = a.sorted + (int64_t)c.gc * CHUNK;
  for (int i = 4 * tid; i < nwrite; i += 4 * kQThreads)
    *reinterpret_cast<u32x4 *>(dst + i) = *reinterpret_cast<const u32x4 *>(stage + i);
  if (tid == 0) {
    float sq = 0.f;
    for (int i = 0; i < kQWaves; ++i) sq += sh.r2[i];
    a.chunk[(int64_t)c.gc * kQChunkWords + CK_SUMSQ] = __builtin_bit_cast(uint32_t, sq);
  }
}

// Pass 1 of the one-launch form, the sequence's last arrival: digit B1 = the bin with
// CEX[B1] < K_c <= CEX[B1 - 1], CEX[b] being the sequence's keys above bin b (the chunks' cumulative
// counts summed), found in two steps -- the group of 16 bins from the chunks' coarse counts, then
// the bin from that group's 16 counts of each chunk -- with the keys of B1 (sh.cnt) and above it
// (sh.above), and the normaliser.
template <int KPT>
__device__ __forceinline__ void pass1_last_sorted(const SelArgs &a, const Chunk<KPT> &c, SelShared &sh) {
  constexpr int UNROLL = 8;
  const int tid = threadIdx.x;
  const uint32_t kc = (uint32_t)c.kc;
  if (tid < c.G) sh.r2c[tid] = __builtin_bit_cast(float, a.chunk[(int64_t)(c.g0 + tid) * kQChunkWords + CK_SUMSQ]);
  if (tid == 0) {                 // exactly one group and one bin qualify; these only keep indexes in range
    sh.d = 0;
    sh.above = 0;
    sh.cnt = c.n;
  }
  // coarse: thread t sums group 255 - (t % 256) over the even (t < 256) or odd chunks
  {
    const int g = kQGroups - 1 - (tid & (kQGroups - 1)), half = tid >> 8;
    const uint32_t *cb = a.coarse + (int64_t)c.g0 * kQGroups + g;
    uint32_t acc = 0u;
    for (int w0 = half; w0 < c.G; w0 += 2 * UNROLL) {
      uint32_t x[UNROLL];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) x[u] = cb[(int64_t)min(w0 + 2 * u, c.G - 1) * kQGroups];   // all in flight
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) acc += w0 + 2 * u < c.G ? x[u] : 0u;
    }
    sh.hist[half * kQGroups + g] = acc;
  }
  __syncthreads();
  if (tid < kQGroups) {
    const int g = kQGroups - 1 - tid;
    const uint32_t above = sh.hist[g] + sh.hist[kQGroups + g];                              // keys above group g
    const uint32_t ge = g > 0 ? sh.hist[g - 1] + sh.hist[kQGroups + g - 1] : (uint32_t)c.n;  // keys at or above it
    if (above < kc && kc <= ge) {
      sh.d = g;
      sh.above = (int)above;
      sh.cnt = (int)ge;
    }
  }
  for (int i = tid; i < 16; i += kQThreads) sh.hist[2 * kQGroups + i] = 0u;
  __syncthreads();
  // fine: the 16 bins of group C, chunk t / 16 (and t / 16 + 32), bin t % 16
  const int C = min(max(sh.d, 0), kQGroups - 1);
  const uint32_t ge_group = (uint32_t)sh.cnt;
  {
    const int j = tid & 15;
    uint32_t v = 0u;
    for (int w = tid >> 4; w < c.G; w += kQThreads / 16) v += a.hist1[(int64_t)(c.g0 + w) * kQBins1 + 16 * C + j];
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    if ((tid & 63) < 16) atomicAdd(&sh.hist[2 * kQGroups + j], v);
  }
  __syncthreads();
  if (tid < 16) {
    const uint32_t above = sh.hist[2 * kQGroups + tid];
    const uint32_t ge = tid > 0 ? sh.hist[2 * kQGroups + tid - 1] : ge_group;
    if (above < kc && kc <= ge) {
      sh.d = 16 * C + tid;
      sh.cnt = (int)(ge - above);
      sh.above = (int)above;
    }
  }
  __syncthreads();
  if (tid == 0) {
    float sq = 0.f;
    for (int w = 0; w < c.G; ++w) sq += sh.r2c[w];
    c.sq_rec[SQ_B1] = (uint32_t)sh.d;
    c.sq_rec[SQ_R1] = (uint32_t)(c.kc - sh.above);
    c.sq_rec[SQ_RNORM] = __builtin_bit_cast(uint32_t, rsqrtf(sq / (float)c.n + a.eps));
    c.sq_rec[SQ_CNT1] = 0u;           // every chunk has arrived: reset for the next call
  }
}

// Pass-1 last arrival of the one-launch form, when digit B1 holds at most kQLdsCand keys: those
// keys, read from the chunks' ordered lists, resolve T, the ties still needed and each chunk's quota
// in LDS -- what pass2_last writes, without a second pass over the chunks.
template <int KPT>
__device__ void resolve_in_lds(const SelArgs &a, const Chunk<KPT> &c, SelShared &sh, uint32_t *ckey,
                               uint32_t *cchunk) {
  constexpr int CHUNK = Chunk<KPT>::CHUNK;
  constexpr int UNROLL = kQLdsCand / kQThreads;
  const int tid = threadIdx.x;
  const uint32_t B1 = (uint32_t)sh.d;
  const int r1 = c.kc - sh.above;
  // each chunk's range of digit-B1 keys in its ordered list, and where it goes in LDS
  if (tid < 64) {
    int lo = 0, len = 0;
    if (tid < c.G) {
      const uint32_t *cw = a.hist1 + (int64_t)(c.g0 + tid) * kQBins1;
      lo = min((int)cw[B1], CHUNK);   // (the bounds hold by construction; they keep every read in range)
      len = min(max((B1 > 0 ? (int)cw[B1 - 1] : min(CHUNK, c.n - tid * CHUNK)) - lo, 0), CHUNK - lo);
    }
    const int incl = wave_incl_scan(len);
    if (tid < c.G) {
      sh.coff[tid] = incl - len;
      sh.clo[tid] = lo;
      sh.tie[tid] = 0;
      sh.gt[tid] = 0;
    }
    if (tid == 63) sh.ctot = incl;
  }
  for (int i = tid; i < kQBins2; i += kQThreads) sh.hist[i] = 0u;
  __syncthreads();
  const int nc = min(sh.ctot, kQLdsCand);
  if (nc > 0) {
    const int rounds = (nc + kQThreads - 1) / kQThreads;
    uint32_t kk[UNROLL];
    int wk[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {   // every load in flight at once (indices past nc repeat the last)
      if (u >= rounds) break;
      const int i = min(tid + u * kQThreads, nc - 1);
      int lo = 0, hi = c.G - 1;          // the last chunk whose range starts at or before i
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (sh.coff[mid] <= i) lo = mid; else hi = mid - 1;
      }
      wk[u] = lo;
      kk[u] = a.sorted[(int64_t)(c.g0 + lo) * CHUNK + sh.clo[lo] + (i - sh.coff[lo])];
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      if (u >= rounds) break;
      const int i = tid + u * kQThreads;
      if (i < nc) {
        ckey[i] = kk[u];
        cchunk[i] = (uint32_t)wk[u];
      }
    }
  }
  __syncthreads();
  // digit B2 (bits 19..9) among them
  for (int i = tid; i < nc; i += kQThreads) atomicAdd(&sh.hist[(ckey[i] >> 9) & (kQBins2 - 1)], 1u);
  __syncthreads();
  constexpr int PER = kQBins2 / kQThreads;
  const int bin0 = kQBins2 - PER * (tid + 1);
  uint32_t tv[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) tv[j] = sh.hist[bin0 + j];
  find_digit<PER>(tv, bin0, r1, sh.w, &sh.d, &sh.cnt, &sh.above);
  const uint32_t pre = (B1 << 11) | (uint32_t)sh.d;
  const int r2 = r1 - sh.above;
  for (int i = tid; i < kQBins3; i += kQThreads) sh.hist[i] = 0u;
  __syncthreads();
  // the last digit (bits 8..0) among the keys of prefix B1.B2
  for (int i = tid; i < nc; i += kQThreads) {
    const uint32_t k = ckey[i];
    if ((k >> 9) == pre) atomicAdd(&sh.hist[k & (kQBins3 - 1)], 1u);
  }
  __syncthreads();
  uint32_t tv3[1] = {sh.hist[kQBins3 - 1 - tid]};
  find_digit<1>(tv3, kQBins3 - 1 - tid, r2, sh.w, &sh.d, &sh.cnt, &sh.above);
  const uint32_t T = (pre << 9) | (uint32_t)sh.d;
  const int rT = r2 - sh.above;                       // ties of T still needed
  for (int i = tid; i < nc; i += kQThreads) {
    const uint32_t k = ckey[i];
    if (k >= T) atomicAdd(k == T ? &sh.tie[cchunk[i]] : &sh.gt[cchunk[i]], 1);
  }
  __syncthreads();
  // each chunk's quota of ties (lowest positions first) and output offset: its keys above digit B1,
  // its digit-B1 keys above T and its quota, summed over the chunks before it (wave 0, a lane per
  // chunk in position order)
  if (tid < 64) {
    const bool in = tid < c.G;
    const int tie = in ? sh.tie[tid] : 0;
    const int q = in ? max(0, min(tie, rT - (wave_incl_scan(tie) - tie))) : 0;
    const int kept = in ? sh.clo[tid] + sh.gt[tid] + q : 0;
    const int off = wave_incl_scan(kept) - kept;
    if (in) {
      uint32_t *ck = a.chunk + (int64_t)(c.g0 + tid) * kQChunkWords;
      ck[CK_QUOTA] = (uint32_t)q;
      ck[CK_OFF] = (uint32_t)off;
    }
    if (tid == 0) c.sq_rec[SQ_T] = T;
  }
}

template <int KPT>
__global__ __launch_bounds__(kQThreads) void gate_select_fused_kernel(SelArgs a) {
  constexpr int POOL = KPT * kQThreads > 2 * kQLdsCand ? KPT * kQThreads : 2 * kQLdsCand;
  __shared__ SelShared sh;
  __shared__ __align__(16) uint32_t pool[POOL];     // pass 1: the ordered keys; then the digit-B1 keys
  if ((int)blockIdx.x >= a.n_sel) {      // prefix / suffix rows: no counters, no waits
    write_meta_rows(a, (int64_t)blockIdx.x - a.n_sel);
    return;
  }
  for (int i = threadIdx.x; i < kQBins1; i += kQThreads) sh.hist[i] = 0u;   // pass 1's histogram, while
  if (threadIdx.x == 0) sh.base = 0;                                         // the keys load
  __syncthreads();
  Chunk<KPT> c;
  c.init(a, blockIdx.x);
  uint32_t *flag = c.sq_rec + SQ_FLAG;
  pass1_chunk_sorted<KPT>(a, c, sh, pool);
  if (arrive_last(c.sq_rec + SQ_CNT1, c.G, &sh.flag)) {
    pass1_last_sorted<KPT>(a, c, sh);
    // phase 3 when T and the offsets are resolved here (digit B1 small enough for LDS), else
    // phase 1: pass 2 runs, then phase 2 and the compaction's look-back
    const bool in_lds = sh.cnt <= kQLdsCand;
    if (in_lds) resolve_in_lds<KPT>(a, c, sh, pool, pool + kQLdsCand);
    raise_flag(flag, in_lds ? 3u : 1u);
  }
  if (wait_flag(a, flag, 1u, &sh.flag) == 3u) {
    // resolved: the flag is not read again and the look-back words not at all, so the chunk counts
    // itself done now (the count's latency hides behind the compaction); the last one resets
    uint32_t prev = 0u;
    if (threadIdx.x == 0)
      prev = __hip_atomic_fetch_add(c.sq_rec + SQ_DONE, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    compact_chunk<KPT>(a, c, sh, true);
    if (threadIdx.x == 0 && prev == (uint32_t)(c.G - 1)) {
      c.sq_rec[SQ_FLAG] = 0u;
      c.sq_rec[SQ_DONE] = 0u;
    }
    return;
  }
  pass2_chunk<KPT>(a, c, sh);
  if (arrive_last(c.sq_rec + SQ_CNT2, c.G, &sh.flag)) {
    pass2_last<KPT>(a, c, sh);
    raise_flag(flag, 2u);
  }
  wait_flag(a, flag, 2u, &sh.flag);
  compact_chunk<KPT>(a, c, sh, false);
  seq_done(a, c.sq_rec, c.g0, c.G, sh);
}

// Workspace layout for up to seq_cap sequences and chunk_cap chunks.  The counters that must be
// zero when a call starts (global words, per-sequence records) come first at offsets that depend
// only on the capacities, so calls of any size within them find the counters the previous call
// left zeroed.
int64_t ws_layout(int32_t seq_cap, int32_t chunk_cap, int64_t off[8]) {
  int64_t o = 0;
  auto take = [&](int64_t bytes) { const int64_t r = o; o += (bytes + 255) / 256 * 256; return r; };
  off[0] = take(64 * 4);                                       // global words
  off[1] = take((int64_t)seq_cap * kQSeqWords * 4);            // sequence records
  off[2] = take((int64_t)chunk_cap * kQChunkWords * 4);        // chunk records
  off[3] = take((int64_t)chunk_cap * kQBins1 * 4);             // hist1
  off[4] = take((int64_t)chunk_cap * kQBins2 * 4);             // hist2
  off[5] = take((int64_t)seq_cap * kQCap * 8);                 // candidates
  off[6] = take((int64_t)std::min(chunk_cap, kQFusedMaxChunks) * kQMaxChunkKeys * 4);   // ordered keys
  off[7] = take((int64_t)std::min(chunk_cap, kQFusedMaxChunks) * kQGroups * 4);         // coarse counts
  return o;
}

template <int KPT>
void launch_select(const SelArgs &a, int grid, bool fused, hipStream_t stream) {
  if (fused) {
    hipLaunchKernelGGL(gate_select_fused_kernel<KPT>, dim3(grid), dim3(kQThreads), 0, stream, a);
    return;
  }
  hipLaunchKernelGGL(gate_select1_kernel<KPT>, dim3(a.n_sel), dim3(kQThreads), 0, stream, a);
  hipLaunchKernelGGL(gate_select2_kernel<KPT>, dim3(a.n_sel), dim3(kQThreads), 0, stream, a);
  hipLaunchKernelGGL(gate_compact_kernel<KPT>, dim3(grid), dim3(kQThreads), 0, stream, a);
}

}  // namespace
}  // namespace tg

using namespace tg;

extern "C" int64_t tg_gate_select_pack_workspace_size(int32_t seq_capacity, int32_t chunk_capacity) {
  if (seq_capacity <= 0 || chunk_capacity < 0) return 0;
  int64_t off[8];
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
  TG_CHECK(keys_per_thread == 4 || keys_per_thread == 8 || keys_per_thread == 16 || keys_per_thread == 32,
           "keys_per_thread must be 4, 8, 16 or 32");
  if (num_seqs == 0 || total_kept == 0) return 0;
  TG_CHECK(num_seqs <= seq_capacity && n_select_wgs <= chunk_capacity,
           "workspace capacity (%d sequences, %d chunks) below this call's (%d, %d)", seq_capacity, chunk_capacity,
           num_seqs, n_select_wgs);
  TG_CHECK((reinterpret_cast<uintptr_t>(workspace) & 255) == 0, "workspace must be 256-byte aligned");
  const int64_t meta_wgs = (total_kept + kQThreads - 1) / kQThreads;   // prefix / suffix rows, 512 per workgroup
  TG_CHECK((int64_t)n_select_wgs + meta_wgs < (1ll << 31), "grid too large");
  int64_t off[8];
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
  a.sorted = reinterpret_cast<uint32_t *>(w + off[6]);
  a.coarse = reinterpret_cast<uint32_t *>(w + off[7]);
  a.spin_limit = 1 << 22;
  const int grid = (int)(n_select_wgs + meta_wgs);
  // one launch when every chunk workgroup fits the chip at once (its waits are for chunks of the
  // same sequence, which must be resident); three otherwise
  const bool fused = n_select_wgs <= std::min(device_cus(), std::min(chunk_capacity, kQFusedMaxChunks));
  if (n_select_wgs == 0) {
    hipLaunchKernelGGL(gate_compact_kernel<8>, dim3(grid), dim3(kQThreads), 0, stream, a);
  } else {
    switch (keys_per_thread) {
      case 4: launch_select<4>(a, grid, fused, stream); break;
      case 8: launch_select<8>(a, grid, fused, stream); break;
      case 16: launch_select<16>(a, grid, fused, stream); break;
      default: launch_select<32>(a, grid, fused, stream); break;
    }
  }
  TG_HIP_CHECK(hipPeekAtLastError());
  // the rows themselves: the pack over the keep lists just written (positions and bias are done)
  if (n_streams > 0)
    return gate_pack_launch(streams, n_streams, keep, geom, num_seqs, total_kept, nullptr, nullptr, nullptr, rms_eps,
                            nullptr, a.glob + GL_ERROR, stream);
  return 0;
}
