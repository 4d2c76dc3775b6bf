// Key-bias causal GQA attention, forward, for gfx950 (MI355X).
//
// Math (reference: kernels/fa2bias/keybias.patch:279-332, 394-464 and keybias.py:40-49,85-87):
//   z[i,j]  = scale * (q_i . k_j + bias_raw[b,h,j]),   masked to -inf for j > i + Sk - Sq (causal)
//   lse[i]  = ln sum_j exp(z[i,j]);   out_i = sum_j exp(z[i,j] - lse[i]) v_j
// with the query head h reading kv head h / (H / Hkv).
//
// Work decomposition (one workgroup = 8 waves = 512 threads per CU, two waves per SIMD; 4-wave
// workgroups, two per CU, when the grid is too small for 8-wave ones):
//   * a workgroup owns one KV head and HP query heads of its GQA group (HP = 2 when the group
//     size is even) over NW * 32/HP consecutive query positions; every K/V tile it streams
//     through LDS serves all HP heads;
//   * each wave owns 32 MFMA columns in two blocks of 16: 32 consecutive query positions of one
//     head (half the waves take each head of a pair), so a wave reads one head's key bias per
//     tile; the KV sequence is streamed in 64-key tiles by LDS DMA (buffer_load ...
//     lds: no staging registers, zero fill past Sk), double-buffered, one barrier per tile, the
//     next tile in flight during compute;
//   * scores are computed transposed, S^T = K Q^T, on v_mfma_f32_16x16x32_bf16 (on gfx950 it
//     sustains ~2.4 PFLOP/s against ~2.0 for the 32x32x16 form): the accumulators then hold
//     one column per lane and block and 16 of its keys, the other 48 in the lanes l^16, l^32,
//     l^48, so the online-softmax max is in-lane plus two permlane swaps;
//   * K rows are stored in LDS in a permuted order (kperm) chosen so that lane group G of a
//     32-key step's S^T accumulators holds keys 8G .. 8G+7; the accumulators, rounded to bf16, are
//     then directly the B operand of O^T = V^T P^T, whose A operand (8 consecutive keys at one d
//     per lane) comes from row-major V through the transposing LDS read ds_read_b64_tr_b16;
//   * O^T accumulates per lane for one column per block, so the per-query rescale is a scalar per
//     lane, and it is applied lazily (only when the running max grows by more than 2^8); the row
//     sums run on the matrix cores too (ones . P^T, the same bf16 weights P V uses);
//   * two waves per SIMD let one wave's softmax (VALU) run under the other's matrix-core work;
//     all NW waves share every K/V tile and each issues 1/NW of its LDS DMA.
// Workgroups are issued heaviest-first (largest query tile first) with the KV head varying
// fastest, so that consecutive workgroups, which land on different XCDs, keep one KV head per
// XCD when Hkv is a multiple of 8.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "tg_common.h"
#include "../../include/tokengate_hip.h"

namespace tg {
namespace {

constexpr int kD = 128;        // head dim
constexpr int kBN = 64;        // keys per tile
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// A wave's 32 MFMA columns are 32 consecutive query positions of one head; a workgroup of NW waves
// covers NW * 32/HP positions of its HP heads.  NW = 8 (two waves per SIMD, one workgroup per CU)
// unless the grid would then be too small to fill the chip, where NW = 4 (two workgroups per CU)
// halves the query tile.
template <int HP> constexpr int qpw() { return 32 / HP; }
template <int NW, int HP> constexpr int bm() { return NW * qpw<HP>(); }
constexpr int kQW = 32;   // query positions per wave

constexpr int kKRowBytes = kD * 2;      // one K or V row in LDS (256 B, 16 chunks of 16 B)
constexpr int kKTileBytes = kBN * kKRowBytes;
constexpr int kStages = 2;              // K/V/bias ring: tile t resident, tile t+1 in flight

struct FwdArgs {
  const bf16_t *q, *k, *v;
  const float *bias;
  bf16_t *o;
  float *lse;
  const int32_t *cu_seqlens;   // varlen only: query rows of sequence b are cu_seqlens[b] .. [b+1]-1
  // varlen key geometry when the keys live elsewhere (a cache with room after each sequence):
  // keys of sequence b are rows cu_k[b] .. cu_k[b] + used_k[b] - 1 (used_k NULL: cu_k[b + 1] - 1);
  // cu_k NULL: the keys are the query rows
  const int32_t *cu_k, *used_k;
  int64_t q_bs, q_rs, q_hs, k_bs, k_rs, k_hs, v_bs, v_rs, v_hs, o_bs, o_rs, o_hs;
  int64_t bias_bs, bias_hs;
  int64_t lse_total;           // varlen: total rows (lse is (H, total)); dense: unused
  int batch;                   // dense: B; varlen: number of sequences
  int sq, sk;                  // dense lengths (varlen: per sequence, read from cu_seqlens)
  int h, hkv, group;
  int n_qtiles;
  float scale_log2;            // softmax_scale * log2(e)
  // Key-range split of the heaviest query tiles (small grids): the n_heavy heaviest query tiles
  // of every (sequence, head group) are each processed by ns workgroups over consecutive key
  // ranges; each writes a partial result (O normalised by its own row sum, bf16, and the running
  // max / row sum) and the combine kernel merges them.  ns = 1, n_heavy = 0: no split.
  int ns, n_heavy;
  int64_t heavy_blocks;        // n_heavy * ns * (head groups) * batch: the grid's leading part
  bf16_t *ws_o;                // [heavy unit][chunk][wave][8][64 lanes] x 16 B
  float *ws_ml;                // [heavy unit][chunk][wave][column block][64 lanes] x (m, l)
};

// LDS row lr of a 64-key tile holds key kperm(lr): within each 32-key step, S^T block kb' (rows
// 16kb' .. 16kb'+15) row m carries key 8(m/4) + 4kb' + m%4, so that lane group G of the two S^T
// accumulators of a step holds keys 8G .. 8G+7 of the step — exactly the k range of the B operand
// (P^T) of O^T += V^T P^T for that step.
__device__ __forceinline__ int kperm(int lr) {
  const int m = lr & 15;
  return 32 * (lr >> 5) + 8 * (m >> 2) + 4 * ((lr >> 4) & 1) + (m & 3);
}

// Lazy rescaling threshold (log2 units): the running max used for exp2 is raised only when a tile
// exceeds it by more than this, so P <= 2^8 (exact in bf16's exponent range) and the O rescale
// is skipped on almost every tile.
constexpr float kRescaleTau = 8.0f;

// LDS tile layouts (64 keys x 128 d, 256 B per row, 16-byte chunks):
//   K: row lr holds key kperm(lr); logical chunk c at physical chunk c ^ (lr%16)
//      -> the S^T A-operand read (16 consecutive rows, one chunk per 16 lanes) is conflict free.
//   V: row = key (natural order); logical chunk c at physical chunk c ^ vswz(key), vswz moving
//      32-byte pairs of chunks by (key%4) + 4((key/8)%2), so that the transposing reads of half a
//      wave (8 keys x the same 32 bytes) fall on 8 different 32-byte bank groups.
// Both are filled by LDS DMA straight from global memory (no staging registers); keys past Sk
// read as zero through the buffer descriptor's range check.
__device__ __forceinline__ int vswz(int key) { return 2 * ((key & 3) | (((key >> 3) & 1) << 2)); }

// v_max3_f32 without the canonicalising v_max the compiler adds in IEEE mode (the inputs are
// MFMA results or -inf, never signalling NaNs).
__device__ __forceinline__ float vmax3(float a, float b, float c) {
  float d;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}

// Wave w owns head wave_head(w) of the workgroup's HP heads (waves 0 .. NW/2-1 the first of a pair,
// the others the second) at positions wave_pos(w) .. +31 of the workgroup's query tile; its column
// block cb (0, 1) is positions 16 cb .. 16 cb + 15 of those, lane l holding column l%16 of each.
// One head per wave means one bias row per wave.
template <int NW, int HP> __device__ __forceinline__ int wave_head(int w) { return HP == 2 ? w / (NW / 2) : 0; }
template <int NW, int HP> __device__ __forceinline__ int wave_pos(int w) { return kQW * (HP == 2 ? w % (NW / 2) : w); }
__device__ __forceinline__ int col_query(int cb, int c16) { return 16 * cb + c16; }

template <int NW, int HP, bool CAUSAL, bool HAS_BIAS, bool VARLEN>
__global__ __launch_bounds__(64 * NW, 8 / NW) void keybias_fwd_kernel(FwdArgs a) {
  constexpr int kWaves = NW;
  constexpr int BM = bm<NW, HP>();
  // One __shared__ object per ring slot: the compiler separates LDS-DMA writes from LDS reads only
  // across distinct objects, so the DMA of tile t+1 does not hold up the reads of tile t.
  static_assert(kStages == 2, "two named LDS objects per operand");
  __shared__ __attribute__((aligned(1024))) char ks0[kKTileBytes], ks1[kKTileBytes];
  __shared__ __attribute__((aligned(1024))) char vs0[kKTileBytes], vs1[kKTileBytes];
  // bias rows padded by 4 floats so that the two heads' rows fall on different banks
  __shared__ __attribute__((aligned(256))) float bs0[HP][kBN + 4], bs1[HP][kBN + 4];
  auto kslot = [&](auto b) -> char * { if constexpr (decltype(b)::value == 0) return ks0; else return ks1; };
  auto vslot = [&](auto b) -> char * { if constexpr (decltype(b)::value == 0) return vs0; else return vs1; };
  auto bslot = [&](auto b) -> float (*)[kBN + 4] {
    if constexpr (decltype(b)::value == 0) return bs0; else return bs1;
  };

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int c16 = lane & 15;     // MFMA column within each 16-column block
  const int G = lane >> 4;       // lane group: rows 4G .. 4G+3 of every 16x16 accumulator

  // ---- which (query tile, sequence, kv head, head pair) this workgroup owns ----
  const int hgroups = a.group / HP;
  const int per_q = a.hkv * hgroups;
  const int bid = blockIdx.x;
  const int x = bid % per_q;
  const int kh = x % a.hkv;
  const int hg = x / a.hkv;
  // Dense: heaviest q tile of every batch row first.  Varlen: sequence-major (all tiles of
  // sequence b before sequence b+1, heaviest first within it), so the workgroups resident at one
  // time share one sequence's K/V in L2 / MALL instead of streaming every sequence's K/V at once.
  // A split launch lists the chunks of the n_heavy heaviest tiles first, then the other tiles.
  int b, rank, chunk = -1;
  int64_t hunit = 0;
  if (bid < a.heavy_blocks) {
    const int r = bid / per_q;
    chunk = r % a.ns;
    const int r2 = r / a.ns;
    b = VARLEN ? r2 / a.n_heavy : r2 % a.batch;
    rank = VARLEN ? r2 % a.n_heavy : r2 / a.batch;
    hunit = (int64_t)r2 * per_q + x;
  } else {
    const int r2 = (int)((bid - a.heavy_blocks) / per_q);
    const int n_light = a.n_qtiles - a.n_heavy;
    b = VARLEN ? r2 / n_light : r2 % a.batch;
    rank = a.n_heavy + (VARLEN ? r2 % n_light : r2 / a.batch);
  }
  const int qt = a.n_qtiles - 1 - rank;

  int sq = a.sq, sk = a.sk;
  int64_t row0 = 0, krow0 = 0;
  if constexpr (VARLEN) {
    const int s0 = a.cu_seqlens[b], s1 = a.cu_seqlens[b + 1];
    row0 = s0;
    sq = min(s1 - s0, a.sq);   // rows past max_seqlen are outside the bias row: not computed
    if (a.cu_k != nullptr) {
      krow0 = a.cu_k[b];
      const int nk = a.used_k != nullptr ? a.used_k[b] : a.cu_k[b + 1] - a.cu_k[b];
      sk = max(0, min(nk, a.sk));
    } else {
      krow0 = row0;
      sk = sq;
    }
  }
  const int q0 = qt * BM;
  if (q0 >= sq) return;   // workgroup-uniform: past the end of this sequence
  const int off = sk - sq;   // causal: query i sees keys j <= i + off (bottom-right aligned)
  const int h0 = kh * a.group + hg * HP;

  const bf16_t *qbase = a.q + (VARLEN ? row0 * a.q_rs : (int64_t)b * a.q_bs) + (int64_t)h0 * a.q_hs;
  const bf16_t *kbase = a.k + (VARLEN ? krow0 * a.k_rs : (int64_t)b * a.k_bs) + (int64_t)kh * a.k_hs;
  const bf16_t *vbase = a.v + (VARLEN ? krow0 * a.v_rs : (int64_t)b * a.v_bs) + (int64_t)kh * a.v_hs;
  bf16_t *obase = a.o + (VARLEN ? row0 * a.o_rs : (int64_t)b * a.o_bs) + (int64_t)h0 * a.o_hs;

  // Buffer descriptors: exactly the bytes of rows [0, sk) of this (sequence, kv head).
  const uint32_t kspan = sk > 0 ? (uint32_t)(((int64_t)(sk - 1) * a.k_rs + kD) * 2) : 0u;
  const uint32_t vspan = sk > 0 ? (uint32_t)(((int64_t)(sk - 1) * a.v_rs + kD) * 2) : 0u;
  const brsrc_t krs = make_rsrc(kbase, kspan);
  const brsrc_t vrs = make_rsrc(vbase, vspan);
  // the bias row of head h0 + w is loaded by wave w < HP, through a descriptor of exactly its sk
  // columns: columns past the sequence's keys read as 0 (whatever the table holds there)
  const int bwave = __builtin_amdgcn_readfirstlane(wave < HP ? wave : 0);
  const float *bbase =
      HAS_BIAS ? a.bias + (int64_t)b * a.bias_bs + (int64_t)(h0 + bwave) * a.bias_hs : nullptr;
  const brsrc_t brs = make_rsrc(bbase, (HAS_BIAS && sk > 0) ? (uint32_t)sk * 4u : 0u);

  // ---- this wave's head and queries, and its Q fragments (B operand of S^T = K Q^T, 32 d per
  // k-step) ----
  const int hw = wave_head<NW, HP>(wave);
  const int qw0 = q0 + wave_pos<NW, HP>(wave);
  int qrow[2];
  bool qvalid[2];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    qrow[cb] = qw0 + col_query(cb, c16);
    qvalid[cb] = qrow[cb] < sq;
  }
  const bool wave_has_rows = qw0 < sq;
  const int qw_hi = min(qw0 + kQW, sq) - 1;
  bf16x8 qf[2][4];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qf[cb][ks] = __builtin_bit_cast(
          bf16x8, gload16(qbase + (int64_t)qrow[cb] * a.q_rs + (int64_t)hw * a.q_hs + 32 * ks + 8 * G, qvalid[cb]));

  int kv_end = sk;
  if constexpr (CAUSAL) kv_end = min(sk, q0 + BM + off);
  const int n_tiles = kv_end > 0 ? (kv_end + kBN - 1) / kBN : 0;
  // key tiles [t_lo, t_hi) of this workgroup (a split tile's chunk covers its share of them)
  int t_lo = 0, t_hi = n_tiles;
  if (chunk >= 0) {
    t_lo = (int)((int64_t)n_tiles * chunk / a.ns);
    t_hi = (int)((int64_t)n_tiles * (chunk + 1) / a.ns);
  }

  // ---- per-lane DMA source offsets (bytes within a tile; + tile * 64 rows per tile) ----
  // A 16 KB tile is 16 wave-loads of 1 KB; wave w issues loads w, w + kWaves, ...
  constexpr int kLoads = kKTileBytes / 1024 / kWaves;
  uint32_t koff[kLoads], voff[kLoads];
#pragma unroll
  for (int it = 0; it < kLoads; ++it) {
    const int slot = wave + it * kWaves;                  // 1 KB slot = 4 rows
    const int lr = slot * 4 + (lane >> 4);                // K LDS row written by this lane
    const int kc = (lane & 15) ^ (lr & 15);               // logical chunk stored there
    koff[it] = (uint32_t)(kperm(lr) * a.k_rs * 2 + kc * 16);
    const int vkey = slot * 4 + (lane >> 4);              // V LDS row (= key) written by this lane
    const int vc = (lane & 15) ^ vswz(vkey);
    voff[it] = (uint32_t)(vkey * a.v_rs * 2 + vc * 16);
  }
  auto issue_tile = [&](int tile, auto buf_c) {
    const uint32_t kb0 = (uint32_t)((int64_t)tile * kBN * a.k_rs * 2);
    const uint32_t vb0 = (uint32_t)((int64_t)tile * kBN * a.v_rs * 2);
    char *kd = kslot(buf_c), *vd = vslot(buf_c);
    // the LDS destination goes to M0: with the wave index in a scalar register it is scalar
    // arithmetic instead of a per-lane add and a readfirstlane per DMA (+0.5 % at 32k)
    const int wv = __builtin_amdgcn_readfirstlane(wave);
#pragma unroll
    for (int it = 0; it < kLoads; ++it) {
      dma16(krs, kd + (wv + it * kWaves) * 1024, kb0 + koff[it]);
      dma16(vrs, vd + (wv + it * kWaves) * 1024, vb0 + voff[it]);
    }
    if constexpr (HAS_BIAS) {
      if (wave < HP)
        dma4(brs, &bslot(buf_c)[wave][0], (uint32_t)((tile * kBN + lane) * 4));
    }
  };

  // V transposed reads (A operand of O^T += V^T P^T: d = 16 dblk + l%16, keys 8G .. 8G+7 of a
  // 32-key step): lane r of group G addresses key 8G + r/4 (+4 for the upper four keys) and the
  // 8 bytes of d = 16 dblk + 4(r%4) .. +3; the transposing read hands lane r the four keys at
  // d = 16 dblk + r.  The swizzle vswz(key) depends only on r/4 and G%2 here.  The lane part of
  // each address is masked to the 8 KB it can reach, which tells the compiler these reads stay
  // inside their ring slot (and need not wait for DMA into the other one).
  const int vsw = 2 * ((c16 >> 2) | ((G & 1) << 2));
  const uint32_t v_lane = (uint32_t)((8 * G + (c16 >> 2)) * kKRowBytes + 16 * ((c16 & 3) >> 1) + 8 * (c16 & 1));
  uint32_t vch[8];
#pragma unroll
  for (int dblk = 0; dblk < 8; ++dblk) vch[dblk] = (v_lane + (uint32_t)(((2 * dblk) ^ vsw) << 4)) & 0x1FF8u;

  f32x4 oacc[2][8];
  // Row sums on the matrix cores: lacc[cb] += ones(16x32) . P^T puts column c's sum of the step's
  // bf16 P values (exactly the weights P V uses) in all four values of every lane of column c, so
  // the softmax spends no VALU on it and needs no cross-lane sum at the end.
  f32x4 lacc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  bf16x8 ones;
#pragma unroll
  for (int i = 0; i < 8; ++i) ones[i] = (__bf16)1.0f;
  // Per column block: the running max mrun (log2 units), -mrun as the exponent offset (0 before the
  // first visible key), and the tile max in raw-score units above which mrun is raised; all three
  // change only when the running max is raised.
  float mrun[2] = {-INFINITY, -INFINITY}, mneg[2] = {0.f, 0.f}, thr[2] = {-INFINITY, -INFINITY};
  const float inv_scale_log2 = 1.f / a.scale_log2;
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int d = 0; d < 8; ++d) oacc[cb][d] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Two-slot ring, unrolled by two so that every slot index is a compile-time constant: tile t
  // lives in slot t % 2; at the top of tile t this wave's DMA for t is complete (nothing later
  // is in flight yet), the barrier makes every wave's part visible and frees the slot of t-1,
  // and tile t+1 is issued into it while tile t is computed.
  auto tile_step = [&](int t, auto buf_c) {
    constexpr int BUF = decltype(buf_c)::value;
    const int n0 = t * kBN;
    wait_vm<0>();
    ring_barrier();
    if (t + 1 < t_hi) issue_tile(t + 1, std::integral_constant<int, 1 - BUF>());
    if (!wave_has_rows || (CAUSAL && n0 > qw_hi + off)) return;

    // ---- S^T = K Q^T + bias: 2 column blocks x 4 key blocks x 4 d-steps.  The accumulators start
    // from the bias of their keys (raw-score units), so the bias add costs no VALU work. ----
    f32x4 sacc[2][4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      if constexpr (HAS_BIAS) {
        // both column blocks are the wave's head: one read of its 16 keys' bias serves both
        sacc[0][kb] = *reinterpret_cast<const f32x4 *>(&bslot(buf_c)[hw][32 * (kb >> 1) + 8 * G + 4 * (kb & 1)]);
      } else {
        sacc[0][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      sacc[1][kb] = sacc[0][kb];
    }
    // all 16 K fragments of the tile are read before the first MFMA, so LDS latency is paid once
    bf16x8 kfr[4][4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const int lr = 16 * kb + c16;
        kfr[kb][ks] = lds_load16(kslot(buf_c), lr * kKRowBytes + ((uint32_t)((4 * ks + G) ^ c16) << 4));
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) sacc[cb][kb] = mfma16(kfr[kb][ks], qf[cb][ks], sacc[cb][kb]);
      }
    }

    // ---- online softmax: lane holds 16 keys of one column per block; the other 48 keys of that
    // column sit in lanes l^16, l^32, l^48 ----
    const bool need_mask = (n0 + kBN > sk) || (CAUSAL && n0 + kBN - 1 > qw0 + off);
    if (need_mask) {
      // key > lim -> -inf by adding 0 or -inf, selected by the sign of lim - key (an arithmetic
      // shift the compiler cannot turn back into per-element compares, whose 64-bit results would
      // crowd the scalar registers)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        int lim = sk - 1;
        if constexpr (CAUSAL) lim = min(lim, qrow[cb] + off);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          const int rel = lim - (n0 + 32 * (kb >> 1) + 8 * G + 4 * (kb & 1));
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            int sgn;
            asm("v_ashrrev_i32 %0, 31, %1" : "=v"(sgn) : "v"(rel - i));   // -1 where key > lim
            const float pen = __builtin_bit_cast(float, (uint32_t)sgn & 0xFF800000u);
            sacc[cb][kb][i] += pen;
          }
        }
      }
    }
    float mt[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const f32x4 *s = sacc[cb];
      const float m0 = vmax3(s[0][0], s[0][1], s[0][2]), m1 = vmax3(s[0][3], s[1][0], s[1][1]);
      const float m2 = vmax3(s[1][2], s[1][3], s[2][0]), m3 = vmax3(s[2][1], s[2][2], s[2][3]);
      const float m4 = vmax3(s[3][0], s[3][1], s[3][2]);
      mt[cb] = vmax3(vmax3(m0, m1, m2), vmax3(m3, m4, s[3][3]), m0);
    }
    // Both column blocks' maxima over the four lane groups in three permlane swaps:
    // swap16(cb0, cb1) + max leaves cb0's pair maxima (groups 0|1, 2|3) in groups 0 and 2 and cb1's
    // in groups 1 and 3; swap32 + max folds the halves; a last swap16 of that value with itself
    // returns (cb0's max in every lane, cb1's max in every lane).  Raw-score units, -inf if the
    // tile is fully masked for the column.
    float mxr[2];
    {
      const float x = swap_pair_max(__builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, mt[0]),
                                                                     __builtin_bit_cast(uint32_t, mt[1]), false, false));
      const float y = half_swap_max(x);
      const auto sw = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, y), __builtin_bit_cast(uint32_t, y),
                                                       false, false);
      const uint32_t lo = sw[0], hi = sw[1];
      mxr[0] = u32_as_f32(lo);
      mxr[1] = u32_as_f32(hi);
    }
    if (__builtin_amdgcn_ballot_w64(mxr[0] > thr[0] || mxr[1] > thr[1]) != 0) {
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const float m_new = fmaxf(mrun[cb], mxr[cb] * a.scale_log2);
        // 0 on the first visible tile; columns that have seen no key yet (m_new = -inf) keep 1.
        const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(mrun[cb] - m_new);
        mrun[cb] = m_new;
        mneg[cb] = m_new == -INFINITY ? 0.f : -m_new;
        thr[cb] = (m_new + kRescaleTau) * inv_scale_log2;
        lacc[cb] *= alpha;
#pragma unroll
        for (int d = 0; d < 8; ++d) oacc[cb][d] *= alpha;
      }
    }
    // P rounded to bf16 pairs (the B operand of P V and of the row-sum product)
    uint32_t pk[2][4][2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
          const float p0 = fast_exp2(fmaf(sacc[cb][kb][i], a.scale_log2, mneg[cb]));
          const float p1 = fast_exp2(fmaf(sacc[cb][kb][i + 1], a.scale_log2, mneg[cb]));
          pk[cb][kb][i >> 1] = pack_bf16x2(p0, p1);
        }
      }
    }

    // ---- O^T += V^T P^T: 2 key steps x 8 d-blocks x 2 column blocks ----
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      bf16x8 pb[2];
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const u32x4 w = {pk[cb][2 * st][0], pk[cb][2 * st][1], pk[cb][2 * st + 1][0], pk[cb][2 * st + 1][1]};
        pb[cb] = __builtin_bit_cast(bf16x8, w);
      }
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) lacc[cb] = mfma16(ones, pb[cb], lacc[cb]);
      const uint32_t krow = (uint32_t)(32 * st * kKRowBytes);
#pragma unroll
      for (int dblk = 0; dblk < 8; ++dblk) {
        const s16x4 lo = lds_read_tr16(vslot(buf_c) + krow + vch[dblk]);
        const s16x4 hi = lds_read_tr16(vslot(buf_c) + krow + 4 * kKRowBytes + vch[dblk]);
        const bf16x8 vf = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) oacc[cb][dblk] = mfma16(vf, pb[cb], oacc[cb][dblk]);
      }
    }
  };
  if (t_lo < t_hi) issue_tile(t_lo, std::integral_constant<int, 0>());
  int t = t_lo;
  for (; t + 1 < t_hi; t += 2) {
    tile_step(t, std::integral_constant<int, 0>());
    tile_step(t + 1, std::integral_constant<int, 1>());
  }
  if (t < t_hi) tile_step(t, std::integral_constant<int, 0>());

  // ---- epilogue: normalise, write O (bf16) and LSE (natural log) ----
  float l[2], inv[2];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    l[cb] = lacc[cb][0];
    inv[cb] = l[cb] > 0.f ? 1.f / l[cb] : 0.f;
  }
  if (chunk >= 0) {
    // partial result of this key chunk: O / l as bf16 (piece j = 4 cb + p holds d-blocks 2p and
    // 2p+1 of column block cb; each piece a coalesced 1 KB wave store) and, per column block,
    // (running max in log2 units, row sum l)
    const int64_t pw = (hunit * a.ns + chunk) * kWaves + wave;
    u32x4 *po = reinterpret_cast<u32x4 *>(a.ws_o) + pw * (8 * 64) + lane;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int cb = j >> 2, p = j & 3;
      const f32x4 &o0 = oacc[cb][2 * p], &o1 = oacc[cb][2 * p + 1];
      const float s = inv[cb];
      const u32x4 w = {pack_bf16x2(o0[0] * s, o0[1] * s), pack_bf16x2(o0[2] * s, o0[3] * s),
                       pack_bf16x2(o1[0] * s, o1[1] * s), pack_bf16x2(o1[2] * s, o1[3] * s)};
      po[j * 64] = w;
    }
    float2 *pml = reinterpret_cast<float2 *>(a.ws_ml) + pw * 128 + lane;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      float2 ml;
      ml.x = mrun[cb];
      ml.y = l[cb];
      pml[cb * 64] = ml;
    }
    return;
  }
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    if (!qvalid[cb]) continue;
    const int hl = hw;
    bf16_t *orow = obase + (int64_t)qrow[cb] * a.o_rs + (int64_t)hl * a.o_hs;
    const float s = inv[cb];
#pragma unroll
    for (int dblk = 0; dblk < 8; ++dblk) {
      const f32x4 &o = oacc[cb][dblk];
      const u32x2 w = {pack_bf16x2(o[0] * s, o[1] * s), pack_bf16x2(o[2] * s, o[3] * s)};
      *reinterpret_cast<u32x2 *>(orow + 16 * dblk + 4 * G) = w;
    }
    if (G == 0) {
      const float lse = l[cb] > 0.f ? (mrun[cb] + __log2f(l[cb])) * kLn2 : INFINITY;
      const int hh = h0 + hl;
      if constexpr (VARLEN)
        a.lse[(int64_t)hh * a.lse_total + row0 + qrow[cb]] = lse;
      else
        a.lse[((int64_t)b * a.h + hh) * sq + qrow[cb]] = lse;
    }
  }
}

// Merge of the key chunks of every split query tile.  A 512-thread workgroup covers 8 / CG of the
// eight 16-byte pieces (8 O values of each of the 64 lanes of one forward wave) of one split
// tile; per piece, thread (group cg, lane) folds chunks cg, cg + CG, ... of its column and group 0
// merges the CG partial results through LDS, so that a long chunk list (a decode row over a long
// cache) is walked CG ways in parallel.
// With chunk c's running max m_c (log2 units), row sum l_c and normalised partial O_c:
// m = max m_c, w_c = l_c 2^(m_c - m), O = sum w_c O_c / sum w_c, lse = (m + log2 sum w_c) ln 2.
// Chunks that saw no key (l_c = 0) weigh nothing.
constexpr int kCombineMaxGroups = 8;
template <int NW, int HP, bool VARLEN>
__global__ __launch_bounds__(512) void keybias_fwd_combine_kernel(FwdArgs a, int CG) {
  constexpr int BM = bm<NW, HP>();
  // (m, wsum, acc[8]) of groups 1..CG-1 of each piece: PP * (CG - 1) < 8 slots
  __shared__ float part[kCombineMaxGroups - 1][10][64];
  const int PP = 8 / CG;                                   // pieces per workgroup
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int cg = wv % CG, pj = wv / CG;
  const int j = (int)(blockIdx.x % CG) * PP + pj;          // piece
  const int wave = (int)((blockIdx.x / CG) % NW);          // forward wave whose columns these are
  const int64_t hunit = (blockIdx.x / CG) / NW;
  float (*mypart)[10][64] = part + pj * (CG - 1);
  const int c16 = lane & 15, G = lane >> 4;
  const int cb = j >> 2, p = j & 3;                        // column block, d-block pair of the piece
  const int hl = wave_head<NW, HP>(wave);
  const int per_q = a.hkv * (a.group / HP);
  const int x = (int)(hunit % per_q), r2 = (int)(hunit / per_q);
  const int kh = x % a.hkv, hg = x / a.hkv;
  const int b = VARLEN ? r2 / a.n_heavy : r2 % a.batch;
  const int rank = VARLEN ? r2 % a.n_heavy : r2 / a.batch;
  const int qt = a.n_qtiles - 1 - rank;
  int sq = a.sq;
  int64_t row0 = 0;
  if constexpr (VARLEN) {
    const int s0 = a.cu_seqlens[b], s1 = a.cu_seqlens[b + 1];
    row0 = s0;
    sq = min(s1 - s0, a.sq);
  }
  const int qw0 = qt * BM + wave_pos<NW, HP>(wave);
  if (qw0 >= sq) return;   // workgroup-uniform: the forward computed nothing for these rows
  const int qrow = qw0 + col_query(cb, c16);
  const bool valid = qrow < sq;

  const float2 *ml = reinterpret_cast<const float2 *>(a.ws_ml);
  const u32x4 *po = reinterpret_cast<const u32x4 *>(a.ws_o);
  const int64_t pw0 = hunit * a.ns * NW + wave;   // chunk c: pw0 + c * NW
  // fold this group's chunks, the weights relative to the largest m seen so far
  float mmax = -INFINITY, wsum = 0.f;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (valid) {
#pragma unroll 4
    for (int c = cg; c < a.ns; c += CG) {
      const int64_t pw = pw0 + (int64_t)c * NW;
      const float2 mc = ml[pw * 128 + cb * 64 + lane];
      const u32x4 pv = po[pw * (8 * 64) + j * 64 + lane];
      if (!(mc.y > 0.f)) continue;
      if (mc.x > mmax) {
        const float sc = fast_exp2(mmax - mc.x);   // 0 while nothing has been added yet
        wsum *= sc;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] *= sc;
        mmax = mc.x;
      }
      const float w = mc.y * fast_exp2(mc.x - mmax);
      wsum += w;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[2 * e] += w * __builtin_bit_cast(float, pv[e] << 16);
        acc[2 * e + 1] += w * __builtin_bit_cast(float, pv[e] & 0xffff0000u);
      }
    }
  }
  if (cg > 0) {
    mypart[cg - 1][0][lane] = mmax;
    mypart[cg - 1][1][lane] = wsum;
#pragma unroll
    for (int i = 0; i < 8; ++i) mypart[cg - 1][2 + i][lane] = acc[i];
  }
  __syncthreads();
  if (cg > 0 || !valid) return;
  for (int q = 0; q < CG - 1; ++q) {
    const float m2 = mypart[q][0][lane], w2 = mypart[q][1][lane];
    if (!(w2 > 0.f)) continue;
    const float mn = fmaxf(mmax, m2);
    const float s1 = fast_exp2(mmax - mn), s2 = fast_exp2(m2 - mn);   // s1 = 0 if mmax = -inf
    wsum = wsum * s1 + w2 * s2;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = acc[i] * s1 + mypart[q][2 + i][lane] * s2;
    mmax = mn;
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  const int h0 = kh * a.group + hg * HP;
  bf16_t *orow = a.o + (VARLEN ? row0 * a.o_rs : (int64_t)b * a.o_bs) + (int64_t)qrow * a.o_rs +
                 (int64_t)(h0 + hl) * a.o_hs;
  // piece j holds d-blocks 2p and 2p+1 of column block cb: d = 32p + 4G + {0..3} and the same + 16
  const int d0 = 32 * p + 4 * G;
  const u32x2 w0 = {pack_bf16x2(acc[0] * inv, acc[1] * inv), pack_bf16x2(acc[2] * inv, acc[3] * inv)};
  const u32x2 w1 = {pack_bf16x2(acc[4] * inv, acc[5] * inv), pack_bf16x2(acc[6] * inv, acc[7] * inv)};
  *reinterpret_cast<u32x2 *>(orow + d0) = w0;
  *reinterpret_cast<u32x2 *>(orow + d0 + 16) = w1;
  if (p == 0 && G == 0) {
    const float lse = wsum > 0.f ? (mmax + __log2f(wsum)) * kLn2 : INFINITY;
    const int hh = h0 + hl;
    if constexpr (VARLEN)
      a.lse[(int64_t)hh * a.lse_total + row0 + qrow] = lse;
    else
      a.lse[((int64_t)b * a.h + hh) * sq + qrow] = lse;
  }
}

template <int NW, int HP, bool CAUSAL, bool HAS_BIAS, bool VARLEN>
void launch_fwd(const FwdArgs &a, int nblocks, hipStream_t stream) {
  hipLaunchKernelGGL((keybias_fwd_kernel<NW, HP, CAUSAL, HAS_BIAS, VARLEN>), dim3(nblocks), dim3(64 * NW), 0,
                     stream, a);
  if (a.heavy_blocks > 0) {
    // chunk groups: up to 8, and at least two chunks per group; CG workgroups of 512 threads per
    // (split tile, forward wave)
    int cgroups = 1;
    while (cgroups < kCombineMaxGroups && 2 * cgroups * 2 <= a.ns) cgroups *= 2;
    const int64_t blocks = a.heavy_blocks / a.ns * NW * cgroups;
    hipLaunchKernelGGL((keybias_fwd_combine_kernel<NW, HP, VARLEN>), dim3((unsigned)blocks), dim3(512), 0, stream, a,
                       cgroups);
  }
}

template <bool VARLEN>
void dispatch_fwd(const FwdArgs &a, int nw, int hp, bool causal, bool has_bias, int nblocks, hipStream_t s) {
#define TG_FWD_CASE(HPV, C, B)                                              \
  if (hp == HPV && causal == C && has_bias == B) {                          \
    if (nw == 8)                                                            \
      launch_fwd<8, HPV, C, B, VARLEN>(a, nblocks, s);                      \
    else                                                                    \
      launch_fwd<4, HPV, C, B, VARLEN>(a, nblocks, s);                      \
    return;                                                                 \
  }
  TG_FWD_CASE(2, true, true)
  TG_FWD_CASE(2, true, false)
  TG_FWD_CASE(2, false, true)
  TG_FWD_CASE(2, false, false)
  TG_FWD_CASE(1, true, true)
  TG_FWD_CASE(1, true, false)
  TG_FWD_CASE(1, false, true)
  TG_FWD_CASE(1, false, false)
#undef TG_FWD_CASE
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Waves per workgroup and query tiles for a launch over `rows` query positions x `units` (sequence,
// head group) pairs: 8-wave workgroups when that still gives at least two per CU, else 4-wave ones.
void pick_tiling(int hp, int rows, int64_t units, int &nw, int &n_qtiles) {
  const int bm8 = hp == 2 ? bm<8, 2>() : bm<8, 1>();
  const int bm4 = hp == 2 ? bm<4, 2>() : bm<4, 1>();
  const int64_t t8 = (rows + bm8 - 1) / bm8;
  nw = t8 * units >= 2 * (int64_t)device_cus() ? 8 : 4;
  n_qtiles = nw == 8 ? (int)t8 : (rows + bm4 - 1) / bm4;
}

// Key-range split plan.  A grid that leaves at least a quarter of the resident-workgroup slots
// empty from the start (Phase 2 at small K, a few rows over a long cache, single-row decode) is
// bound by its longest tiles while the chip idles: the tiles whose key range exceeds 1/ns of the
// longest are split into ns chunks of consecutive key tiles (ns from the free slots, at least 4
// key tiles per chunk), merged by the combine kernel.  A grid that fills the slots (a 4k prompt)
// is not split: measured, the split's partial traffic and second launch cost more there than the
// causal tail it removes.  Returns ns = 1 when nothing is split.
struct SplitPlan {
  int ns = 1, n_heavy = 0;
  int64_t heavy_units = 0, bytes = 0;
};
constexpr int64_t kPartialBytesPerLane = 8 * 16 + 2 * 8;   // O / l as 64 bf16, then (m, l) per column block
SplitPlan plan_split(int nw, int hp, int n_qtiles, int64_t units, int sq, int sk, bool causal) {
  SplitPlan p;
  const int bmq = nw == 8 ? (hp == 2 ? bm<8, 2>() : bm<8, 1>()) : (hp == 2 ? bm<4, 2>() : bm<4, 1>());
  const int64_t slots = (int64_t)device_cus() * (8 / nw);
  const int64_t nblocks = (int64_t)n_qtiles * units;
  if (nblocks <= 0 || 4 * nblocks > 3 * slots || sk <= 0) return p;
  const int off = sk - sq;
  auto tiles = [&](int qt) -> int {
    int kv_end = sk;
    if (causal) kv_end = std::min<int64_t>(sk, (int64_t)(qt + 1) * bmq + off);
    return kv_end > 0 ? (kv_end + kBN - 1) / kBN : 0;
  };
  const int tmax = tiles(n_qtiles - 1);
  int ns = (int)std::min<int64_t>(32, std::max<int64_t>(2, slots / nblocks));
  // at least 4 key tiles per chunk; 2 for a few query rows (a decode step), whose chunks are short
  // enough that the tile count, not the merge, sets their time (decode at 2.3k keys: -2 %)
  ns = std::min(ns, tmax / (sq <= 16 ? 2 : 4));
  if (ns < 2) return p;
  int n_heavy = 0;
  for (int qt = n_qtiles - 1; qt >= 0 && (int64_t)tiles(qt) * ns > tmax; --qt) ++n_heavy;
  // The split grid (nblocks + heavy_units * (ns - 1) workgroups) must fit the resident slots: past
  // that, extra chunks only queue behind the others.  ns <= slots / nblocks already ensures it
  // unless ns was raised to 2 for a grid of more than half the slots; then only the heaviest tiles
  // that fit are split.  Hence heavy_units * ns <= slots, and the partials take at most
  // CUs x 8 waves x 64 lanes x kPartialBytesPerLane bytes.
  n_heavy = (int)std::min<int64_t>(n_heavy, (slots - nblocks) / ((int64_t)(ns - 1) * units));
  if (n_heavy <= 0) return p;
  p.ns = ns;
  p.n_heavy = n_heavy;
  p.heavy_units = (int64_t)n_heavy * units;
  p.bytes = p.heavy_units * ns * nw * 64 * kPartialBytesPerLane;
  return p;
}

// Apply a plan to the launch arguments (no split if the workspace is missing or too small).
// Returns the grid size.
int64_t apply_split(FwdArgs &a, SplitPlan p, int nw, int64_t units, void *workspace, int64_t workspace_bytes) {
  if (p.ns < 2 || workspace == nullptr || workspace_bytes < p.bytes) p = SplitPlan{};
  a.ns = p.ns;
  a.n_heavy = p.n_heavy;
  a.heavy_blocks = p.heavy_units * p.ns;
  a.ws_o = static_cast<bf16_t *>(workspace);
  a.ws_ml = workspace ? reinterpret_cast<float *>(static_cast<char *>(workspace) + p.heavy_units * p.ns * nw * 64 * 128)
                      : nullptr;
  return a.heavy_blocks + (int64_t)(a.n_qtiles - a.n_heavy) * units;
}

int check_common(const void *q, const void *k, const void *v, const void *out, const float *lse,
                 int32_t num_heads, int32_t num_heads_k, int32_t head_dim) {
  TG_CHECK(head_dim == kD, "this library supports bf16 with head_dim 128 only (got head_dim %d)", head_dim);
  TG_CHECK(q && k && v && out && lse, "null tensor pointer");
  TG_CHECK(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out),
           "q, k, v and out must be 16-byte aligned");
  TG_CHECK(num_heads > 0 && num_heads_k > 0 && num_heads % num_heads_k == 0,
           "Number of heads in key/value must divide number of heads in query (%d, %d)", num_heads,
           num_heads_k);
  return 0;
}

// Buffer descriptors address at most 4 GiB: rows x row stride of bf16 (or fp32 bias) must fit.
bool span_ok(int64_t rows, int64_t row_stride) { return (rows + 1) * row_stride * 2 < (1ll << 32) - 1024; }

bool strides_ok(std::initializer_list<int64_t> s) {
  for (int64_t x : s)
    if (x % 8 != 0) return false;
  return true;
}

}  // namespace
}  // namespace tg

using namespace tg;

namespace tg {
namespace {
// The dense forward behind tg_keybias_fwd and tg_keybias_fwd_noalloc (workspace: the key-range
// split's partials, or NULL for an unsplit launch).
int keybias_fwd_dense(const void *q, const void *k, const void *v, const float *bias_raw, void *out, float *lse,
                      int32_t batch, int32_t seqlen_q, int32_t seqlen_k, int32_t num_heads, int32_t num_heads_k,
                      int32_t head_dim, int64_t q_batch_stride, int64_t q_row_stride, int64_t q_head_stride,
                      int64_t k_batch_stride, int64_t k_row_stride, int64_t k_head_stride, int64_t v_batch_stride,
                      int64_t v_row_stride, int64_t v_head_stride, int64_t o_batch_stride, int64_t o_row_stride,
                      int64_t o_head_stride, int64_t bias_batch_stride, int64_t bias_head_stride,
                      float softmax_scale, int32_t causal, void *workspace, int64_t workspace_bytes,
                      hipStream_t stream) {
  if (int e = check_common(q, k, v, out, lse, num_heads, num_heads_k, head_dim)) return e;
  TG_CHECK(batch >= 0 && seqlen_q >= 0 && seqlen_k >= 0, "negative size");
  TG_CHECK(strides_ok({q_batch_stride, q_row_stride, q_head_stride, k_batch_stride, k_row_stride,
                       k_head_stride, v_batch_stride, v_row_stride, v_head_stride, o_batch_stride,
                       o_row_stride, o_head_stride}),
           "q/k/v/out strides must be multiples of 8 elements");
  TG_CHECK(softmax_scale > 0.f, "softmax_scale must be positive");
  if (batch == 0 || seqlen_q == 0) return 0;
  TG_CHECK(span_ok(seqlen_k, k_row_stride) && span_ok(seqlen_k, v_row_stride) &&
               (bias_raw == nullptr || span_ok(seqlen_k + bias_head_stride, 2)),
           "one (batch, kv head) slice of k/v/bias must span less than 4 GiB");
  FwdArgs a{};
  a.q = static_cast<const bf16_t *>(q);
  a.k = static_cast<const bf16_t *>(k);
  a.v = static_cast<const bf16_t *>(v);
  a.bias = bias_raw;
  a.o = static_cast<bf16_t *>(out);
  a.lse = lse;
  a.q_bs = q_batch_stride; a.q_rs = q_row_stride; a.q_hs = q_head_stride;
  a.k_bs = k_batch_stride; a.k_rs = k_row_stride; a.k_hs = k_head_stride;
  a.v_bs = v_batch_stride; a.v_rs = v_row_stride; a.v_hs = v_head_stride;
  a.o_bs = o_batch_stride; a.o_rs = o_row_stride; a.o_hs = o_head_stride;
  a.bias_bs = bias_batch_stride; a.bias_hs = bias_head_stride;
  a.batch = batch; a.sq = seqlen_q; a.sk = seqlen_k;
  a.h = num_heads; a.hkv = num_heads_k; a.group = num_heads / num_heads_k;
  a.scale_log2 = softmax_scale * kLog2e;
  const int hp = (a.group % 2 == 0) ? 2 : 1;
  int nw = 8;
  const int64_t units = (int64_t)batch * (num_heads / hp);
  pick_tiling(hp, seqlen_q, units, nw, a.n_qtiles);
  TG_CHECK(workspace == nullptr || aligned16(workspace), "workspace must be 16-byte aligned");
  const int64_t nblocks = apply_split(a, plan_split(nw, hp, a.n_qtiles, units, seqlen_q, seqlen_k, causal != 0), nw,
                                      units, workspace, workspace_bytes);
  TG_CHECK(nblocks < (1ll << 31), "grid too large");
  dispatch_fwd<false>(a, nw, hp, causal != 0, bias_raw != nullptr, (int)nblocks, stream);
  TG_HIP_CHECK(hipPeekAtLastError());
  return 0;
}

int64_t fwd_workspace_size(int32_t units_batch, int32_t seqlen_q, int32_t seqlen_k, int32_t num_heads,
                           int32_t num_heads_k, int32_t causal) {
  if (units_batch <= 0 || seqlen_q <= 0 || seqlen_k <= 0 || num_heads <= 0 || num_heads_k <= 0 ||
      num_heads % num_heads_k != 0)
    return 0;
  const int hp = ((num_heads / num_heads_k) % 2 == 0) ? 2 : 1;
  const int64_t units = (int64_t)units_batch * (num_heads / hp);
  int nw = 8, nq = 0;
  pick_tiling(hp, seqlen_q, units, nw, nq);
  return plan_split(nw, hp, nq, units, seqlen_q, seqlen_k, causal != 0).bytes;
}

// Device scratch of tg_keybias_fwd_noalloc: the key-range split's partial results.  plan_split
// keeps the split chunks within the resident-workgroup slots (heavy units x ns <= slots), so a
// split needs at most CUs x 8 waves x 64 lanes x 144 B (18 MiB on a 256-CU MI355X); 24 MiB
// covers devices of up to 341 CUs.  One copy per device, held until the process ends; every call
// on a device shares it.
constexpr int64_t kScratchBytes = 24ll << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void *g_scratch_ptr[64] = {};

// The device address of this device's scratch, looked up once per device with it current.
int scratch_address(void **ptr) {
  int dev = 0;
  TG_HIP_CHECK(hipGetDevice(&dev));
  TG_CHECK(dev >= 0 && dev < 64, "device id %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void *p = nullptr;
    TG_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    TG_CHECK(p != nullptr && aligned16(p), "scratch address lookup failed");
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return 0;
}
}  // namespace
}  // namespace tg

extern "C" int tg_keybias_fwd(const void *q, const void *k, const void *v, const float *bias_raw,
                              void *out, float *lse, int32_t batch, int32_t seqlen_q, int32_t seqlen_k,
                              int32_t num_heads, int32_t num_heads_k, int32_t head_dim,
                              int64_t q_batch_stride, int64_t q_row_stride, int64_t q_head_stride,
                              int64_t k_batch_stride, int64_t k_row_stride, int64_t k_head_stride,
                              int64_t v_batch_stride, int64_t v_row_stride, int64_t v_head_stride,
                              int64_t o_batch_stride, int64_t o_row_stride, int64_t o_head_stride,
                              int64_t bias_batch_stride, int64_t bias_head_stride, float softmax_scale,
                              int32_t causal, void *workspace, int64_t workspace_bytes, hipStream_t stream) {
  clear_error();
  return keybias_fwd_dense(q, k, v, bias_raw, out, lse, batch, seqlen_q, seqlen_k, num_heads, num_heads_k,
                           head_dim, q_batch_stride, q_row_stride, q_head_stride, k_batch_stride, k_row_stride,
                           k_head_stride, v_batch_stride, v_row_stride, v_head_stride, o_batch_stride,
                           o_row_stride, o_head_stride, bias_batch_stride, bias_head_stride, softmax_scale, causal,
                           workspace, workspace_bytes, stream);
}

extern "C" int tg_keybias_fwd_noalloc(const void *q, const void *k, const void *v, const float *bias_raw,
                                      void *out, float *lse, int32_t batch, int32_t seqlen_q, int32_t seqlen_k,
                                      int32_t num_heads, int32_t num_heads_k, int32_t head_dim,
                                      int64_t q_batch_stride, int64_t q_row_stride, int64_t q_head_stride,
                                      int64_t k_batch_stride, int64_t k_row_stride, int64_t k_head_stride,
                                      int64_t v_batch_stride, int64_t v_row_stride, int64_t v_head_stride,
                                      int64_t o_batch_stride, int64_t o_row_stride, int64_t o_head_stride,
                                      int64_t bias_batch_stride, int64_t bias_head_stride, float softmax_scale,
                                      int32_t causal, hipStream_t stream) {
  clear_error();
  const int64_t need = fwd_workspace_size(batch, seqlen_q, seqlen_k, num_heads, num_heads_k, causal);
  TG_CHECK(need <= kScratchBytes,
           "tg_keybias_fwd_noalloc: this launch's key-range split needs %lld bytes of scratch, above the "
           "library's static %lld; call tg_keybias_fwd with a workspace instead",
           (long long)need, (long long)kScratchBytes);
  void *ws = nullptr;
  if (need > 0)
    if (int e = scratch_address(&ws)) return e;
  return keybias_fwd_dense(q, k, v, bias_raw, out, lse, batch, seqlen_q, seqlen_k, num_heads, num_heads_k,
                           head_dim, q_batch_stride, q_row_stride, q_head_stride, k_batch_stride, k_row_stride,
                           k_head_stride, v_batch_stride, v_row_stride, v_head_stride, o_batch_stride,
                           o_row_stride, o_head_stride, bias_batch_stride, bias_head_stride, softmax_scale, causal,
                           ws, need, stream);
}

namespace tg {
namespace {
// The varlen forward behind tg_keybias_varlen_fwd (keys = the query rows) and
// tg_keybias_varlen_kv_fwd (keys at cu_k / used_k).
int keybias_fwd_varlen(const void *q, const void *k, const void *v, const float *bias_raw, void *out, float *lse,
                       const int32_t *cu_seqlens, const int32_t *cu_k, const int32_t *used_k, int32_t num_seqs,
                       int32_t max_seqlen_q, int32_t max_seqlen_k, int32_t total_q, int32_t num_heads,
                       int32_t num_heads_k, int32_t head_dim, int64_t q_row_stride, int64_t q_head_stride,
                       int64_t k_row_stride, int64_t k_head_stride, int64_t v_row_stride, int64_t v_head_stride,
                       int64_t o_row_stride, int64_t o_head_stride, int64_t bias_seq_stride,
                       int64_t bias_head_stride, float softmax_scale, int32_t causal, void *workspace,
                       int64_t workspace_bytes, hipStream_t stream) {
  if (int e = check_common(q, k, v, out, lse, num_heads, num_heads_k, head_dim)) return e;
  TG_CHECK(cu_seqlens != nullptr, "cu_seqlens is null");
  TG_CHECK(num_seqs >= 0 && max_seqlen_q >= 0 && max_seqlen_k >= 0 && total_q >= 0, "negative size");
  TG_CHECK(strides_ok({q_row_stride, q_head_stride, k_row_stride, k_head_stride, v_row_stride, v_head_stride,
                       o_row_stride, o_head_stride}),
           "q/k/v/out strides must be multiples of 8 elements");
  TG_CHECK(softmax_scale > 0.f, "softmax_scale must be positive");
  if (num_seqs == 0 || max_seqlen_q == 0 || total_q == 0) return 0;
  // kernel addresses are 64-bit per sequence; one sequence's k/v/bias rows go through a buffer
  // descriptor (< 4 GiB)
  TG_CHECK(span_ok(max_seqlen_k, k_row_stride) && span_ok(max_seqlen_k, v_row_stride) &&
               (cu_k != nullptr || (span_ok(total_q, k_row_stride) && span_ok(total_q, v_row_stride))) &&
               (bias_raw == nullptr || span_ok(max_seqlen_k + bias_head_stride, 2)),
           "the k/v/bias rows of one sequence must span less than 4 GiB");
  FwdArgs a{};
  a.q = static_cast<const bf16_t *>(q);
  a.k = static_cast<const bf16_t *>(k);
  a.v = static_cast<const bf16_t *>(v);
  a.bias = bias_raw;
  a.o = static_cast<bf16_t *>(out);
  a.lse = lse;
  a.cu_seqlens = cu_seqlens;
  a.cu_k = cu_k;
  a.used_k = used_k;
  a.q_rs = q_row_stride; a.q_hs = q_head_stride;
  a.k_rs = k_row_stride; a.k_hs = k_head_stride;
  a.v_rs = v_row_stride; a.v_hs = v_head_stride;
  a.o_rs = o_row_stride; a.o_hs = o_head_stride;
  a.bias_bs = bias_seq_stride; a.bias_hs = bias_head_stride;
  a.lse_total = total_q;
  a.batch = num_seqs; a.sq = max_seqlen_q; a.sk = max_seqlen_k;
  a.h = num_heads; a.hkv = num_heads_k; a.group = num_heads / num_heads_k;
  a.scale_log2 = softmax_scale * kLog2e;
  const int hp = (a.group % 2 == 0) ? 2 : 1;
  int nw = 8;
  const int64_t units = (int64_t)num_seqs * (num_heads / hp);
  pick_tiling(hp, max_seqlen_q, units, nw, a.n_qtiles);
  TG_CHECK(workspace == nullptr || aligned16(workspace), "workspace must be 16-byte aligned");
  const int64_t nblocks = apply_split(
      a, plan_split(nw, hp, a.n_qtiles, units, max_seqlen_q, max_seqlen_k, causal != 0), nw, units, workspace,
      workspace_bytes);
  TG_CHECK(nblocks < (1ll << 31), "grid too large");
  dispatch_fwd<true>(a, nw, hp, causal != 0, bias_raw != nullptr, (int)nblocks, stream);
  TG_HIP_CHECK(hipPeekAtLastError());
  return 0;
}
}  // namespace
}  // namespace tg

extern "C" int tg_keybias_varlen_fwd(const void *q, const void *k, const void *v, const float *bias_raw,
                                     void *out, float *lse, const int32_t *cu_seqlens, int32_t num_seqs,
                                     int32_t max_seqlen, int32_t total, int32_t num_heads,
                                     int32_t num_heads_k, int32_t head_dim, int64_t q_row_stride,
                                     int64_t q_head_stride, int64_t k_row_stride, int64_t k_head_stride,
                                     int64_t v_row_stride, int64_t v_head_stride, int64_t o_row_stride,
                                     int64_t o_head_stride, int64_t bias_seq_stride,
                                     int64_t bias_head_stride, float softmax_scale, int32_t causal,
                                     void *workspace, int64_t workspace_bytes, hipStream_t stream) {
  clear_error();
  return keybias_fwd_varlen(q, k, v, bias_raw, out, lse, cu_seqlens, nullptr, nullptr, num_seqs, max_seqlen,
                            max_seqlen, total, num_heads, num_heads_k, head_dim, q_row_stride, q_head_stride,
                            k_row_stride, k_head_stride, v_row_stride, v_head_stride, o_row_stride, o_head_stride,
                            bias_seq_stride, bias_head_stride, softmax_scale, causal, workspace, workspace_bytes,
                            stream);
}

extern "C" int tg_keybias_varlen_kv_fwd(const void *q, const void *k, const void *v, const float *bias_raw,
                                        void *out, float *lse, const int32_t *cu_seqlens_q,
                                        const int32_t *cu_seqlens_k, const int32_t *seqused_k, int32_t num_seqs,
                                        int32_t max_seqlen_q, int32_t max_seqlen_k, int32_t total_q,
                                        int32_t num_heads, int32_t num_heads_k, int32_t head_dim,
                                        int64_t q_row_stride, int64_t q_head_stride, int64_t k_row_stride,
                                        int64_t k_head_stride, int64_t v_row_stride, int64_t v_head_stride,
                                        int64_t o_row_stride, int64_t o_head_stride, int64_t bias_seq_stride,
                                        int64_t bias_head_stride, float softmax_scale, int32_t causal,
                                        void *workspace, int64_t workspace_bytes, hipStream_t stream) {
  clear_error();
  TG_CHECK(cu_seqlens_k != nullptr, "cu_seqlens_k is null");
  return keybias_fwd_varlen(q, k, v, bias_raw, out, lse, cu_seqlens_q, cu_seqlens_k, seqused_k, num_seqs,
                            max_seqlen_q, max_seqlen_k, total_q, num_heads, num_heads_k, head_dim, q_row_stride,
                            q_head_stride, k_row_stride, k_head_stride, v_row_stride, v_head_stride, o_row_stride,
                            o_head_stride, bias_seq_stride, bias_head_stride, softmax_scale, causal, workspace,
                            workspace_bytes, stream);
}

extern "C" int64_t tg_keybias_varlen_kv_fwd_workspace_size(int32_t num_seqs, int32_t max_seqlen_q,
                                                            int32_t max_seqlen_k, int32_t num_heads,
                                                            int32_t num_heads_k, int32_t causal) {
  return fwd_workspace_size(num_seqs, max_seqlen_q, max_seqlen_k, num_heads, num_heads_k, causal);
}

extern "C" int64_t tg_keybias_fwd_workspace_size(int32_t batch, int32_t seqlen_q, int32_t seqlen_k,
                                                  int32_t num_heads, int32_t num_heads_k, int32_t causal) {
  return fwd_workspace_size(batch, seqlen_q, seqlen_k, num_heads, num_heads_k, causal);
}

extern "C" int64_t tg_keybias_varlen_fwd_workspace_size(int32_t num_seqs, int32_t max_seqlen, int32_t num_heads,
                                                         int32_t num_heads_k, int32_t causal) {
  return fwd_workspace_size(num_seqs, max_seqlen, max_seqlen, num_heads, num_heads_k, causal);
}
