// Key-bias causal GQA attention, backward, for gfx950 (MI355X).
//
// Math (reference: kernels/fa2bias/keybias.patch:87-129, 219-271; keybias.py:52-82):
//   P = exp(z - lse), D_i = sum_d dO_i * O_i, dS = P * (dO V^T - D),
//   dQ = scale dS K,  dK = scale sum_{h in group} dS^T Q,  dV = sum_{h in group} P^T dO,
//   dbias_raw[b,h,j] = scale * sum_i dS[i,j]   (the gradient with respect to bias_raw).
//
// Three launches, no atomics (every output element is written exactly once, so results are
// deterministic, unlike the reference's atomicAdd dBias, keybias.patch:267):
//   1. preprocess: D = rowsum(dO * O) (returned as softmax_d, like FA2);
//   2. dQ kernel, query-parallel (same 8-wave / 32-column structure as the forward): per 64-key
//      tile recompute S^T = K Q^T and dP^T = V dO^T, form dS^T, accumulate dQ^T += K^T dS^T;
//   3. dK/dV/dBias kernel, key-parallel: each wave owns 16 keys (K^T and V^T resident in
//      registers) of one KV head and loops over every query head of its GQA group and every
//      32-query tile: S = Q K^T, dP = dO V^T, P, dS, dV^T += dO^T P, dK^T += Q^T dS, and the dBias
//      column sums stay in registers (one scalar per lane per head).
// Both kernels run on v_mfma_f32_16x16x32_bf16.  Tiles that are read both row-major (MFMA A
// operand) and transposed (ds_read_b64_tr_b16) use a chunk swizzle chosen so that both access
// patterns are bank-conflict free (dq_kswz() for the dQ kernel's K tile, k16_swz() for the dK/dV
// kernel's Q / dO tiles).
#include <type_traits>

#include "tg_common.h"
#include "../../include/tokengate_hip.h"

namespace tg {
namespace {

constexpr int kD = 128;
constexpr int kRow = kD * 2;          // bytes per K/V/Q/dO row
constexpr float kLog2e = 1.4426950408889634f;

struct BwdArgs {
  const bf16_t *q, *k, *v, *o, *dout;
  const float *lse, *bias;
  float *softmax_d;
  bf16_t *dq, *dk, *dv;
  float *dbias;
  const int32_t *cu_seqlens;
  int64_t q_bs, q_rs, q_hs, k_bs, k_rs, k_hs, v_bs, v_rs, v_hs, o_bs, o_rs, o_hs;
  int64_t do_bs, do_rs, do_hs, dq_bs, dq_rs, dq_hs, dk_bs, dk_rs, dk_hs, dv_bs, dv_rs, dv_hs;
  int64_t bias_bs, bias_hs, dbias_bs, dbias_hs;
  int64_t lse_total;       // varlen: lse / softmax_d are (H, total)
  int batch, sq, sk, h, hkv, group;
  int n_tiles;             // grid decomposition (q tiles for dQ, key tiles for dK/dV; set per launch)
  float scale, scale_log2;
};


// Sequence geometry shared by the kernels.
struct Seq {
  int64_t row0;
  int sq, sk;
};
template <bool VARLEN>
__device__ __forceinline__ Seq seq_of(const BwdArgs &a, int b) {
  Seq s{0, a.sq, a.sk};
  if constexpr (VARLEN) {
    const int s0 = a.cu_seqlens[b], s1 = a.cu_seqlens[b + 1];
    s.row0 = s0;
    s.sq = min(s1 - s0, a.sq);
    s.sk = s.sq;
  }
  return s;
}

// ---- 1. D = rowsum(dO * O): 16 lanes per (row, head) ----------------------------------------
template <bool VARLEN>
__global__ __launch_bounds__(256) void bwd_preprocess_kernel(BwdArgs a, int64_t nrows) {
  const int64_t r = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 4;   // (b, i, h) flattened
  const int sub = threadIdx.x & 15;
  float acc = 0.f;
  int64_t b = 0, i = 0, hh = 0;
  bool valid = r < nrows;
  if (valid) {
    hh = r % a.h;
    const int64_t bi = r / a.h;
    if constexpr (VARLEN) {
      i = bi;   // packed row
    } else {
      b = bi / a.sq;
      i = bi % a.sq;
    }
    const bf16_t *o = a.o + b * a.o_bs + i * a.o_rs + hh * a.o_hs + 8 * sub;
    const bf16_t *d = a.dout + b * a.do_bs + i * a.do_rs + hh * a.do_hs + 8 * sub;
    const u32x4 ov = *reinterpret_cast<const u32x4 *>(o);
    const u32x4 dv = *reinterpret_cast<const u32x4 *>(d);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      acc += bf16_to_f32((bf16_t)(ov[w] & 0xffff)) * bf16_to_f32((bf16_t)(dv[w] & 0xffff));
      acc += bf16_to_f32((bf16_t)(ov[w] >> 16)) * bf16_to_f32((bf16_t)(dv[w] >> 16));
    }
  }
  acc += __shfl_xor(acc, 1);
  acc += __shfl_xor(acc, 2);
  acc += __shfl_xor(acc, 4);
  acc += __shfl_xor(acc, 8);
  if (valid && sub == 0) {
    if constexpr (VARLEN)
      a.softmax_d[hh * a.lse_total + i] = acc;
    else
      a.softmax_d[(b * a.h + hh) * a.sq + i] = acc;
  }
}

// ---- 2. dQ kernel ------------------------------------------------------------------------
constexpr int kQWaves = 8;
constexpr int kQThreads = 64 * kQWaves;
constexpr int kBN = 64;                 // keys per tile
constexpr int kTileBytes = kBN * kRow;  // 16 KiB
template <int HP> constexpr int dq_bm() { return kQWaves * (32 / HP); }

// dQ kernel tile layouts (16x16x32 MFMAs).  LDS row lr of a 64-key tile holds key dq_perm(lr):
// within each 32-key step, S^T block kb' row m carries key 8(m/4) + 4kb' + m%4, so that lane group
// G of a step's S^T / dP^T accumulators holds keys 8G .. 8G+7 — the k range of the B operand
// (dS^T) of dQ^T += K^T dS^T.  K's chunk swizzle dq_kswz (physical chunk = logical chunk ^
// dq_kswz(row), a function of the row's low four bits) makes both reads conflict free whether the
// LDS serves a 16-byte read to 8 lanes per cycle over 32 banks or to 16 lanes over 64 banks (the
// rocprofv3 bank-conflict counter of the earlier swizzle, 2 (row & 7) + bit 3, matched the first
// model): each 8 consecutive rows of a row read get 8 distinct chunks mod 8 (and 16 rows 16
// distinct chunks), and the 4 (or 8) rows of a transposing read get distinct 32-byte blocks mod 4
// (mod 8).
__device__ __forceinline__ int dq_perm(int lr) {
  const int m = lr & 15;
  return 32 * (lr >> 5) + 8 * (m >> 2) + 4 * ((lr >> 4) & 1) + (m & 3);
}
__device__ __forceinline__ uint32_t dq_kswz(int row) {
  return (uint32_t)(((row >> 2) & 1) | ((row & 3) << 1) | ((((row >> 2) ^ (row >> 3)) & 1) << 3));
}

// LDS DMA issued from inline assembly.  The compiler keeps a wave's LDS reads behind its own
// in-flight LDS DMA whenever it cannot tell the two apart, and with a ring slot chosen at run time
// (ks[buf]) it cannot: every read of tile t would wait for the DMA of tile t+1.  Issued this way
// the DMA is invisible to that bookkeeping; completion is waited for explicitly (wait_all_mem at
// the top of the next tile), and the reads of a tile never touch the slot being filled.
struct RawRsrc {
  uint32_t w[4];
};
__device__ __forceinline__ RawRsrc raw_rsrc(const void *base, uint32_t num_bytes) {
  const uint64_t addr = reinterpret_cast<uint64_t>(base);
  return RawRsrc{{(uint32_t)addr, (uint32_t)(addr >> 32), num_bytes, 0x00020000u}};
}
__device__ __forceinline__ uint32_t lds_addr32(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
template <int BYTES>
__device__ __forceinline__ void dma_asm(const RawRsrc &rs, const void *lds_wave_base, uint32_t voff) {
  const u32x4 r = {(uint32_t)__builtin_amdgcn_readfirstlane(rs.w[0]), (uint32_t)__builtin_amdgcn_readfirstlane(rs.w[1]),
                   (uint32_t)__builtin_amdgcn_readfirstlane(rs.w[2]), (uint32_t)__builtin_amdgcn_readfirstlane(rs.w[3])};
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_addr32(lds_wave_base));
  if constexpr (BYTES == 16)
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :: "s"(m0), "v"(voff), "s"(r) : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                 :: "s"(m0), "v"(voff), "s"(r) : "memory", "m0");
}

template <int HP, bool CAUSAL, bool HAS_BIAS, bool VARLEN>
__global__ __launch_bounds__(kQThreads, 1) void bwd_dq_kernel(BwdArgs a) {
  constexpr int QW = 32;   // query positions per wave (all of one head)
  constexpr int BM = dq_bm<HP>();
  // K: rows in dq_perm order, chunk ^ dq_kswz(row) (read row-major and transposed);
  // V: rows in dq_perm order, chunk ^ (row % 16) (read row-major only)
  __shared__ __attribute__((aligned(1024))) char ks[2][kTileBytes];
  __shared__ __attribute__((aligned(1024))) char vs[2][kTileBytes];
  __shared__ __attribute__((aligned(256))) float bs[2][HP][kBN + 4];

  const int tid = threadIdx.x, wave = wave_id(), lane = tid & 63;
  const int c16 = lane & 15, G = lane >> 4;
  const int hgroups = a.group / HP;
  const int per_q = a.hkv * hgroups;
  const int x = blockIdx.x % per_q, rest = blockIdx.x / per_q;
  const int kh = x % a.hkv, hg = x / a.hkv;
  // varlen: sequence-major (resident workgroups share one sequence's K/V in L2 / MALL)
  const int b = VARLEN ? rest / a.n_tiles : rest % a.batch;
  const int qt = a.n_tiles - 1 - (VARLEN ? rest % a.n_tiles : rest / a.batch);
  const Seq sq_ = seq_of<VARLEN>(a, b);
  const int sq = sq_.sq, sk = sq_.sk;
  const int64_t row0 = sq_.row0;
  const int q0 = qt * BM;
  if (q0 >= sq) return;
  const int off = sk - sq;
  const int h0 = kh * a.group + hg * HP;

  const int64_t qb = VARLEN ? row0 * a.q_rs : (int64_t)b * a.q_bs;
  const int64_t dob = VARLEN ? row0 * a.do_rs : (int64_t)b * a.do_bs;
  const bf16_t *kbase = a.k + (VARLEN ? row0 * a.k_rs : (int64_t)b * a.k_bs) + (int64_t)kh * a.k_hs;
  const bf16_t *vbase = a.v + (VARLEN ? row0 * a.v_rs : (int64_t)b * a.v_bs) + (int64_t)kh * a.v_hs;
  const uint32_t kspan = sk > 0 ? (uint32_t)(((int64_t)(sk - 1) * a.k_rs + kD) * 2) : 0u;
  const uint32_t vspan = sk > 0 ? (uint32_t)(((int64_t)(sk - 1) * a.v_rs + kD) * 2) : 0u;
  const RawRsrc krs = raw_rsrc(kbase, kspan), vrs = raw_rsrc(vbase, vspan);
  const brsrc_t krs_b = make_rsrc(kbase, kspan), vrs_b = make_rsrc(vbase, vspan);
  const float *bbase = HAS_BIAS ? a.bias + (int64_t)b * a.bias_bs + (int64_t)h0 * a.bias_hs : nullptr;
  const RawRsrc brs =
      raw_rsrc(bbase, (HAS_BIAS && sk > 0) ? (uint32_t)(((int64_t)(HP - 1) * a.bias_hs + sk) * 4) : 0u);

  // this wave's 32 columns: 32 query positions of one head (HP = 2: waves 0-3 the first head of the
  // pair, 4-7 the second), block cb (0, 1) = positions 16 cb .. 16 cb + 15, lane l holding column
  // l % 16 of each block; one head per wave means one bias row per wave
  const int hw = HP == 2 ? wave / (kQWaves / 2) : 0;
  const int qw0 = q0 + QW * (HP == 2 ? wave % (kQWaves / 2) : wave);
  int qrow[2], hh[2];
  bool qvalid[2];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    qrow[cb] = qw0 + 16 * cb + c16;
    hh[cb] = h0 + hw;
    qvalid[cb] = qrow[cb] < sq;
  }
  const bool wave_has_rows = qw0 < sq;
  const int qw_hi = min(qw0 + QW, sq) - 1;
  // Q and dO fragments (B operands of S^T = K Q^T and dP^T = V dO^T, 32 d per k-step)
  bf16x8 qf[2][4], df[2][4];
  float lse2[2], dsum[2];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
#pragma unroll
    for (int ks4 = 0; ks4 < 4; ++ks4) {
      qf[cb][ks4] = __builtin_bit_cast(bf16x8, gload16(a.q + qb + (int64_t)qrow[cb] * a.q_rs + (int64_t)hh[cb] * a.q_hs +
                                                           32 * ks4 + 8 * G, qvalid[cb]));
      df[cb][ks4] = __builtin_bit_cast(bf16x8, gload16(a.dout + dob + (int64_t)qrow[cb] * a.do_rs +
                                                           (int64_t)hh[cb] * a.do_hs + 32 * ks4 + 8 * G, qvalid[cb]));
    }
    lse2[cb] = INFINITY;
    dsum[cb] = 0.f;
    if (qvalid[cb]) {
      const int64_t li = VARLEN ? (int64_t)hh[cb] * a.lse_total + row0 + qrow[cb]
                                : ((int64_t)b * a.h + hh[cb]) * sq + qrow[cb];
      lse2[cb] = a.lse[li] * kLog2e;
      dsum[cb] = a.softmax_d[li];
    }
  }

  const f32x4 nd4[2] = {f32x4{-dsum[0], -dsum[0], -dsum[0], -dsum[0]}, f32x4{-dsum[1], -dsum[1], -dsum[1], -dsum[1]}};
  int kv_end = sk;
  if constexpr (CAUSAL) kv_end = min(sk, q0 + BM + off);
  const int n_tiles = kv_end > 0 ? (kv_end + kBN - 1) / kBN : 0;

  uint32_t koff[2], voff[2];
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int lr = (wave * 2 + it) * 4 + (lane >> 4);          // LDS row written by this lane
    const int key = dq_perm(lr);
    koff[it] = (uint32_t)(key * a.k_rs * 2 + (((lane & 15) ^ dq_kswz(lr)) << 4));
    voff[it] = (uint32_t)(key * a.v_rs * 2 + (((lane & 15) ^ (lr & 15)) << 4));
  }
  auto issue_tile = [&](int tile, int buf) {
    const uint32_t kb0 = (uint32_t)((int64_t)tile * kBN * a.k_rs * 2);
    const uint32_t vb0 = (uint32_t)((int64_t)tile * kBN * a.v_rs * 2);
    // with the bias: the DMA from inline assembly (see dma_asm); without, the builtin (that variant
    // has fewer registers to spare: the assembly form spills 13 VGPRs against 7, 3 % slower)
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      if constexpr (HAS_BIAS) {
        dma_asm<16>(krs, ks[buf] + (wave * 2 + it) * 1024, kb0 + koff[it]);
        dma_asm<16>(vrs, vs[buf] + (wave * 2 + it) * 1024, vb0 + voff[it]);
      } else {
        dma16(krs_b, ks[buf] + (wave * 2 + it) * 1024, kb0 + koff[it]);
        dma16(vrs_b, vs[buf] + (wave * 2 + it) * 1024, vb0 + voff[it]);
      }
    }
    if constexpr (HAS_BIAS) {
      if (wave < HP)
        dma_asm<4>(brs, &bs[buf][wave][0], (uint32_t)(((int64_t)wave * a.bias_hs + tile * kBN + lane) * 4));
    }
  };

  // K^T fragments (A operand of dQ^T += K^T dS^T: d = 16 dblk + l%16, keys 8G .. 8G+7 of a 32-key
  // step) by transposing reads: lane r of group G addresses the key 8G + r/4 (+4 for the upper
  // four), i.e. LDS row 32 st + 16 hi + 4G + r/4, and the 8 bytes of d = 16 dblk + 4(r%4) .. +3.
  // The swizzle dq_kswz depends only on the row's low four bits, so the lane part of every
  // address is one of eight per-lane values.
  const int trow = 4 * G + (c16 >> 2);
  uint32_t ktr[8];
#pragma unroll
  for (int dblk = 0; dblk < 8; ++dblk)
    ktr[dblk] = (uint32_t)(trow * kRow + ((((uint32_t)(2 * dblk + ((c16 & 3) >> 1))) ^ dq_kswz(trow)) << 4) +
                           8 * (c16 & 1));

  // lane parts of the row-major K and V reads of each 32-d step (rows 16 kb + c16: kb adds 4096
  // bytes; the swizzles depend on the row's low four bits, c16), and of the transposing K reads.
  // With the bias they are passed through an empty asm, so that the compiler keeps one register
  // per lane part and adds the offsets to it (no spills, against 4 VGPRs spilled otherwise; +1.8 %
  // at B4 x 8192).
  uint32_t lpk[4] = {}, lpv[4] = {};
  if constexpr (HAS_BIAS)
#pragma unroll
    for (int ks4 = 0; ks4 < 4; ++ks4) {
      lpk[ks4] = (uint32_t)(c16 * kRow) + ((((uint32_t)(4 * ks4 + G)) ^ dq_kswz(c16)) << 4);
      lpv[ks4] = (uint32_t)(c16 * kRow) + ((uint32_t)((4 * ks4 + G) ^ c16) << 4);
      asm volatile("" : "+v"(lpk[ks4]), "+v"(lpv[ks4]));
    }
  if constexpr (HAS_BIAS)
#pragma unroll
    for (int dblk = 0; dblk < 8; ++dblk) asm volatile("" : "+v"(ktr[dblk]));

  f32x4 dqacc[2][8];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int d = 0; d < 8; ++d) dqacc[cb][d] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (n_tiles > 0) issue_tile(0, 0);
  for (int t = 0; t < n_tiles; ++t) {
    const int buf = t & 1;
    const int n0 = t * kBN;
    wait_all_mem();
    __syncthreads();
    if (t + 1 < n_tiles) issue_tile(t + 1, buf ^ 1);
    if (!wave_has_rows || (CAUSAL && n0 > qw_hi + off)) continue;

    // S^T = K Q^T (+ bias, as the accumulators' start) and dP^T = V dO^T: 2 column blocks x 4 key
    // blocks x 4 d-steps each
    f32x4 sacc[2][4], pacc[2][4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      if constexpr (HAS_BIAS)   // both column blocks are the wave's head: one read serves both
        sacc[0][kb] = *reinterpret_cast<const f32x4 *>(&bs[buf][hw][32 * (kb >> 1) + 8 * G + 4 * (kb & 1)]);
      else
        sacc[0][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
      sacc[1][kb] = sacc[0][kb];
      pacc[0][kb] = nd4[0];   // dP^T - D accumulated from -D (D is per column)
      pacc[1][kb] = nd4[1];
    }
    // keys past the end or in the causal future start from -inf (one uniform branch, before the
    // MFMAs), so that P = exp2(-inf) = +0 below needs no per-element test
    const bool need_mask = (n0 + kBN > sk) || (CAUSAL && n0 + kBN - 1 > qw0 + off);
    if (need_mask) {
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        int lim = sk - 1;
        if constexpr (CAUSAL) lim = min(lim, qrow[cb] + off);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          const int rel = lim - (n0 + 32 * (kb >> 1) + 8 * G + 4 * (kb & 1));
#pragma unroll
          for (int i = 0; i < 4; ++i) sacc[cb][kb][i] = rel - i < 0 ? -__builtin_inff() : sacc[cb][kb][i];
        }
      }
    }
#pragma unroll
    for (int ks4 = 0; ks4 < 4; ++ks4) {
      bf16x8 kf[4], vf[4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        if constexpr (HAS_BIAS) {
          kf[kb] = lds_load16(ks[buf] + 16 * kb * kRow, lpk[ks4]);
          vf[kb] = lds_load16(vs[buf] + 16 * kb * kRow, lpv[ks4]);
        } else {
          const int lr = 16 * kb + c16;
          kf[kb] = lds_load16(ks[buf], lr * kRow + ((((uint32_t)(4 * ks4 + G)) ^ dq_kswz(lr)) << 4));
          vf[kb] = lds_load16(vs[buf], lr * kRow + ((uint32_t)((4 * ks4 + G) ^ c16) << 4));
        }
      }
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          sacc[cb][kb] = mfma16(kf[kb], qf[cb][ks4], sacc[cb][kb]);
          pacc[cb][kb] = mfma16(vf[kb], df[cb][ks4], pacc[cb][kb]);
        }
      }
    }
    // dS = P (dP - D), P = exp2(S scale log2e - lse log2e) (+0 for the masked keys); the
    // scheduling fences keep the three phases apart (hoisting across them raises the register
    // pressure past the file)
    __builtin_amdgcn_sched_barrier(0);
    uint32_t dsk[2][4][2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        float ds[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = fast_exp2(fmaf(sacc[cb][kb][i], a.scale_log2, -lse2[cb]));
          ds[i] = p * pacc[cb][kb][i];
        }
        dsk[cb][kb][0] = pack_bf16x2(ds[0], ds[1]);
        dsk[cb][kb][1] = pack_bf16x2(ds[2], ds[3]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    // dQ^T += K^T dS^T: 2 key steps x 8 d-blocks x 2 column blocks
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      bf16x8 bop[2];
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const u32x4 w = {dsk[cb][2 * st][0], dsk[cb][2 * st][1], dsk[cb][2 * st + 1][0], dsk[cb][2 * st + 1][1]};
        bop[cb] = __builtin_bit_cast(bf16x8, w);
      }
#pragma unroll
      for (int dblk = 0; dblk < 8; ++dblk) {
        const s16x4 lo = lds_read_tr16(ks[buf] + 32 * st * kRow + ktr[dblk]);
        const s16x4 hi = lds_read_tr16(ks[buf] + (32 * st + 16) * kRow + ktr[dblk]);
        const bf16x8 aop = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) dqacc[cb][dblk] = mfma16(aop, bop[cb], dqacc[cb][dblk]);
      }
    }
  }
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    if (!qvalid[cb]) continue;
    bf16_t *row = a.dq + (VARLEN ? row0 * a.dq_rs : (int64_t)b * a.dq_bs) + (int64_t)qrow[cb] * a.dq_rs +
                  (int64_t)hh[cb] * a.dq_hs;
#pragma unroll
    for (int dblk = 0; dblk < 8; ++dblk) {
      const f32x4 &o = dqacc[cb][dblk];
      const u32x2 w = {pack_bf16x2(o[0] * a.scale, o[1] * a.scale), pack_bf16x2(o[2] * a.scale, o[3] * a.scale)};
      *reinterpret_cast<u32x2 *>(row + 16 * dblk + 4 * G) = w;
    }
  }
}

// ---- 3. dK / dV / dBias kernel -----------------------------------------------------------
constexpr int kKBlock = 128;            // keys per workgroup
constexpr int kQT = 32;                 // queries per tile
constexpr int kQSub = 2;                // query tiles per LDS ring slot (per workgroup barrier)
constexpr int kQTileBytes = kQT * kRow; // 8 KiB

// Eight waves; each owns 16 keys of one KV head and loops over every query head of its GQA group
// and every 32-query tile (two tiles per LDS ring slot, so one workgroup barrier per 64 queries),
// on v_mfma_f32_16x16x32_bf16
// (lane l: A row l%16 with k = 8(l/16)+j, B column l%16 with the same k, C rows 4(l/16)+i at
// column l%16).  Per wave: K^T / V^T fragments 2 x 16 VGPRs, dK^T / dV^T accumulators 2 x 32,
// S / dP 2 x 8, so that eight waves (two per SIMD) fit where the 32-key form holds one per SIMD.
// Tile rows are read through the row map pi_rb(m) = 8(m/4) + 4rb + m%4, so that the S^T / dP^T
// accumulators of lane group g hold queries 8g .. 8g+7 — the B operand layout of dV^T += dO^T P
// and dK^T += Q^T dS — and the Q / dO tiles use the swizzle k16_swz (physical chunk = logical
// chunk ^ k16_swz(row)), conflict free for the row reads (rows 8(m/4) + 4rb + m%4: each 8-lane
// group gets 8 distinct chunks mod 8, each 16-lane group 16 distinct chunks) and the transposing
// reads (rows 8g + 0..3 / 4..7: distinct 32-byte blocks mod 4 per 16 lanes, mod 8 per 32 lanes),
// under either LDS model (8 lanes x 16 B over 32 banks per cycle, or 16 lanes over 64 banks).
__device__ __forceinline__ uint32_t k16_swz(int row) {
  return (uint32_t)(((row >> 3) & 1) | ((row & 3) << 1) | ((((row >> 3) ^ (row >> 4)) & 1) << 3));
}
constexpr int kK16Waves = 8;
constexpr int kK16Threads = 64 * kK16Waves;
static_assert(16 * kK16Waves == kKBlock, "eight waves of 16 keys");

template <bool CAUSAL, bool HAS_BIAS, bool VARLEN>
__global__ __launch_bounds__(kK16Threads, 1) void bwd_dkdv16_kernel(BwdArgs a) {
  // each ring slot holds kQSub query tiles of kQT rows: one barrier per kQSub tiles
  __shared__ __attribute__((aligned(1024))) char qs0[kQSub * kQTileBytes], qs1[kQSub * kQTileBytes];
  __shared__ __attribute__((aligned(1024))) char dos0[kQSub * kQTileBytes], dos1[kQSub * kQTileBytes];
  __shared__ __attribute__((aligned(256))) float ls0[kQSub * kQT], ls1[kQSub * kQT];
  __shared__ __attribute__((aligned(256))) float dsh0[kQSub * kQT], dsh1[kQSub * kQT];
  auto qslot = [&](auto b) -> char * { if constexpr (decltype(b)::value == 0) return qs0; else return qs1; };
  auto doslot = [&](auto b) -> char * { if constexpr (decltype(b)::value == 0) return dos0; else return dos1; };
  auto lslot = [&](auto b) -> float * { if constexpr (decltype(b)::value == 0) return ls0; else return ls1; };
  auto dslot = [&](auto b) -> float * { if constexpr (decltype(b)::value == 0) return dsh0; else return dsh1; };

  const int tid = threadIdx.x, wave = wave_id(), lane = tid & 63, l16 = lane & 15, g = lane >> 4;
  const int kh = blockIdx.x % a.hkv;
  const int rest = blockIdx.x / a.hkv;
  const int b = VARLEN ? rest / a.n_tiles : rest % a.batch;
  const int kt = VARLEN ? rest % a.n_tiles : rest / a.batch;
  const Seq sq_ = seq_of<VARLEN>(a, b);
  const int sq = sq_.sq, sk = sq_.sk;
  const int64_t row0 = sq_.row0;
  const int n0 = kt * kKBlock;
  if (n0 >= sk) return;
  const int off = sk - sq;
  const int kw0 = n0 + 16 * wave;
  const int key = kw0 + l16;             // this lane's key (MFMA column)
  const bool kvalid = key < sk;
  const bool wave_has_keys = kw0 < sk;

  const bf16_t *kbase = a.k + (VARLEN ? row0 * a.k_rs : (int64_t)b * a.k_bs) + (int64_t)kh * a.k_hs;
  const bf16_t *vbase = a.v + (VARLEN ? row0 * a.v_rs : (int64_t)b * a.v_bs) + (int64_t)kh * a.v_hs;
  bf16x8 kf[4], vf[4];   // B operands: K^T / V^T rows d = 32ks + 8g .. +7 of this lane's key
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    kf[ks] = __builtin_bit_cast(bf16x8, gload16(kbase + (int64_t)key * a.k_rs + 32 * ks + 8 * g, kvalid));
    vf[ks] = __builtin_bit_cast(bf16x8, gload16(vbase + (int64_t)key * a.v_rs + 32 * ks + 8 * g, kvalid));
  }

  int m_start = 0;
  if constexpr (CAUSAL) m_start = max(0, n0 - off) / kQT * kQT;
  constexpr int kQSlot = kQSub * kQT;   // query rows per ring slot
  const int n_qt = sq > m_start ? (sq - m_start + kQSlot - 1) / kQSlot : 0;

  // LDS DMA: wave w fills rows 4w .. 4w+3 of the Q and dO tiles (one 1 KB load each)
  const int drow = 4 * wave + (lane >> 4);
  const uint32_t dchunk = ((uint32_t)(lane & 15) ^ k16_swz(drow)) << 4;
  const uint32_t qoff = (uint32_t)(drow * a.q_rs * 2) + dchunk;
  const uint32_t dooff = (uint32_t)(drow * a.do_rs * 2) + dchunk;

  // row-read addresses (A operands of S and dP): row pi_rb(l16), logical chunk 4ks + g
  uint32_t ra[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) ra[rb] = (uint32_t)(8 * (l16 >> 2) + 4 * rb + (l16 & 3));
  // transposing-read addresses (A operands of dV^T / dK^T): lane 4k+m of group g supplies row
  // 8g + k (+4 for the second read), bytes 32 dblk + 8m
  const int tk = l16 >> 2, tm = l16 & 3;
  const int trow0 = 8 * g + tk, trow1 = trow0 + 4;

  f32x4 dkacc[8], dvacc[8];
#pragma unroll
  for (int d = 0; d < 8; ++d)
#pragma unroll
    for (int v = 0; v < 4; ++v) { dkacc[d][v] = 0.f; dvacc[d][v] = 0.f; }

  for (int hi = 0; hi < a.group; ++hi) {
    const int hh = kh * a.group + hi;
    const bf16_t *qbase = a.q + (VARLEN ? row0 * a.q_rs : (int64_t)b * a.q_bs) + (int64_t)hh * a.q_hs;
    const bf16_t *dobase = a.dout + (VARLEN ? row0 * a.do_rs : (int64_t)b * a.do_bs) + (int64_t)hh * a.do_hs;
    const brsrc_t qrs = make_rsrc(qbase, sq > 0 ? (uint32_t)(((int64_t)(sq - 1) * a.q_rs + kD) * 2) : 0u);
    const brsrc_t dors = make_rsrc(dobase, sq > 0 ? (uint32_t)(((int64_t)(sq - 1) * a.do_rs + kD) * 2) : 0u);
    const int64_t li0 = VARLEN ? (int64_t)hh * a.lse_total + row0 : ((int64_t)b * a.h + hh) * sq;
    const brsrc_t lrs = make_rsrc(a.lse + li0, (uint32_t)sq * 4);
    const brsrc_t drs = make_rsrc(a.softmax_d + li0, (uint32_t)sq * 4);
    float bk = 0.f;
    if constexpr (HAS_BIAS)
      if (kvalid) bk = a.bias[(int64_t)b * a.bias_bs + (int64_t)hh * a.bias_hs + key];
    const f32x4 bk4 = {bk, bk, bk, bk};   // the S accumulators' start: the key's bias costs no VALU per tile
    float dbacc = 0.f;

    auto issue_tile = [&](int m0, auto buf_c) {
#pragma unroll
      for (int sub = 0; sub < kQSub; ++sub) {
        dma16(qrs, qslot(buf_c) + sub * kQTileBytes + wave * 1024,
              (uint32_t)((int64_t)(m0 + sub * kQT) * a.q_rs * 2) + qoff);
        dma16(dors, doslot(buf_c) + sub * kQTileBytes + wave * 1024,
              (uint32_t)((int64_t)(m0 + sub * kQT) * a.do_rs * 2) + dooff);
      }
      // lse / D of the slot: 64 rows per 4-byte DMA, waves 0 .. kLD-1 and kLD .. 2 kLD-1
      constexpr int kLD = kQSub * kQT / 64;
      static_assert(kLD * 64 == kQSub * kQT && 2 * kLD <= kK16Waves, "lse / D rows in 64-row DMAs");
      if (wave < kLD) dma4(lrs, lslot(buf_c) + 64 * wave, (uint32_t)(m0 + 64 * wave + lane) * 4);
      else if (wave < 2 * kLD) dma4(drs, dslot(buf_c) + 64 * (wave - kLD), (uint32_t)(m0 + 64 * (wave - kLD) + lane) * 4);
    };

    auto tile_step = [&](int t, auto buf_c) {
      constexpr int BUF = decltype(buf_c)::value;
      const int m00 = m_start + t * kQSlot;
      wait_vm<0>();
      // the slot's LSE rows (DMA'd by wave 0, now complete) to log2 units and its D rows (wave 1)
      // negated, once for every wave; the barrier below orders these writes before the other
      // waves' reads
      static_assert(kQSub * kQT == 64, "waves 0 and 1 DMA every LSE / D row of a slot");
      if (wave == 0) {
        float *lw = lslot(buf_c) + lane;
        *lw = *lw * kLog2e;
      } else if (wave == 1) {
        float *dw = dslot(buf_c) + lane;
        *dw = -*dw;
      }
      ring_barrier();
      if (t + 1 < n_qt) issue_tile(m00 + kQSlot, std::integral_constant<int, 1 - BUF>());
#pragma unroll
      for (int sub = 0; sub < kQSub; ++sub) {
      const int m0 = m00 + sub * kQT;
      if (!wave_has_keys || m0 >= sq || (CAUSAL && m0 + kQT - 1 + off < kw0)) continue;
      char *const qsl = qslot(buf_c) + sub * kQTileBytes;
      char *const dosl = doslot(buf_c) + sub * kQTileBytes;
      const float *const lsl = lslot(buf_c) + sub * kQT;
      const float *const dsl = dslot(buf_c) + sub * kQT;

      // S = Q K^T and dP = dO V^T for queries m0 + pi_rb(row), this lane's key
      // dP accumulates from -D (the slot's D rows are stored negated), so dS = P * dP needs no
      // subtraction
      f32x4 sacc[2] = {bk4, bk4};
      f32x4 pacc[2] = {*reinterpret_cast<const f32x4 *>(dsl + 8 * g), *reinterpret_cast<const f32x4 *>(dsl + 8 * g + 4)};
#pragma unroll
      for (int k2 = 0; k2 < 4; k2 += 2) {
        bf16x8 qa[2][2], da[2][2];
#pragma unroll
        for (int e = 0; e < 2; ++e)
#pragma unroll
          for (int rb = 0; rb < 2; ++rb) {
            const uint32_t o16 = ra[rb] * kRow + (((uint32_t)(4 * (k2 + e) + g) ^ k16_swz((int)ra[rb])) << 4);
            qa[e][rb] = lds_load16(qsl, o16);
            da[e][rb] = lds_load16(dosl, o16);
          }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int e = 0; e < 2; ++e)
#pragma unroll
          for (int rb = 0; rb < 2; ++rb) {
            sacc[rb] = mfma16(qa[e][rb], kf[k2 + e], sacc[rb]);
            pacc[rb] = mfma16(da[e][rb], vf[k2 + e], pacc[rb]);
          }
      }
      // accumulator value i of row block rb is query m0 + 8g + 4rb + i
      const bool need_mask = (m0 + kQT > sq) || (kw0 + 16 > sk) || (CAUSAL && kw0 + 15 > m0 + off);
      uint32_t pk[4], dk4[4];
      float p[2][4];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        const f32x4 l4 = *reinterpret_cast<const f32x4 *>(lsl + 8 * g + 4 * rb);
#pragma unroll
        for (int i = 0; i < 4; ++i) p[rb][i] = fast_exp2(fmaf(sacc[rb][i], a.scale_log2, -l4[i]));
      }
      // one uniform branch for the whole tile, and no per-element branches inside it: P -> +0 where
      // the query is past the sequence, the key past the keys, or (causal) the key after the query,
      // selected by the sign of the smallest margin
      if (need_mask) {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int qi = m0 + 8 * g + 4 * rb + i;
            int lim = kvalid ? sq - 1 - qi : -1;
            if constexpr (CAUSAL) lim = min(lim, qi + off - key);
            int sgn;
            asm("v_ashrrev_i32 %0, 31, %1" : "=v"(sgn) : "v"(lim));   // -1 where masked
            const uint32_t pbits = __builtin_bit_cast(uint32_t, p[rb][i]) & ~(uint32_t)sgn;
            p[rb][i] = __builtin_bit_cast(float, pbits);
          }
      }
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        float ds[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          ds[i] = p[rb][i] * pacc[rb][i];
          dbacc += ds[i];
        }
        pk[2 * rb] = pack_bf16x2(p[rb][0], p[rb][1]);
        pk[2 * rb + 1] = pack_bf16x2(p[rb][2], p[rb][3]);
        dk4[2 * rb] = pack_bf16x2(ds[0], ds[1]);
        dk4[2 * rb + 1] = pack_bf16x2(ds[2], ds[3]);
      }
      const bf16x8 pop = __builtin_bit_cast(bf16x8, u32x4{pk[0], pk[1], pk[2], pk[3]});
      const bf16x8 dop = __builtin_bit_cast(bf16x8, u32x4{dk4[0], dk4[1], dk4[2], dk4[3]});
      // dV^T += dO^T P and dK^T += Q^T dS: A rows d = 16 dblk + l16, k = queries 8g .. 8g+7;
      // the transposed reads of four d-blocks are issued ahead of their eight MFMAs
#pragma unroll
      for (int d4 = 0; d4 < 8; d4 += 4) {
        bf16x8 dot_[4], qt_[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int dblk = d4 + e;
          const int c = 2 * dblk + (tm >> 1);
          const uint32_t hb = (uint32_t)((tm & 1) * 8);
          const uint32_t o0 = trow0 * kRow + (((uint32_t)c ^ k16_swz(trow0)) << 4) + hb;
          const uint32_t o1 = trow1 * kRow + (((uint32_t)c ^ k16_swz(trow1)) << 4) + hb;
          dot_[e] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lds_read_tr16(dosl + o0),
                                                                       lds_read_tr16(dosl + o1),
                                                                       0, 1, 2, 3, 4, 5, 6, 7));
          qt_[e] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lds_read_tr16(qsl + o0),
                                                                      lds_read_tr16(qsl + o1),
                                                                      0, 1, 2, 3, 4, 5, 6, 7));
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          dvacc[d4 + e] = mfma16(dot_[e], pop, dvacc[d4 + e]);
          dkacc[d4 + e] = mfma16(qt_[e], dop, dkacc[d4 + e]);
        }
      }
      }   // sub-tiles
    };
    ring_barrier();   // previous head's last tile fully consumed before its slots are reused
    if (n_qt > 0) issue_tile(m_start, std::integral_constant<int, 0>());
    {
      int t = 0;
      for (; t + 1 < n_qt; t += 2) {
        tile_step(t, std::integral_constant<int, 0>());
        tile_step(t + 1, std::integral_constant<int, 1>());
      }
      if (t < n_qt) tile_step(t, std::integral_constant<int, 0>());
    }
    if constexpr (HAS_BIAS) {
      float tot = dbacc + __shfl_xor(dbacc, 16);
      tot += __shfl_xor(tot, 32);
      if (g == 0 && kvalid)
        a.dbias[(int64_t)b * a.dbias_bs + (int64_t)hh * a.dbias_hs + key] = tot * a.scale;
    }
  }
  if (kvalid) {
    bf16_t *krow = a.dk + (VARLEN ? row0 * a.dk_rs : (int64_t)b * a.dk_bs) + (int64_t)key * a.dk_rs + (int64_t)kh * a.dk_hs;
    bf16_t *vrow = a.dv + (VARLEN ? row0 * a.dv_rs : (int64_t)b * a.dv_bs) + (int64_t)key * a.dv_rs + (int64_t)kh * a.dv_hs;
#pragma unroll
    for (int dblk = 0; dblk < 8; ++dblk) {
      const int d = 16 * dblk + 4 * g;   // accumulator value i is d + i
      const u32x2 wk = {pack_bf16x2(dkacc[dblk][0] * a.scale, dkacc[dblk][1] * a.scale),
                        pack_bf16x2(dkacc[dblk][2] * a.scale, dkacc[dblk][3] * a.scale)};
      const u32x2 wv = {pack_bf16x2(dvacc[dblk][0], dvacc[dblk][1]), pack_bf16x2(dvacc[dblk][2], dvacc[dblk][3])};
      *reinterpret_cast<u32x2 *>(krow + d) = wk;
      *reinterpret_cast<u32x2 *>(vrow + d) = wv;
    }
  }
}

// ---- host dispatch ---------------------------------------------------------------------------
template <bool VARLEN>
void launch_bwd(const BwdArgs &a0, bool causal, bool has_bias, int64_t nrows, hipStream_t st) {
  BwdArgs a = a0;
  hipLaunchKernelGGL(bwd_preprocess_kernel<VARLEN>, dim3((unsigned)((nrows * 16 + 255) / 256)), dim3(256), 0, st,
                     a, nrows);
  const int hp = (a.group % 2 == 0) ? 2 : 1;
  const int bmq = hp == 2 ? dq_bm<2>() : dq_bm<1>();
  a.n_tiles = (a.sq + bmq - 1) / bmq;
  const unsigned nq = (unsigned)((int64_t)a.n_tiles * a.batch * (a.h / hp));
#define TG_DQ(HPV, C, B)                                                                               \
  if (hp == HPV && causal == C && has_bias == B)                                                       \
    hipLaunchKernelGGL((bwd_dq_kernel<HPV, C, B, VARLEN>), dim3(nq), dim3(kQThreads), 0, st, a);
  TG_DQ(2, true, true) TG_DQ(2, true, false) TG_DQ(2, false, true) TG_DQ(2, false, false)
  TG_DQ(1, true, true) TG_DQ(1, true, false) TG_DQ(1, false, true) TG_DQ(1, false, false)
#undef TG_DQ
  const int nkt = (a.sk + kKBlock - 1) / kKBlock;
  a.n_tiles = nkt;
  const unsigned nk = (unsigned)((int64_t)nkt * a.batch * a.hkv);
#define TG_DKV(C, B)                                                                                   \
  if (causal == C && has_bias == B)                                                                    \
    hipLaunchKernelGGL((bwd_dkdv16_kernel<C, B, VARLEN>), dim3(nk), dim3(kK16Threads), 0, st, a);
  TG_DKV(true, true) TG_DKV(true, false) TG_DKV(false, true) TG_DKV(false, false)
#undef TG_DKV
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool strides_ok(std::initializer_list<int64_t> s) {
  for (int64_t x : s)
    if (x % 8 != 0) return false;
  return true;
}
bool span_ok(int64_t rows, int64_t row_stride) { return (rows + 1) * row_stride * 2 < (1ll << 32) - 1024; }

int check_bwd(const void *dout, const void *q, const void *k, const void *v, const void *out, const float *lse,
              const void *dq, const void *dk, const void *dv, const float *softmax_d, int32_t num_heads,
              int32_t num_heads_k, int32_t head_dim, float softmax_scale) {
  TG_CHECK(head_dim == kD, "this library supports bf16 with head_dim 128 only (got head_dim %d)", head_dim);
  TG_CHECK(dout && q && k && v && out && lse && dq && dk && dv && softmax_d, "null tensor pointer");
  TG_CHECK(aligned16(dout) && aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out) && aligned16(dq) &&
               aligned16(dk) && aligned16(dv),
           "tensors must be 16-byte aligned");
  TG_CHECK(num_heads > 0 && num_heads_k > 0 && num_heads % num_heads_k == 0,
           "Number of heads in key/value must divide number of heads in query (%d, %d)", num_heads, num_heads_k);
  TG_CHECK(softmax_scale > 0.f, "softmax_scale must be positive");
  return 0;
}

}  // namespace
}  // namespace tg

using namespace tg;

extern "C" int tg_keybias_bwd(const void *dout, const void *q, const void *k, const void *v, const void *out,
                              const float *lse, const float *bias_raw, void *dq, void *dk, void *dv, float *dbias,
                              float *softmax_d, int32_t batch, int32_t seqlen_q, int32_t seqlen_k,
                              int32_t num_heads, int32_t num_heads_k, int32_t head_dim,
                              const int64_t *strides, float softmax_scale, int32_t causal, hipStream_t stream) {
  clear_error();
  if (int e = check_bwd(dout, q, k, v, out, lse, dq, dk, dv, softmax_d, num_heads, num_heads_k, head_dim,
                        softmax_scale))
    return e;
  TG_CHECK(strides != nullptr, "null strides");
  TG_CHECK(batch >= 0 && seqlen_q >= 0 && seqlen_k >= 0, "negative size");
  TG_CHECK(bias_raw == nullptr || dbias != nullptr, "dbias is required with a bias");
  BwdArgs a{};
  const int64_t *s = strides;
  a.q_bs = s[0]; a.q_rs = s[1]; a.q_hs = s[2];
  a.k_bs = s[3]; a.k_rs = s[4]; a.k_hs = s[5];
  a.v_bs = s[6]; a.v_rs = s[7]; a.v_hs = s[8];
  a.o_bs = s[9]; a.o_rs = s[10]; a.o_hs = s[11];
  a.do_bs = s[12]; a.do_rs = s[13]; a.do_hs = s[14];
  a.dq_bs = s[15]; a.dq_rs = s[16]; a.dq_hs = s[17];
  a.dk_bs = s[18]; a.dk_rs = s[19]; a.dk_hs = s[20];
  a.dv_bs = s[21]; a.dv_rs = s[22]; a.dv_hs = s[23];
  a.bias_bs = s[24]; a.bias_hs = s[25]; a.dbias_bs = s[26]; a.dbias_hs = s[27];
  TG_CHECK(strides_ok({a.q_bs, a.q_rs, a.q_hs, a.k_bs, a.k_rs, a.k_hs, a.v_bs, a.v_rs, a.v_hs, a.o_bs, a.o_rs,
                       a.o_hs, a.do_bs, a.do_rs, a.do_hs, a.dq_bs, a.dq_rs, a.dq_hs, a.dk_bs, a.dk_rs, a.dk_hs,
                       a.dv_bs, a.dv_rs, a.dv_hs}),
           "tensor strides must be multiples of 8 elements");
  if (batch == 0 || seqlen_q == 0 || seqlen_k == 0) return 0;
  TG_CHECK(span_ok(seqlen_k, a.k_rs) && span_ok(seqlen_k, a.v_rs) && span_ok(seqlen_q, a.q_rs) &&
               span_ok(seqlen_q, a.do_rs),
           "one (batch, head) slice must span less than 4 GiB");
  a.dout = static_cast<const bf16_t *>(dout);
  a.q = static_cast<const bf16_t *>(q);
  a.k = static_cast<const bf16_t *>(k);
  a.v = static_cast<const bf16_t *>(v);
  a.o = static_cast<const bf16_t *>(out);
  a.lse = lse;
  a.bias = bias_raw;
  a.dq = static_cast<bf16_t *>(dq);
  a.dk = static_cast<bf16_t *>(dk);
  a.dv = static_cast<bf16_t *>(dv);
  a.dbias = dbias;
  a.softmax_d = softmax_d;
  a.batch = batch; a.sq = seqlen_q; a.sk = seqlen_k;
  a.h = num_heads; a.hkv = num_heads_k; a.group = num_heads / num_heads_k;
  a.scale = softmax_scale;
  a.scale_log2 = softmax_scale * kLog2e;
  launch_bwd<false>(a, causal != 0, bias_raw != nullptr, (int64_t)batch * seqlen_q * num_heads, stream);
  TG_HIP_CHECK(hipPeekAtLastError());
  return 0;
}

extern "C" int tg_keybias_varlen_bwd(const void *dout, const void *q, const void *k, const void *v,
                                     const void *out, const float *lse, const float *bias_raw, void *dq, void *dk,
                                     void *dv, float *dbias, float *softmax_d, const int32_t *cu_seqlens,
                                     int32_t num_seqs, int32_t max_seqlen, int32_t total, int32_t num_heads,
                                     int32_t num_heads_k, int32_t head_dim, const int64_t *strides,
                                     float softmax_scale, int32_t causal, hipStream_t stream) {
  clear_error();
  if (int e = check_bwd(dout, q, k, v, out, lse, dq, dk, dv, softmax_d, num_heads, num_heads_k, head_dim,
                        softmax_scale))
    return e;
  TG_CHECK(strides != nullptr && cu_seqlens != nullptr, "null strides or cu_seqlens");
  TG_CHECK(num_seqs >= 0 && max_seqlen >= 0 && total >= 0, "negative size");
  TG_CHECK(bias_raw == nullptr || dbias != nullptr, "dbias is required with a bias");
  BwdArgs a{};
  const int64_t *s = strides;   // (row, head) pairs; batch strides unused
  a.q_rs = s[0]; a.q_hs = s[1]; a.k_rs = s[2]; a.k_hs = s[3]; a.v_rs = s[4]; a.v_hs = s[5];
  a.o_rs = s[6]; a.o_hs = s[7]; a.do_rs = s[8]; a.do_hs = s[9]; a.dq_rs = s[10]; a.dq_hs = s[11];
  a.dk_rs = s[12]; a.dk_hs = s[13]; a.dv_rs = s[14]; a.dv_hs = s[15];
  a.bias_bs = s[16]; a.bias_hs = s[17]; a.dbias_bs = s[18]; a.dbias_hs = s[19];
  TG_CHECK(strides_ok({a.q_rs, a.q_hs, a.k_rs, a.k_hs, a.v_rs, a.v_hs, a.o_rs, a.o_hs, a.do_rs, a.do_hs, a.dq_rs,
                       a.dq_hs, a.dk_rs, a.dk_hs, a.dv_rs, a.dv_hs}),
           "tensor strides must be multiples of 8 elements");
  if (num_seqs == 0 || max_seqlen == 0 || total == 0) return 0;
  TG_CHECK(span_ok(total, a.k_rs) && span_ok(total, a.v_rs) && span_ok(total, a.q_rs) && span_ok(total, a.do_rs),
           "the packed tensors must span less than 4 GiB");
  a.dout = static_cast<const bf16_t *>(dout);
  a.q = static_cast<const bf16_t *>(q);
  a.k = static_cast<const bf16_t *>(k);
  a.v = static_cast<const bf16_t *>(v);
  a.o = static_cast<const bf16_t *>(out);
  a.lse = lse;
  a.bias = bias_raw;
  a.dq = static_cast<bf16_t *>(dq);
  a.dk = static_cast<bf16_t *>(dk);
  a.dv = static_cast<bf16_t *>(dv);
  a.dbias = dbias;
  a.softmax_d = softmax_d;
  a.cu_seqlens = cu_seqlens;
  a.lse_total = total;
  a.batch = num_seqs; a.sq = max_seqlen; a.sk = max_seqlen;
  a.h = num_heads; a.hkv = num_heads_k; a.group = num_heads / num_heads_k;
  a.scale = softmax_scale;
  a.scale_log2 = softmax_scale * kLog2e;
  launch_bwd<true>(a, causal != 0, bias_raw != nullptr, (int64_t)total * num_heads, stream);
  TG_HIP_CHECK(hipPeekAtLastError());
  return 0;
}
