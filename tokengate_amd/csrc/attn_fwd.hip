// Key-bias causal GQA attention, forward, for gfx950 (MI355X).
//
// Math (reference: kernels/fa2bias/keybias.patch:279-332, 394-464 and keybias.py:40-49,85-87):
//   z[i,j]  = scale * (q_i . k_j + bias_raw[b,h,j]),   masked to -inf for j > i + Sk - Sq (causal)
//   lse[i]  = ln sum_j exp(z[i,j]);   out_i = sum_j exp(z[i,j] - lse[i]) v_j
// with the query head h reading kv head h / (H / Hkv).
//
// Work decomposition (one workgroup = 4 waves = 256 threads):
//   * a workgroup owns 128 consecutive query positions of one KV head and HP query heads of its
//     GQA group (HP = 2 when the group size is even): every K/V fragment a wave reads from LDS
//     feeds HP matrix-core products;
//   * each wave owns 32 query positions x HP heads; the KV sequence is streamed in 64-key tiles,
//     double-buffered in LDS (K as rows, V transposed), one barrier per tile;
//   * scores are computed transposed, S^T = K Q^T, on v_mfma_f32_32x32x16_bf16: the accumulator
//     then holds one query per lane (column l%32) and 16 keys per lane, so the online-softmax max
//     and sum are in-lane plus one permlane32 swap;
//   * K rows are stored in LDS in a permuted order (sigma) chosen so that lane group g of the
//     S^T accumulator holds 16 CONSECUTIVE keys; the accumulator, rounded to bf16, is then directly
//     the B operand of O^T = V^T P^T, whose A operand is 8 consecutive keys of V^T (16-byte LDS
//     read);
//   * O^T accumulates per lane for one query, so the per-query rescale is a scalar per lane.
// Workgroups are issued heaviest-first (largest query tile first) with the KV head varying
// fastest, so that consecutive workgroups, which land on different XCDs, keep one KV head per
// XCD when Hkv is a multiple of 8.
#include "tg_common.h"
#include "../../include/tokengate_hip.h"

namespace tg {
namespace {

constexpr int kD = 128;        // head dim
constexpr int kBN = 64;        // keys per tile
constexpr int kWQ = 32;        // query positions per wave
constexpr int kWaves = 4;
constexpr int kBM = kWQ * kWaves;   // query positions per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

constexpr int kKRowBytes = kD * 2;      // one K row in LDS (256 B, 16 chunks of 16 B)
constexpr int kVRowBytes = kBN * 2;     // one V^T row (one d) in LDS (128 B, 8 chunks)
constexpr int kKTileBytes = kBN * kKRowBytes;
constexpr int kVTileBytes = kD * kVRowBytes;

struct FwdArgs {
  const bf16_t *q, *k, *v;
  const float *bias;
  bf16_t *o;
  float *lse;
  const int32_t *cu_seqlens;   // varlen only
  int64_t q_bs, q_rs, q_hs, k_bs, k_rs, k_hs, v_bs, v_rs, v_hs, o_bs, o_rs, o_hs;
  int64_t bias_bs, bias_hs;
  int64_t lse_total;           // varlen: total rows (lse is (H, total)); dense: unused
  int batch;                   // dense: B; varlen: number of sequences
  int sq, sk;                  // dense lengths (varlen: per sequence, read from cu_seqlens)
  int h, hkv, group;
  int n_qtiles;
  float scale_log2;            // softmax_scale * log2(e)
};

// Key j (0..31) of a 32-key block is stored at LDS row sigma_inv(j) so that MFMA row
// m = 8a + 4g + b (a, b in 0..3) carries key 16g + 4a + b: lane group g of the S^T accumulator
// then holds keys 16g .. 16g+15 of the block, in register order.
__device__ __forceinline__ int sigma_inv(int j) {
  return ((j & 15) >> 2) * 8 + (j >> 4) * 4 + (j & 3);
}
// XOR swizzle of the 16-byte chunks of a V^T row: conflict-free reads of 8 consecutive rows and
// 4-cycle transposed writes.
__device__ __forceinline__ uint32_t v_swz(int d) { return (uint32_t)((d + (d >> 3)) & 7); }

template <int HP, bool CAUSAL, bool HAS_BIAS, bool VARLEN>
__global__ __launch_bounds__(kThreads) void keybias_fwd_kernel(FwdArgs a) {
  __shared__ __attribute__((aligned(16))) char ks[2][kKTileBytes];
  __shared__ __attribute__((aligned(16))) char vs[2][kVTileBytes];
  __shared__ __attribute__((aligned(16))) float bs[2][HP][kBN];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int lq = lane & 31;
  const int g = lane >> 5;

  // ---- which (query tile, sequence, kv head, head pair) this workgroup owns ----
  const int hgroups = a.group / HP;
  const int per_q = a.hkv * hgroups;
  const int bid = blockIdx.x;
  const int x = bid % per_q;
  const int rest = bid / per_q;
  const int kh = x % a.hkv;
  const int hg = x / a.hkv;
  const int b = rest % a.batch;
  const int qt = a.n_qtiles - 1 - rest / a.batch;

  int sq = a.sq, sk = a.sk;
  int64_t row0 = 0;
  if constexpr (VARLEN) {
    const int s0 = a.cu_seqlens[b], s1 = a.cu_seqlens[b + 1];
    row0 = s0;
    sq = min(s1 - s0, a.sq);   // rows past max_seqlen are outside the bias row: not computed
    sk = sq;
  }
  const int q0 = qt * kBM;
  if (q0 >= sq) return;   // workgroup-uniform: past the end of this sequence
  const int off = sk - sq;
  const int h0 = kh * a.group + hg * HP;

  const bf16_t *qbase = a.q + (VARLEN ? row0 * a.q_rs : (int64_t)b * a.q_bs) + (int64_t)h0 * a.q_hs;
  const bf16_t *kbase = a.k + (VARLEN ? row0 * a.k_rs : (int64_t)b * a.k_bs) + (int64_t)kh * a.k_hs;
  const bf16_t *vbase = a.v + (VARLEN ? row0 * a.v_rs : (int64_t)b * a.v_bs) + (int64_t)kh * a.v_hs;
  bf16_t *obase = a.o + (VARLEN ? row0 * a.o_rs : (int64_t)b * a.o_bs) + (int64_t)h0 * a.o_hs;
  const float *bbase = nullptr;
  if constexpr (HAS_BIAS) bbase = a.bias + (int64_t)b * a.bias_bs + (int64_t)h0 * a.bias_hs;

  // ---- this wave's queries and its Q fragments (B operand of S^T = K Q^T) ----
  const int qw0 = q0 + wave * kWQ;
  const int qrow = qw0 + lq;
  const bool qvalid = qrow < sq;
  const bool wave_has_rows = qw0 < sq;
  const int qw_hi = min(qw0 + kWQ, sq) - 1;
  bf16x8 qf[HP][8];
#pragma unroll
  for (int h = 0; h < HP; ++h)
#pragma unroll
    for (int s = 0; s < 8; ++s)
      qf[h][s] = __builtin_bit_cast(
          bf16x8, gload16(qbase + (int64_t)qrow * a.q_rs + (int64_t)h * a.q_hs + 16 * s + 8 * g, qvalid));

  int kv_end = sk;
  if constexpr (CAUSAL) kv_end = min(sk, q0 + kBM + off);
  const int n_tiles = kv_end > 0 ? (kv_end + kBN - 1) / kBN : 0;

  // ---- global -> register -> LDS staging of one KV tile ----
  u32x4 kreg[4], vreg[4];
  float breg[HP];
  const int ld_c = tid & 15;     // 16-byte chunk along d
  const int ld_r = tid >> 4;     // 0..15
  auto gload_tile = [&](int n0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = n0 + ld_r + 16 * i;
      kreg[i] = gload16(kbase + (int64_t)key * a.k_rs + 8 * ld_c, key < sk);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = n0 + 4 * ld_r + i;
      vreg[i] = gload16(vbase + (int64_t)key * a.v_rs + 8 * ld_c, key < sk);
    }
    if constexpr (HAS_BIAS) {
      if (tid < kBN) {
        const int key = n0 + tid;
#pragma unroll
        for (int h = 0; h < HP; ++h)
          breg[h] = key < sk ? bbase[(int64_t)h * a.bias_hs + key] * a.scale_log2 : 0.f;
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = ld_r + 16 * i;
      const int lr = (r & 32) + sigma_inv(r & 31);
      lds_store16(ks[buf], lr * kKRowBytes + ((ld_c ^ (lr & 15)) << 4), kreg[i]);
    }
    // V: thread holds keys 4*ld_r .. +3 at d = 8*ld_c .. +7; write V^T rows d, 4 keys (8 B) each.
    const int kq = ld_r;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t w0 = vreg[0][p], w1 = vreg[1][p], w2 = vreg[2][p], w3 = vreg[3][p];
      const u32x2 lo = {(w0 & 0xffffu) | (w1 << 16), (w2 & 0xffffu) | (w3 << 16)};
      const u32x2 hi = {(w0 >> 16) | (w1 & 0xffff0000u), (w2 >> 16) | (w3 & 0xffff0000u)};
      const int d0 = 8 * ld_c + 2 * p;
      const int d1 = d0 + 1;
      lds_store8(vs[buf], d0 * kVRowBytes + (((uint32_t)(kq >> 1) ^ v_swz(d0)) << 4) + (kq & 1) * 8, lo);
      lds_store8(vs[buf], d1 * kVRowBytes + (((uint32_t)(kq >> 1) ^ v_swz(d1)) << 4) + (kq & 1) * 8, hi);
    }
    if constexpr (HAS_BIAS) {
      if (tid < kBN) {
#pragma unroll
        for (int h = 0; h < HP; ++h) bs[buf][h][tid] = breg[h];
      }
    }
  };

  f32x16 oacc[HP][4];
  float mrun[HP], lrun[HP];
#pragma unroll
  for (int h = 0; h < HP; ++h) {
    mrun[h] = -INFINITY;
    lrun[h] = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int v = 0; v < 16; ++v) oacc[h][d][v] = 0.f;
  }

  if (n_tiles > 0) {
    gload_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int t = 0; t < n_tiles; ++t) {
    const int buf = t & 1;
    const int n0 = t * kBN;
    if (t + 1 < n_tiles) gload_tile(n0 + kBN);

    const bool active = wave_has_rows && !(CAUSAL && n0 > qw_hi + off);
    if (active) {
      const bool need_mask = (n0 + kBN > sk) || (CAUSAL && n0 + kBN - 1 > qw0 + off);
      // ---- S^T = K Q^T ----
      f32x16 sacc[HP][2];
#pragma unroll
      for (int h = 0; h < HP; ++h)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int v = 0; v < 16; ++v) sacc[h][kb][v] = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const int lr = 32 * kb + lq;
          const bf16x8 kf = lds_load16(ks[buf], lr * kKRowBytes + ((uint32_t)((2 * s + g) ^ (lq & 15)) << 4));
#pragma unroll
          for (int h = 0; h < HP; ++h) sacc[h][kb] = mfma32(kf, qf[h][s], sacc[h][kb]);
        }
      }
      // ---- online softmax (one query per lane; 32 keys per lane per head) ----
      uint32_t pk[HP][2][8];
#pragma unroll
      for (int h = 0; h < HP; ++h) {
        float tv[2][16];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          if constexpr (HAS_BIAS) {
            const f32x4 *bp = reinterpret_cast<const f32x4 *>(&bs[buf][h][32 * kb + 16 * g]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const f32x4 bb = bp[i];
#pragma unroll
              for (int e = 0; e < 4; ++e) tv[kb][4 * i + e] = fmaf(sacc[h][kb][4 * i + e], a.scale_log2, bb[e]);
            }
          } else {
#pragma unroll
            for (int v = 0; v < 16; ++v) tv[kb][v] = sacc[h][kb][v] * a.scale_log2;
          }
          if (need_mask) {
            const int kbase_idx = n0 + 32 * kb + 16 * g;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const int key = kbase_idx + v;
              bool masked = key >= sk;
              if constexpr (CAUSAL) masked = masked || (key > qrow + off);
              tv[kb][v] = masked ? -INFINITY : tv[kb][v];
            }
          }
        }
        float mx = tv[0][0];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int v = 0; v < 16; ++v) mx = fmaxf(mx, tv[kb][v]);
        mx = pair_max(mx);
        const float m_new = fmaxf(mrun[h], mx);
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = fast_exp2(mrun[h] - m_use);
        mrun[h] = m_new;
        lrun[h] *= alpha;
#pragma unroll
        for (int d = 0; d < 4; ++d) oacc[h][d] *= alpha;
        float psum = 0.f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
          for (int v = 0; v < 16; v += 2) {
            const float p0 = fast_exp2(tv[kb][v] - m_use);
            const float p1 = fast_exp2(tv[kb][v + 1] - m_use);
            psum += p0 + p1;
            pk[h][kb][v >> 1] = pack_bf16x2(p0, p1);
          }
        }
        lrun[h] += psum;
      }
      // ---- O^T += V^T P^T ----
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          bf16x8 pb[HP];
#pragma unroll
          for (int h = 0; h < HP; ++h) {
            const u32x4 w = {pk[h][kb][4 * s], pk[h][kb][4 * s + 1], pk[h][kb][4 * s + 2], pk[h][kb][4 * s + 3]};
            pb[h] = __builtin_bit_cast(bf16x8, w);
          }
          const uint32_t kc = 4 * kb + 2 * g + s;
#pragma unroll
          for (int dblk = 0; dblk < 4; ++dblk) {
            const int d = 32 * dblk + lq;
            const bf16x8 vf = lds_load16(vs[buf], d * kVRowBytes + ((kc ^ v_swz(d)) << 4));
#pragma unroll
            for (int h = 0; h < HP; ++h) oacc[h][dblk] = mfma32(vf, pb[h], oacc[h][dblk]);
          }
        }
      }
    }

    if (t + 1 < n_tiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: normalise, write O (bf16) and LSE (natural log) ----
#pragma unroll
  for (int h = 0; h < HP; ++h) {
    const float l = pair_sum(lrun[h]);
    const float inv = l > 0.f ? 1.f / l : 0.f;
    if (qvalid) {
      bf16_t *orow = obase + (int64_t)qrow * a.o_rs + (int64_t)h * a.o_hs;
#pragma unroll
      for (int dblk = 0; dblk < 4; ++dblk) {
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4) {
          const int d = 32 * dblk + 8 * a4 + 4 * g;
          const u32x2 w = {pack_bf16x2(oacc[h][dblk][4 * a4] * inv, oacc[h][dblk][4 * a4 + 1] * inv),
                           pack_bf16x2(oacc[h][dblk][4 * a4 + 2] * inv, oacc[h][dblk][4 * a4 + 3] * inv)};
          *reinterpret_cast<u32x2 *>(orow + d) = w;
        }
      }
      if (g == 0) {
        const float lse = l > 0.f ? (mrun[h] + __log2f(l)) * kLn2 : INFINITY;
        const int hh = h0 + h;
        if constexpr (VARLEN)
          a.lse[(int64_t)hh * a.lse_total + row0 + qrow] = lse;
        else
          a.lse[((int64_t)b * a.h + hh) * sq + qrow] = lse;
      }
    }
  }
}

template <int HP, bool CAUSAL, bool HAS_BIAS, bool VARLEN>
void launch_fwd(const FwdArgs &a, int nblocks, hipStream_t stream) {
  hipLaunchKernelGGL((keybias_fwd_kernel<HP, CAUSAL, HAS_BIAS, VARLEN>), dim3(nblocks), dim3(kThreads), 0,
                     stream, a);
}

template <bool VARLEN>
void dispatch_fwd(const FwdArgs &a, int hp, bool causal, bool has_bias, int nblocks, hipStream_t s) {
#define TG_FWD_CASE(HPV, C, B)                                              \
  if (hp == HPV && causal == C && has_bias == B) {                          \
    launch_fwd<HPV, C, B, VARLEN>(a, nblocks, s);                           \
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

int check_common(const void *q, const void *k, const void *v, const void *out, const float *lse,
                 int32_t num_heads, int32_t num_heads_k, int32_t head_dim) {
  TG_CHECK(head_dim == kD, "this build supports bf16 with head_dim 128 only (got head_dim %d)", head_dim);
  TG_CHECK(q && k && v && out && lse, "null tensor pointer");
  TG_CHECK(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out),
           "q, k, v and out must be 16-byte aligned");
  TG_CHECK(num_heads > 0 && num_heads_k > 0 && num_heads % num_heads_k == 0,
           "Number of heads in key/value must divide number of heads in query (%d, %d)", num_heads,
           num_heads_k);
  return 0;
}

bool strides_ok(std::initializer_list<int64_t> s) {
  for (int64_t x : s)
    if (x % 8 != 0) return false;
  return true;
}

}  // namespace
}  // namespace tg

using namespace tg;

extern "C" int tg_keybias_fwd(const void *q, const void *k, const void *v, const float *bias_raw,
                              void *out, float *lse, int32_t batch, int32_t seqlen_q, int32_t seqlen_k,
                              int32_t num_heads, int32_t num_heads_k, int32_t head_dim,
                              int64_t q_batch_stride, int64_t q_row_stride, int64_t q_head_stride,
                              int64_t k_batch_stride, int64_t k_row_stride, int64_t k_head_stride,
                              int64_t v_batch_stride, int64_t v_row_stride, int64_t v_head_stride,
                              int64_t o_batch_stride, int64_t o_row_stride, int64_t o_head_stride,
                              int64_t bias_batch_stride, int64_t bias_head_stride, float softmax_scale,
                              int32_t causal, hipStream_t stream) {
  clear_error();
  if (int e = check_common(q, k, v, out, lse, num_heads, num_heads_k, head_dim)) return e;
  TG_CHECK(batch >= 0 && seqlen_q >= 0 && seqlen_k >= 0, "negative size");
  TG_CHECK(strides_ok({q_batch_stride, q_row_stride, q_head_stride, k_batch_stride, k_row_stride,
                       k_head_stride, v_batch_stride, v_row_stride, v_head_stride, o_batch_stride,
                       o_row_stride, o_head_stride}),
           "q/k/v/out strides must be multiples of 8 elements");
  if (batch == 0 || seqlen_q == 0) return 0;
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
  a.n_qtiles = (seqlen_q + kBM - 1) / kBM;
  a.scale_log2 = softmax_scale * kLog2e;
  const int hp = (a.group % 2 == 0) ? 2 : 1;
  const int64_t nblocks = (int64_t)a.n_qtiles * batch * (num_heads / hp);
  TG_CHECK(nblocks < (1ll << 31), "grid too large");
  dispatch_fwd<false>(a, hp, causal != 0, bias_raw != nullptr, (int)nblocks, stream);
  TG_HIP_CHECK(hipPeekAtLastError());
  return 0;
}

extern "C" int tg_keybias_varlen_fwd(const void *q, const void *k, const void *v, const float *bias_raw,
                                     void *out, float *lse, const int32_t *cu_seqlens, int32_t num_seqs,
                                     int32_t max_seqlen, int32_t total, int32_t num_heads,
                                     int32_t num_heads_k, int32_t head_dim, int64_t q_row_stride,
                                     int64_t q_head_stride, int64_t k_row_stride, int64_t k_head_stride,
                                     int64_t v_row_stride, int64_t v_head_stride, int64_t o_row_stride,
                                     int64_t o_head_stride, int64_t bias_seq_stride,
                                     int64_t bias_head_stride, float softmax_scale, int32_t causal,
                                     hipStream_t stream) {
  clear_error();
  if (int e = check_common(q, k, v, out, lse, num_heads, num_heads_k, head_dim)) return e;
  TG_CHECK(cu_seqlens != nullptr, "cu_seqlens is null");
  TG_CHECK(num_seqs >= 0 && max_seqlen >= 0 && total >= 0, "negative size");
  TG_CHECK(strides_ok({q_row_stride, q_head_stride, k_row_stride, k_head_stride, v_row_stride, v_head_stride,
                       o_row_stride, o_head_stride}),
           "q/k/v/out strides must be multiples of 8 elements");
  if (num_seqs == 0 || max_seqlen == 0 || total == 0) return 0;
  FwdArgs a{};
  a.q = static_cast<const bf16_t *>(q);
  a.k = static_cast<const bf16_t *>(k);
  a.v = static_cast<const bf16_t *>(v);
  a.bias = bias_raw;
  a.o = static_cast<bf16_t *>(out);
  a.lse = lse;
  a.cu_seqlens = cu_seqlens;
  a.q_rs = q_row_stride; a.q_hs = q_head_stride;
  a.k_rs = k_row_stride; a.k_hs = k_head_stride;
  a.v_rs = v_row_stride; a.v_hs = v_head_stride;
  a.o_rs = o_row_stride; a.o_hs = o_head_stride;
  a.bias_bs = bias_seq_stride; a.bias_hs = bias_head_stride;
  a.lse_total = total;
  a.batch = num_seqs; a.sq = max_seqlen; a.sk = max_seqlen;
  a.h = num_heads; a.hkv = num_heads_k; a.group = num_heads / num_heads_k;
  a.n_qtiles = (max_seqlen + kBM - 1) / kBM;
  a.scale_log2 = softmax_scale * kLog2e;
  const int hp = (a.group % 2 == 0) ? 2 : 1;
  const int64_t nblocks = (int64_t)a.n_qtiles * num_seqs * (num_heads / hp);
  TG_CHECK(nblocks < (1ll << 31), "grid too large");
  dispatch_fwd<true>(a, hp, causal != 0, bias_raw != nullptr, (int)nblocks, stream);
  TG_HIP_CHECK(hipPeekAtLastError());
  return 0;
}
