// Per-token decoder work around the attention of the gated prefill, one HBM pass each:
//   * residual add + RMSNorm (the input / post-attention norms of a Qwen3 layer and the final norm),
//   * per-head q/k RMSNorm + rotary embedding at each token's own position, writing q in place
//     and k / v into the layer's KV cache rows,
//   * SiLU(gate) * up of the fused gate/up projection;
//   * for the few rows of a decode step: the projections as HBM-bound GEMVs (a row form for rows
//     of up to 2048 inputs, a split-K form for longer ones), optionally with the RMSNorm or the
//     SwiGLU product folded into their input, and the greedy argmax over the logits.
// The prefill's projections (many rows) are plain GEMMs and stay on hipBLASLt.
#include <type_traits>

#include "tg_common.h"
#include "../../include/tokengate_hip.h"

namespace tg {
namespace {

__device__ __forceinline__ void unpack8(u32x4 v, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __builtin_bit_cast(float, v[i] << 16);
    f[2 * i + 1] = __builtin_bit_cast(float, v[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
  u32x4 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
  return v;
}
__device__ __forceinline__ u32x4 ld16(const bf16_t *p) { return *reinterpret_cast<const u32x4 *>(p); }
__device__ __forceinline__ void st16(bf16_t *p, u32x4 v) { *reinterpret_cast<u32x4 *>(p) = v; }

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) x += __shfl_xor(x, m);
  return x;
}

// ---- residual add + RMSNorm: one wave per row, CPL chunks of 8 elements per lane ----------------
// s = residual ? bf16(x + residual) : x;  residual_out = s;  out = bf16(w * s / sqrt(mean(s^2) + eps))
template <int CPL>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const bf16_t *x, int64_t x_rs,
                                                      const bf16_t *res, int64_t res_rs, bf16_t *res_out,
                                                      int64_t ro_rs, const bf16_t *__restrict__ w,
                                                      bf16_t *out, int64_t o_rs, int64_t rows, int d, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave_id();
  if (row >= rows) return;
  const int nch = d >> 3;
  float v[CPL][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = lane + 64 * c;
    if (ch < nch) {
      unpack8(ld16(x + row * x_rs + 8 * ch), v[c]);
      if (res) {
        float r[8];
        unpack8(ld16(res + row * res_rs + 8 * ch), r);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[c][e] = (float)(__bf16)(v[c][e] + r[e]);  // bf16 residual stream
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[c][e] * v[c][e];
    }
  }
  ss = wave_sum(ss);
  const float rinv = rsqrtf(ss / (float)d + eps);
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = lane + 64 * c;
    if (ch < nch) {
      if (res_out) st16(res_out + row * ro_rs + 8 * ch, pack8(v[c]));
      float wf[8], y[8];
      unpack8(ld16(w + 8 * ch), wf);
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = wf[e] * (v[c][e] * rinv);
      st16(out + row * o_rs + 8 * ch, pack8(y));
    }
  }
}

// ---- q/k RMSNorm + RoPE + KV-cache write -----------------------------------------------------
// A workgroup handles kTok tokens.  Their (cos, sin) tables are computed once into LDS; then each
// 16-lane group takes one 128-element head row at a time (lane j holds elements 8j..8j+7, the
// rotate-half partner 8j+-64 sits in lane j^8).
constexpr int kRopeTok = 2;
constexpr int kHeadDim = 128;

__global__ __launch_bounds__(256) void qk_rope_kernel(const bf16_t *qkv, int64_t qkv_rs,
                                                      const int64_t *__restrict__ pos, int64_t T, int H,
                                                      int Hkv, const bf16_t *__restrict__ qw,
                                                      const bf16_t *__restrict__ kw, float eps,
                                                      const float *__restrict__ inv_freq,
                                                      const float *__restrict__ q_head_scale,
                                                      const float *__restrict__ q_row_scale, bf16_t *q_out,
                                                      int64_t q_rs, bf16_t *__restrict__ k_out, int64_t k_rs,
                                                      bf16_t *__restrict__ v_out, int64_t v_rs,
                                                      const int32_t *__restrict__ kv_rows) {
  __shared__ float cs[kRopeTok][kHeadDim / 2][2];
  const int tid = threadIdx.x;
  const int64_t tok0 = (int64_t)blockIdx.x * kRopeTok;
  if (tid < kRopeTok * 64) {
    const int tt = tid >> 6, i = tid & 63;
    const int64_t t = tok0 + tt;
    float s = 0.f, c = 1.f;
    if (t < T) {
      // angle = position * inv_freq, both fp32 (the rotary table's own arithmetic)
      const float ang = (float)pos[t] * inv_freq[i];
      sincosf(ang, &s, &c);
    }
    cs[tt][i][0] = c;
    cs[tt][i][1] = s;
  }
  __syncthreads();
  const int grp = tid >> 4, j = tid & 15;
  const int R = H + 2 * Hkv;
  for (int r = grp; r < kRopeTok * R; r += 16) {
    const int tt = r / R, rr = r - tt * R;
    const int64_t t = tok0 + tt;
    if (t >= T) continue;  // uniform over the 16-lane group
    const bf16_t *src = qkv + t * qkv_rs + (int64_t)rr * kHeadDim + 8 * j;
    const u32x4 raw = ld16(src);
    const int64_t crow = kv_rows ? (int64_t)kv_rows[t] : t;   // this token's KV-cache row
    if (rr >= H + Hkv) {  // value row: copied into the cache
      st16(v_out + crow * v_rs + (int64_t)(rr - H - Hkv) * kHeadDim + 8 * j, raw);
      continue;
    }
    const bool is_q = rr < H;
    float x[8], wf[8];
    unpack8(raw, x);
    unpack8(ld16((is_q ? qw : kw) + 8 * j), wf);
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
    ss += __shfl_xor(ss, 1);
    ss += __shfl_xor(ss, 2);
    ss += __shfl_xor(ss, 4);
    ss += __shfl_xor(ss, 8);
    const float rinv = rsqrtf(ss * (1.f / kHeadDim) + eps);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = wf[e] * (x[e] * rinv);
    const float sgn = j < 8 ? -1.f : 1.f;
    // Query multiplier s = bf16(head * row), applied to the bf16-rounded rotated query with one
    // more bf16 rounding: the reference scales its bf16 query states in bf16 (q * s_eff,
    // qwen3_flex_attention.py:442-451, :400).  With no multiplier s = 1 and the second rounding
    // is exact.
    const float hs = is_q ? (float)(__bf16)((q_head_scale ? q_head_scale[rr] : 1.f) *
                                            (q_row_scale ? q_row_scale[t] : 1.f))
                          : 1.f;
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float p = __shfl_xor(x[e], 8);
      const int fi = (8 * j + e) & 63;
      y[e] = hs * (float)(__bf16)(x[e] * cs[tt][fi][0] + sgn * p * cs[tt][fi][1]);
    }
    bf16_t *dst = is_q ? q_out + t * q_rs + (int64_t)rr * kHeadDim
                       : k_out + crow * k_rs + (int64_t)(rr - H) * kHeadDim;
    st16(dst + 8 * j, pack8(y));
  }
}

// ---- SiLU(gate) * up -----------------------------------------------------------------------
__global__ __launch_bounds__(256) void silu_mul_kernel(const bf16_t *__restrict__ gu, int64_t gu_rs,
                                                       int64_t rows, int inter, bf16_t *__restrict__ out,
                                                       int64_t o_rs) {
  const int nch = inter >> 3;
  const int64_t total = rows * nch;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / nch;
    const int ch = (int)(i - r * nch);
    float g[8], u[8], y[8];
    unpack8(ld16(gu + r * gu_rs + 8 * ch), g);
    unpack8(ld16(gu + r * gu_rs + inter + 8 * ch), u);
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = g[e] / (1.f + __expf(-g[e])) * u[e];
    st16(out + r * o_rs + 8 * ch, pack8(y));
  }
}

// ---- scoring-branch readout: one wave per row --------------------------------------------------
// score[r] = bf16(sum_i bf16(bf16(silu(g_ri)) * u_ri) * w_i) stored as fp32: the finalized gate's
// SwiGLU branch with its down projection absorbed into one (1, inter) row, evaluated with the
// bf16 roundings of an eager bf16 Qwen3MLP (silu output, gate * up product, the GEMM's output);
// the dot product accumulates in fp32.  silu uses the accurate expf, as torch's bf16 silu does.
__global__ __launch_bounds__(256) void branch_readout_kernel(const bf16_t *__restrict__ gu, int64_t gu_rs,
                                                             int64_t rows, int inter,
                                                             const bf16_t *__restrict__ w,
                                                             float *__restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave_id();
  if (row >= rows) return;
  const int nch = inter >> 3;
  const bf16_t *g = gu + row * gu_rs;
  const bf16_t *u = g + inter;
  float acc = 0.f;
#pragma unroll 4
  for (int ch = lane; ch < nch; ch += 64) {
    float gf[8], uf[8], wf[8];
    unpack8(ld16(g + 8 * ch), gf);
    unpack8(ld16(u + 8 * ch), uf);
    unpack8(ld16(w + 8 * ch), wf);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float sl = (float)(__bf16)(gf[e] / (1.f + expf(-gf[e])));
      acc = fmaf((float)(__bf16)(sl * uf[e]), wf[e], acc);
    }
  }
  acc = wave_sum(acc);
  if (lane == 0) out[row] = (float)(__bf16)acc;
}

// ---- Linear layer on a few rows: y[b, v] = bf16(sum_d x[b, d] * w[v, d]) ------------------------
// F.linear on bf16 tensors for the rows of a decode step (1..8): the vocab projection of the rows
// that produce the next token (written as fp32, .float() of the bf16 result) and the decoder
// layers' projections (written as bf16).  HBM-bound on the (n_out, dim) weight: each wave owns 4
// consecutive output rows and issues the 16-byte loads of up to four 512-element column chunks
// of them (16 KB per wave) before their bf16 pair dot products, so that enough of the weight is
// in flight to cover HBM latency even for a 2048 x 2048 matrix; the NR input rows come from L2.
// The input x can be formed on the fly from the previous kernel's output, removing a launch:
//   kPreNorm:   x = bf16(w_n * s / sqrt(mean(s^2) + eps)) with s = bf16(h + res) (res optional),
//               exactly the RMSNorm kernel's arithmetic and summation order; block 0 writes
//               res_out = s (a buffer other than res: every block reads res);
//   kPreSwiGLU: x = bf16(silu(g) * u) of the gate/up rows [g | u], as the silu_mul kernel.
constexpr int kLmMaxRows = 8;
constexpr int kPrePlain = 0, kPreNorm = 1, kPreSwiGLU = 2;
struct LinIn {
  const bf16_t *x;          // plain: input rows; norm: h; swiglu: [gate | up] rows
  int64_t x_rs;
  const bf16_t *res;        // norm: residual stream in (NULL: s = h)
  int64_t res_rs;
  bf16_t *res_out;          // norm: s out (NULL: not written)
  int64_t ro_rs;
  const bf16_t *nw;         // norm weight (dim)
  float eps;
  int inter;                // swiglu: offset of u within a row (= dim)
};
template <int NR, int PRE>
__device__ __forceinline__ u32x4 lin_input(const LinIn &in, int b, int c, const float (&rinv)[NR]) {
  if constexpr (PRE == kPrePlain) {
    return ld16(in.x + b * in.x_rs + c);
  } else if constexpr (PRE == kPreSwiGLU) {
    float g[8], u[8], y[8];
    unpack8(ld16(in.x + b * in.x_rs + c), g);
    unpack8(ld16(in.x + b * in.x_rs + in.inter + c), u);
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = g[e] / (1.f + __expf(-g[e])) * u[e];
    return pack8(y);
  } else {
    float v[8], wf[8], y[8];
    unpack8(ld16(in.x + b * in.x_rs + c), v);
    if (in.res) {
      float r[8];
      unpack8(ld16(in.res + b * in.res_rs + c), r);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (float)(__bf16)(v[e] + r[e]);
    }
    unpack8(ld16(in.nw + c), wf);
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = wf[e] * (v[e] * rinv[b]);
    return pack8(y);
  }
}
// NCH consecutive 512-column chunks of a wave's 4 output rows: every weight load first
// (lin_load), then the bf16 pair dot products against the NR input rows (lin_dot).
template <int NCH>
__device__ __forceinline__ void lin_load(const bf16_t *const (&wr)[4], int cg, u32x4 (&wv)[NCH][4]) {
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
    for (int r = 0; r < 4; ++r) wv[ch][r] = ld16(wr[r] + cg + 512 * ch);
}
// xs: the NR input rows formed once per workgroup in LDS (norm / SwiGLU stages), row stride
// kLinXsRow; NULL for the plain stage, whose rows are read from global memory (L2).
constexpr int kLinXsRow = 2048;
template <int NCH, int NR, int PRE>
__device__ __forceinline__ void lin_dot(const LinIn &in, const bf16_t *xs, const u32x4 (&wv)[NCH][4], int cg,
                                        int lane, float (&acc)[4][NR]) {
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    const int c = cg + 512 * ch + 8 * lane;
#pragma unroll
    for (int b = 0; b < NR; ++b) {
      const u32x4 xv = PRE == kPrePlain ? ld16(in.x + b * in.x_rs + c)
                                        : *reinterpret_cast<const u32x4 *>(xs + b * kLinXsRow + c);
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t wd = wv[ch][r][e], xd = xv[e];   // scalar copies: see u32_as_f32
          acc[r][b] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, wd), __builtin_bit_cast(bf16x2, xd),
                                                      acc[r][b], false);
        }
    }
  }
}
// Rows of at most 2048 inputs (longer ones take the split-K form below).  The norm / SwiGLU
// input stage is formed once per workgroup into LDS: with the norm, wave w computes the sum of
// squares of input rows w, w + 4, ... (in the RMSNorm kernel's order), then the 256 threads
// write the normalised (or SwiGLU) rows; every wave's dot products read them from LDS.
template <int NR, typename OutT, int PRE>
__global__ __launch_bounds__(256) void linear_rows_kernel(LinIn in, const bf16_t *__restrict__ w, int64_t vocab,
                                                          int dim, OutT *__restrict__ out, int64_t out_rs) {
  constexpr bool kStage = PRE != kPrePlain;
  __shared__ __attribute__((aligned(16))) bf16_t xs[kStage ? NR * kLinXsRow : 8];
  __shared__ float rinv_s[NR];
  const int lane = threadIdx.x & 63, wv = wave_id();
  const int64_t v0 = ((int64_t)blockIdx.x * 4 + wv) * 4;
  // rows past the end read the last row (in bounds; their sums are not stored); a wave whose rows
  // are all past the end still takes part in the workgroup's barriers
  const bf16_t *wr[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) wr[r] = w + min(v0 + r, vocab - 1) * dim + 8 * lane;
  const int groups = dim / 8;   // NR * groups <= 256 * NR: thread t owns chunks t + 256 i, i < NR
  // The norm stage's inputs are requested first, then the first 2048 columns of the weight:
  // loads complete in issue order, so the stage can run while the weight bytes stream in.
  constexpr int kIn = PRE == kPreNorm ? NR : 1;
  u32x4 xin[kIn], rin[kIn], nwv[kIn];
  if constexpr (PRE == kPreNorm) {
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const int idx = threadIdx.x + 256 * i;
      if (idx < NR * groups) {
        const int b = idx / groups, c = 8 * (idx - b * groups);
        nwv[i] = ld16(in.nw + c);
        xin[i] = ld16(in.x + b * in.x_rs + c);
        if (in.res) rin[i] = ld16(in.res + b * in.res_rs + c);
      }
    }
  }
  u32x4 wfirst[4][4];
  const bool first = dim >= 2048;
  if (first) lin_load<4>(wr, 0, wfirst);
  if constexpr (kStage) {
    if constexpr (PRE == kPreNorm) {
      // One read of the input rows: s = bf16(h + res) (exact in bf16) goes to LDS (block 0 also
      // writes res_out) and the norm weight of the thread's chunks to registers.  The sums of
      // squares then come from LDS in the RMSNorm kernel's order (lane l sums its chunks l,
      // l + 64, ... element by element, then the wave butterfly), and each thread scales its own
      // chunks in place: the same arithmetic as lin_input, one global round trip fewer.
      const bool writer = blockIdx.x == 0 && in.res_out != nullptr;
#pragma unroll
      for (int i = 0; i < NR; ++i) {
        const int idx = threadIdx.x + 256 * i;
        if (idx < NR * groups) {
          const int b = idx / groups, c = 8 * (idx - b * groups);
          float v[8];
          unpack8(xin[i], v);
          if (in.res) {
            float r[8];
            unpack8(rin[i], r);
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = (float)(__bf16)(v[e] + r[e]);
          }
          const u32x4 pv = pack8(v);
          if (writer) st16(in.res_out + b * in.ro_rs + c, pv);
          *reinterpret_cast<u32x4 *>(xs + b * kLinXsRow + c) = pv;
        }
      }
      __syncthreads();
      for (int b = wv; b < NR; b += 4) {
        float ss = 0.f;
        for (int c = 8 * lane; c < dim; c += 512) {
          float v[8];
          unpack8(*reinterpret_cast<const u32x4 *>(xs + b * kLinXsRow + c), v);
#pragma unroll
          for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
        }
        ss = wave_sum(ss);
        if (lane == 0) rinv_s[b] = rsqrtf(ss / (float)dim + in.eps);
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < NR; ++i) {
        const int idx = threadIdx.x + 256 * i;
        if (idx < NR * groups) {
          const int b = idx / groups, c = 8 * (idx - b * groups);
          float v[8], wf[8], y[8];
          unpack8(*reinterpret_cast<const u32x4 *>(xs + b * kLinXsRow + c), v);
          unpack8(nwv[i], wf);
          const float ri = rinv_s[b];
#pragma unroll
          for (int e = 0; e < 8; ++e) y[e] = wf[e] * (v[e] * ri);
          *reinterpret_cast<u32x4 *>(xs + b * kLinXsRow + c) = pack8(y);
        }
      }
    } else {
      const float rinv[NR] = {};
      for (int idx = threadIdx.x; idx < NR * groups; idx += 256) {
        const int b = idx / groups, c = 8 * (idx - b * groups);
        *reinterpret_cast<u32x4 *>(xs + b * kLinXsRow + c) = lin_input<NR, PRE>(in, b, c, rinv);
      }
    }
    __syncthreads();
  }
  float acc[4][NR];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int b = 0; b < NR; ++b) acc[r][b] = 0.f;
  int cg = 0;
  if (first) {
    lin_dot<4, NR, PRE>(in, xs, wfirst, 0, lane, acc);
    cg = 2048;
  }
  for (; cg + 2048 <= dim; cg += 2048) {
    u32x4 wv_[4][4];
    lin_load<4>(wr, cg, wv_);
    lin_dot<4, NR, PRE>(in, xs, wv_, cg, lane, acc);
  }
  if (dim - cg >= 1024) {
    u32x4 wv_[2][4];
    lin_load<2>(wr, cg, wv_);
    lin_dot<2, NR, PRE>(in, xs, wv_, cg, lane, acc);
    cg += 1024;
  }
  if (dim - cg >= 512) {
    u32x4 wv_[1][4];
    lin_load<1>(wr, cg, wv_);
    lin_dot<1, NR, PRE>(in, xs, wv_, cg, lane, acc);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int b = 0; b < NR; ++b) acc[r][b] = wave_sum(acc[r][b]);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (v0 + r < vocab)
#pragma unroll
        for (int b = 0; b < NR; ++b) {
          const __bf16 y = (__bf16)acc[r][b];
          if constexpr (std::is_same<OutT, float>::value)
            out[b * out_rs + v0 + r] = (float)y;
          else
            out[b * out_rs + v0 + r] = __builtin_bit_cast(bf16_t, y);
        }
  }
}

// Split-K form for dim > 2048 (the down projection, 6144 inputs): the kernel above walks a long
// row in 2048-column steps, one HBM round trip each, over only n_out / 16 workgroups.  Here a
// workgroup (4 waves) owns 4 output rows and wave wv takes the 512-column chunks wv, wv + 4,
// wv + 8, ... of them, so the four waves split the dot products 4 ways.  When dim is 2048 * NJ
// (NJ = 3: 6144) every wave has exactly NJ chunks and requests all of them (NJ x 4 rows x 16 B
// per lane) before anything else, so a workgroup's whole 4-row slice of the weight is in flight
// at once; other multiples of 512 take them one at a time (NJ = 0).
template <int NCH>
__device__ __forceinline__ void lin_load_sk(const bf16_t *const (&wr)[4], int c0, u32x4 (&wv_)[NCH][4]) {
#pragma unroll
  for (int j = 0; j < NCH; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) wv_[j][r] = ld16(wr[r] + c0 + 2048 * j);
}
template <int NCH, int NR, int PRE>
__device__ __forceinline__ void lin_dot_sk(const LinIn &in, const u32x4 (&wv_)[NCH][4], int c0, int lane,
                                        const float (&rinv)[NR], float (&acc)[4][NR]) {
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = c0 + 2048 * j + 8 * lane;
#pragma unroll
    for (int b = 0; b < NR; ++b) {
      const u32x4 xv = lin_input<NR, PRE>(in, b, c, rinv);
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t wd = wv_[j][r][e], xd = xv[e];   // scalar copies: see u32_as_f32
          acc[r][b] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, wd), __builtin_bit_cast(bf16x2, xd),
                                                      acc[r][b], false);
        }
    }
  }
}
// One workgroup (4 waves) per 4 output rows; per wave the bf16 pair dot products of its chunks,
// a wave butterfly per (row, input row), then the four waves' partial sums added in wave order
// through LDS.
template <int NR, typename OutT, int PRE, int NJ>
__global__ __launch_bounds__(256) void linear_rows_splitk_kernel(LinIn in, const bf16_t *__restrict__ w, int64_t vocab,
                                                          int dim, OutT *__restrict__ out, int64_t out_rs) {
  __shared__ float part[4][4][NR];
  const int lane = threadIdx.x & 63, wv = wave_id();
  const int64_t v0 = (int64_t)blockIdx.x * 4;
  // rows past the end read the last row (in bounds; their sums are not stored)
  const bf16_t *wr[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) wr[r] = w + min(v0 + r, vocab - 1) * dim + 8 * lane;
  // the wave's chunks of the weight are requested before the input is formed
  u32x4 wfirst[NJ > 0 ? NJ : 1][4];
  if constexpr (NJ > 0) lin_load_sk<NJ>(wr, 512 * wv, wfirst);
  float rinv[NR];
  if constexpr (PRE == kPreNorm) {
    // sum of squares in the RMSNorm kernel's order: lane l sums its chunks l, l + 64, ... element
    // by element, then the wave butterfly
    const bool writer = blockIdx.x == 0 && wv == 0 && in.res_out != nullptr;
#pragma unroll
    for (int b = 0; b < NR; ++b) {
      float ss = 0.f;
      for (int c = 8 * lane; c < dim; c += 512) {
        float v[8];
        unpack8(ld16(in.x + b * in.x_rs + c), v);
        if (in.res) {
          float r[8];
          unpack8(ld16(in.res + b * in.res_rs + c), r);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = (float)(__bf16)(v[e] + r[e]);
        }
        if (writer) st16(in.res_out + b * in.ro_rs + c, pack8(v));
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
      }
      ss = wave_sum(ss);
      rinv[b] = rsqrtf(ss / (float)dim + in.eps);
    }
  }
  float acc[4][NR];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int b = 0; b < NR; ++b) acc[r][b] = 0.f;
  if constexpr (NJ > 0) {
    lin_dot_sk<NJ, NR, PRE>(in, wfirst, 512 * wv, lane, rinv, acc);
  } else {
    for (int c0 = 512 * wv; c0 < dim; c0 += 2048) {
      u32x4 wv_[1][4];
      lin_load_sk<1>(wr, c0, wv_);
      lin_dot_sk<1, NR, PRE>(in, wv_, c0, lane, rinv, acc);
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int b = 0; b < NR; ++b) acc[r][b] = wave_sum(acc[r][b]);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int b = 0; b < NR; ++b) part[wv][r][b] = acc[r][b];
  }
  __syncthreads();
  const int t = threadIdx.x;
  if (t < 4 * NR) {
    const int r = t / NR, b = t % NR;
    if (v0 + r < vocab) {
      const float sum = ((part[0][r][b] + part[1][r][b]) + part[2][r][b]) + part[3][r][b];
      const __bf16 y = (__bf16)sum;
      if constexpr (std::is_same<OutT, float>::value)
        out[b * out_rs + v0 + r] = (float)y;
      else
        out[b * out_rs + v0 + r] = __builtin_bit_cast(bf16_t, y);
    }
  }
}

// ---- Greedy token: the index of each row's largest logit -----------------------------------------
// torch.argmax semantics: a NaN beats every number, and equal values go to the lower index.  One
// 1024-thread workgroup per row: each thread scans its strided 16-byte pieces, then the (value,
// index) pairs are folded across the wave and, through LDS, across the 16 waves.
__device__ __forceinline__ bool amax_better(float a, int64_t ia, float b, int64_t ib) {
  const bool na = a != a, nb = b != b;
  if (na) return nb ? ia < ib : true;
  if (nb) return false;
  return a == b ? ia < ib : a > b;
}
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const float *__restrict__ x, int64_t rs, int64_t n,
                                                           int64_t *__restrict__ out) {
  const float *row = x + (int64_t)blockIdx.x * rs;
  float best = -INFINITY;
  int64_t bi = n;   // no element yet: loses every comparison with a real one
  const int64_t n4 = n / 4;
  int64_t j = threadIdx.x;
  for (; j + 3 * 1024 < n4; j += 4 * 1024) {   // four independent loads in flight per thread
    f32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = *reinterpret_cast<const f32x4 *>(row + 4 * (j + u * 1024));
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = v[u][e];
        const int64_t ix = 4 * (j + u * 1024) + e;
        if (amax_better(x, ix, best, bi)) { best = x; bi = ix; }
      }
  }
  for (; j < n4; j += 1024) {
    const f32x4 v = *reinterpret_cast<const f32x4 *>(row + 4 * j);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float x = v[e];
      if (amax_better(x, 4 * j + e, best, bi)) { best = x; bi = 4 * j + e; }
    }
  }
  for (int64_t j = 4 * n4 + threadIdx.x; j < n; j += 1024)
    if (amax_better(row[j], j, best, bi)) { best = row[j]; bi = j; }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ob = __shfl_xor(best, o);
    const int64_t oi = __shfl_xor(bi, o);
    if (amax_better(ob, oi, best, bi)) { best = ob; bi = oi; }
  }
  __shared__ float sb[16];
  __shared__ int64_t si[16];
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { sb[w] = best; si[w] = bi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < 16; ++k)
      if (amax_better(sb[k], si[k], best, bi)) { best = sb[k]; bi = si[k]; }
    out[blockIdx.x] = bi;
  }
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace tg

using namespace tg;

extern "C" int tg_rmsnorm(const void *x, int64_t x_row_stride, const void *residual, int64_t residual_row_stride,
                          void *residual_out, int64_t residual_out_row_stride, const void *weight, void *out,
                          int64_t out_row_stride, int64_t n_rows, int32_t dim, float eps, hipStream_t stream) {
  clear_error();
  TG_CHECK(x && weight && out, "rmsnorm: null pointer");
  TG_CHECK(n_rows >= 0, "rmsnorm: negative row count");
  TG_CHECK(dim > 0 && dim % 8 == 0 && dim <= 64 * 8 * 8, "rmsnorm: dim must be a multiple of 8, at most 4096");
  TG_CHECK(x_row_stride >= dim && out_row_stride >= dim && (!residual || residual_row_stride >= dim) &&
               (!residual_out || residual_out_row_stride >= dim),
           "rmsnorm: row strides must be at least dim");
  TG_CHECK(x_row_stride % 8 == 0 && out_row_stride % 8 == 0 && (!residual || residual_row_stride % 8 == 0) &&
               (!residual_out || residual_out_row_stride % 8 == 0),
           "rmsnorm: row strides must be multiples of 8 elements");
  TG_CHECK(aligned16(x) && aligned16(weight) && aligned16(out) && aligned16(residual) && aligned16(residual_out),
           "rmsnorm: pointers must be 16-byte aligned");
  TG_CHECK(eps >= 0.f, "rmsnorm: eps must be non-negative");
  if (n_rows == 0) return 0;
  const int64_t blocks = (n_rows + 3) / 4;
  TG_CHECK(blocks < (1ll << 31), "rmsnorm: too many rows");
  const int cpl = (dim / 8 + 63) / 64;
  auto *xp = static_cast<const bf16_t *>(x);
  auto *rp = static_cast<const bf16_t *>(residual);
  auto *rop = static_cast<bf16_t *>(residual_out);
  auto *wp = static_cast<const bf16_t *>(weight);
  auto *op = static_cast<bf16_t *>(out);
#define TG_RMS(N)                                                                                  \
  case N:                                                                                          \
    hipLaunchKernelGGL(rmsnorm_kernel<N>, dim3((unsigned)blocks), dim3(256), 0, stream, xp, x_row_stride, rp, \
                       residual_row_stride, rop, residual_out_row_stride, wp, op, out_row_stride, n_rows, dim, eps); \
    break;
  switch (cpl) {
    TG_RMS(1) TG_RMS(2) TG_RMS(4) TG_RMS(8)
    case 3: hipLaunchKernelGGL(rmsnorm_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, stream, xp, x_row_stride, rp,
                               residual_row_stride, rop, residual_out_row_stride, wp, op, out_row_stride, n_rows, dim,
                               eps); break;
    default: hipLaunchKernelGGL(rmsnorm_kernel<8>, dim3((unsigned)blocks), dim3(256), 0, stream, xp, x_row_stride, rp,
                                residual_row_stride, rop, residual_out_row_stride, wp, op, out_row_stride, n_rows,
                                dim, eps); break;
  }
#undef TG_RMS
  TG_HIP_CHECK(hipGetLastError());
  return 0;
}

extern "C" int tg_qk_norm_rope(const void *qkv, int64_t qkv_row_stride, const int64_t *positions, int64_t n_tokens,
                               int32_t num_heads, int32_t num_heads_k, int32_t head_dim, const void *q_norm_weight,
                               const void *k_norm_weight, float eps, const float *inv_freq, const float *q_head_scale,
                               const float *q_row_scale, void *q_out, int64_t q_row_stride, void *k_out,
                               int64_t k_row_stride, void *v_out, int64_t v_row_stride, const int32_t *kv_rows,
                               hipStream_t stream) {
  clear_error();
  TG_CHECK(qkv && positions && q_norm_weight && k_norm_weight && inv_freq && q_out && k_out && v_out,
           "qk_norm_rope: null pointer");
  TG_CHECK(head_dim == kHeadDim, "qk_norm_rope: head_dim must be 128");
  TG_CHECK(num_heads > 0 && num_heads_k > 0 && num_heads <= 256 && num_heads_k <= 256,
           "qk_norm_rope: head counts must be in 1..256");
  TG_CHECK(n_tokens >= 0, "qk_norm_rope: negative token count");
  TG_CHECK(qkv_row_stride % 8 == 0 && q_row_stride % 8 == 0 && k_row_stride % 8 == 0 && v_row_stride % 8 == 0,
           "qk_norm_rope: row strides must be multiples of 8 elements");
  TG_CHECK(qkv_row_stride >= (int64_t)(num_heads + 2 * num_heads_k) * kHeadDim,
           "qk_norm_rope: qkv rows must hold q, k and v of every head");
  TG_CHECK(q_row_stride >= (int64_t)num_heads * kHeadDim && k_row_stride >= (int64_t)num_heads_k * kHeadDim &&
               v_row_stride >= (int64_t)num_heads_k * kHeadDim,
           "qk_norm_rope: q/k/v output rows must hold every head");
  TG_CHECK(aligned16(qkv) && aligned16(q_out) && aligned16(k_out) && aligned16(v_out) &&
               aligned16(q_norm_weight) && aligned16(k_norm_weight),
           "qk_norm_rope: pointers must be 16-byte aligned");
  if (n_tokens == 0) return 0;
  const int64_t blocks = (n_tokens + kRopeTok - 1) / kRopeTok;
  TG_CHECK(blocks < (1ll << 31), "qk_norm_rope: too many tokens");
  hipLaunchKernelGGL(qk_rope_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const bf16_t *>(qkv), qkv_row_stride, positions, n_tokens, num_heads, num_heads_k,
                     static_cast<const bf16_t *>(q_norm_weight), static_cast<const bf16_t *>(k_norm_weight), eps,
                     inv_freq, q_head_scale, q_row_scale, static_cast<bf16_t *>(q_out), q_row_stride,
                     static_cast<bf16_t *>(k_out), k_row_stride, static_cast<bf16_t *>(v_out), v_row_stride,
                     kv_rows);
  TG_HIP_CHECK(hipGetLastError());
  return 0;
}

extern "C" int tg_silu_mul(const void *gate_up, int64_t gate_up_row_stride, int64_t n_rows, int32_t inter,
                           void *out, int64_t out_row_stride, hipStream_t stream) {
  clear_error();
  TG_CHECK(gate_up && out, "silu_mul: null pointer");
  TG_CHECK(n_rows >= 0 && inter > 0 && inter % 8 == 0, "silu_mul: inter must be a positive multiple of 8");
  TG_CHECK(gate_up_row_stride % 8 == 0 && out_row_stride % 8 == 0 && gate_up_row_stride >= 2 * (int64_t)inter &&
               out_row_stride >= inter,
           "silu_mul: row strides must be multiples of 8, gate_up rows must hold 2*inter and out rows inter "
           "elements");
  TG_CHECK(aligned16(gate_up) && aligned16(out), "silu_mul: pointers must be 16-byte aligned");
  if (n_rows == 0) return 0;
  const int64_t chunks = n_rows * (inter / 8);
  const int64_t blocks = std::min<int64_t>((chunks + 255) / 256, 256 * 64);
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const bf16_t *>(gate_up), gate_up_row_stride, n_rows, inter,
                     static_cast<bf16_t *>(out), out_row_stride);
  TG_HIP_CHECK(hipGetLastError());
  return 0;
}

extern "C" int tg_gate_branch_readout(const void *gate_up, int64_t gate_up_row_stride, int64_t n_rows,
                                      int32_t inter, const void *w_row, float *scores, hipStream_t stream) {
  clear_error();
  TG_CHECK(gate_up && w_row && scores, "branch_readout: null pointer");
  TG_CHECK(n_rows >= 0 && inter > 0 && inter % 8 == 0, "branch_readout: inter must be a positive multiple of 8");
  TG_CHECK(gate_up_row_stride % 8 == 0 && gate_up_row_stride >= 2 * (int64_t)inter,
           "branch_readout: gate_up row stride must be a multiple of 8 holding 2*inter elements");
  TG_CHECK(aligned16(gate_up) && aligned16(w_row), "branch_readout: gate_up and w_row must be 16-byte aligned");
  if (n_rows == 0) return 0;
  const int64_t blocks = (n_rows + 3) / 4;
  TG_CHECK(blocks < (1ll << 31), "branch_readout: too many rows");
  hipLaunchKernelGGL(branch_readout_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const bf16_t *>(gate_up), gate_up_row_stride, n_rows, inter,
                     static_cast<const bf16_t *>(w_row), scores);
  TG_HIP_CHECK(hipGetLastError());
  return 0;
}

namespace tg {
namespace {

template <typename OutT, int PRE>
int launch_linear_rows(const LinIn &in, int32_t n_rows, const void *weight, int64_t n_out, int32_t dim, OutT *out,
                       int64_t out_row_stride, hipStream_t stream) {
  const int64_t blocks = (n_out + 15) / 16;
  const bf16_t *wp = static_cast<const bf16_t *>(weight);
  const int64_t sk_blocks = (n_out + 3) / 4;
#define TG_LR(NR)                                                                                          \
  if (n_rows == NR) {                                                                                      \
    if (dim <= 2048)                                                                                       \
      hipLaunchKernelGGL((linear_rows_kernel<NR, OutT, PRE>), dim3((unsigned)blocks), dim3(256), 0, stream, in, wp, \
                         n_out, dim, out, out_row_stride);                                                 \
    else if (dim == 6144)                                                                                  \
      hipLaunchKernelGGL((linear_rows_splitk_kernel<NR, OutT, PRE, 3>), dim3((unsigned)sk_blocks), dim3(256), 0,  \
                         stream, in, wp, n_out, dim, out, out_row_stride);                                 \
    else                                                                                                   \
      hipLaunchKernelGGL((linear_rows_splitk_kernel<NR, OutT, PRE, 0>), dim3((unsigned)sk_blocks), dim3(256), 0,  \
                         stream, in, wp, n_out, dim, out, out_row_stride);                                 \
  }
  TG_LR(1) TG_LR(2) TG_LR(3) TG_LR(4) TG_LR(5) TG_LR(6) TG_LR(7) TG_LR(8)
#undef TG_LR
  TG_HIP_CHECK(hipGetLastError());
  return 0;
}
int check_linear_rows(const char *what, const void *x, int64_t x_row_stride, int32_t n_rows, const void *weight,
                      int64_t n_out, int32_t dim, const void *out, int64_t out_row_stride) {
  TG_CHECK(x && weight && out, "%s: null pointer", what);
  TG_CHECK(n_rows >= 1 && n_rows <= kLmMaxRows, "%s: 1 to %d rows (got %d)", what, kLmMaxRows, n_rows);
  TG_CHECK(dim > 0 && dim % 512 == 0, "%s: dim must be a positive multiple of 512 (got %d)", what, dim);
  TG_CHECK(n_out > 0 && x_row_stride % 8 == 0 && x_row_stride >= dim && out_row_stride >= n_out,
           "%s: bad output size or row strides", what);
  TG_CHECK(aligned16(x) && aligned16(weight), "%s: x and weight must be 16-byte aligned", what);
  TG_CHECK((n_out + 15) / 16 < (1ll << 31), "%s: too many output features", what);
  return 0;
}

}  // namespace
}  // namespace tg

using namespace tg;

extern "C" int tg_lm_head(const void *x, int64_t x_row_stride, int32_t n_rows, const void *weight, int64_t vocab,
                          int32_t dim, float *out, int64_t out_row_stride, hipStream_t stream) {
  clear_error();
  if (int e = check_linear_rows("lm_head", x, x_row_stride, n_rows, weight, vocab, dim, out, out_row_stride)) return e;
  LinIn in{};
  in.x = static_cast<const bf16_t *>(x);
  in.x_rs = x_row_stride;
  return launch_linear_rows<float, kPrePlain>(in, n_rows, weight, vocab, dim, out, out_row_stride, stream);
}

extern "C" int tg_linear_rows(const void *x, int64_t x_row_stride, int32_t n_rows, const void *weight,
                              int64_t n_out, int32_t dim, void *out, int64_t out_row_stride, hipStream_t stream) {
  clear_error();
  if (int e = check_linear_rows("linear_rows", x, x_row_stride, n_rows, weight, n_out, dim, out, out_row_stride))
    return e;
  LinIn in{};
  in.x = static_cast<const bf16_t *>(x);
  in.x_rs = x_row_stride;
  return launch_linear_rows<bf16_t, kPrePlain>(in, n_rows, weight, n_out, dim, static_cast<bf16_t *>(out),
                                               out_row_stride, stream);
}

extern "C" int tg_linear_rows_norm(const void *h, int64_t h_row_stride, const void *residual,
                                   int64_t residual_row_stride, void *residual_out, int64_t residual_out_row_stride,
                                   const void *norm_weight, float eps, int32_t n_rows, const void *weight,
                                   int64_t n_out, int32_t dim, void *out, int64_t out_row_stride, int32_t out_fp32,
                                   hipStream_t stream) {
  clear_error();
  if (int e = check_linear_rows("linear_rows_norm", h, h_row_stride, n_rows, weight, n_out, dim, out, out_row_stride))
    return e;
  TG_CHECK(norm_weight && aligned16(norm_weight), "linear_rows_norm: norm weight must be non-null and 16-byte aligned");
  TG_CHECK(!residual || (aligned16(residual) && residual_row_stride % 8 == 0 && residual_row_stride >= dim),
           "linear_rows_norm: bad residual");
  TG_CHECK(!residual_out || (aligned16(residual_out) && residual_out_row_stride % 8 == 0 &&
                             residual_out_row_stride >= dim && residual_out != residual),
           "linear_rows_norm: bad residual_out (it must not be the residual input)");
  TG_CHECK(eps >= 0.f, "linear_rows_norm: eps must be non-negative");
  LinIn in{};
  in.x = static_cast<const bf16_t *>(h);
  in.x_rs = h_row_stride;
  in.res = static_cast<const bf16_t *>(residual);
  in.res_rs = residual_row_stride;
  in.res_out = static_cast<bf16_t *>(residual_out);
  in.ro_rs = residual_out_row_stride;
  in.nw = static_cast<const bf16_t *>(norm_weight);
  in.eps = eps;
  if (out_fp32)
    return launch_linear_rows<float, kPreNorm>(in, n_rows, weight, n_out, dim, static_cast<float *>(out),
                                               out_row_stride, stream);
  return launch_linear_rows<bf16_t, kPreNorm>(in, n_rows, weight, n_out, dim, static_cast<bf16_t *>(out),
                                              out_row_stride, stream);
}

extern "C" int tg_linear_rows_swiglu(const void *gate_up, int64_t gate_up_row_stride, int32_t n_rows, int32_t inter,
                                     const void *weight, int64_t n_out, void *out, int64_t out_row_stride,
                                     hipStream_t stream) {
  clear_error();
  if (int e = check_linear_rows("linear_rows_swiglu", gate_up, gate_up_row_stride, n_rows, weight, n_out, inter, out,
                                out_row_stride))
    return e;
  TG_CHECK(gate_up_row_stride >= 2 * (int64_t)inter, "linear_rows_swiglu: gate/up rows hold 2 * inter values");
  LinIn in{};
  in.x = static_cast<const bf16_t *>(gate_up);
  in.x_rs = gate_up_row_stride;
  in.inter = inter;
  return launch_linear_rows<bf16_t, kPreSwiGLU>(in, n_rows, weight, n_out, inter, static_cast<bf16_t *>(out),
                                                out_row_stride, stream);
}

extern "C" int tg_argmax_rows(const float *x, int64_t x_row_stride, int32_t n_rows, int64_t n_cols, int64_t *out,
                              hipStream_t stream) {
  clear_error();
  TG_CHECK(x && out, "argmax_rows: null pointer");
  TG_CHECK(n_rows >= 0 && n_cols > 0, "argmax_rows: need n_rows >= 0 and n_cols > 0");
  TG_CHECK(x_row_stride >= n_cols && x_row_stride % 4 == 0, "argmax_rows: row stride must be >= n_cols and a multiple of 4");
  TG_CHECK(aligned16(x), "argmax_rows: x must be 16-byte aligned");
  if (n_rows == 0) return 0;
  hipLaunchKernelGGL(argmax_rows_kernel, dim3((unsigned)n_rows), dim3(1024), 0, stream, x, x_row_stride, n_cols, out);
  TG_HIP_CHECK(hipGetLastError());
  return 0;
}
