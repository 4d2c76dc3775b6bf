// Per-token decoder work around the attention of the gated prefill, one HBM pass each:
//   * residual add + RMSNorm (the input / post-attention norms of a Qwen3 layer and the final norm),
//   * per-head q/k RMSNorm + rotary embedding at each token's own position, writing q in place
//     and k / v into the layer's KV cache rows,
//   * SiLU(gate) * up of the fused gate/up projection.
// The projections themselves are plain GEMMs and stay on hipBLASLt.
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

// ---- LM head on a few rows: logits[b, v] = bf16(sum_d x[b, d] * w[v, d]) as fp32 -----------------
// The vocab projection of the rows that produce the next token (F.linear on bf16 tensors, then
// .float()).  HBM-bound on the (vocab, dim) weight: each wave owns 4 consecutive vocab rows and
// issues all their 16-byte loads of a 512-element column chunk before the bf16 pair dot products;
// the NR input rows are read from L2 alongside.
constexpr int kLmMaxRows = 8;
template <int NR>
__global__ __launch_bounds__(256) void lm_head_kernel(const bf16_t *__restrict__ x, int64_t x_rs,
                                                      const bf16_t *__restrict__ w, int64_t vocab, int dim,
                                                      float *__restrict__ out, int64_t out_rs) {
  const int lane = threadIdx.x & 63;
  const int64_t v0 = ((int64_t)blockIdx.x * 4 + wave_id()) * 4;
  if (v0 >= vocab) return;
  float acc[4][NR];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int b = 0; b < NR; ++b) acc[r][b] = 0.f;
  for (int c = 0; c < dim; c += 512) {
    u32x4 wv[4], xv[NR];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      wv[r] = u32x4{0u, 0u, 0u, 0u};
      if (v0 + r < vocab) wv[r] = *reinterpret_cast<const u32x4 *>(w + (v0 + r) * dim + c + 8 * lane);
    }
#pragma unroll
    for (int b = 0; b < NR; ++b) xv[b] = *reinterpret_cast<const u32x4 *>(x + b * x_rs + c + 8 * lane);
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int b = 0; b < NR; ++b)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t wd = wv[r][e], xd = xv[b][e];
          acc[r][b] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, wd), __builtin_bit_cast(bf16x2, xd),
                                                      acc[r][b], false);
        }
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
        for (int b = 0; b < NR; ++b) out[b * out_rs + v0 + r] = (float)(__bf16)acc[r][b];
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

extern "C" int tg_lm_head(const void *x, int64_t x_row_stride, int32_t n_rows, const void *weight, int64_t vocab,
                          int32_t dim, float *out, int64_t out_row_stride, hipStream_t stream) {
  clear_error();
  TG_CHECK(x && weight && out, "lm_head: null pointer");
  TG_CHECK(n_rows >= 1 && n_rows <= kLmMaxRows, "lm_head: 1 to %d rows (got %d)", kLmMaxRows, n_rows);
  TG_CHECK(dim > 0 && dim % 512 == 0, "lm_head: dim must be a positive multiple of 512 (got %d)", dim);
  TG_CHECK(vocab > 0 && x_row_stride % 8 == 0 && x_row_stride >= dim && out_row_stride >= vocab,
           "lm_head: bad vocab or row strides");
  TG_CHECK(aligned16(x) && aligned16(weight), "lm_head: x and weight must be 16-byte aligned");
  const int64_t blocks = (vocab + 15) / 16;
  TG_CHECK(blocks < (1ll << 31), "lm_head: vocab too large");
  const bf16_t *xp = static_cast<const bf16_t *>(x);
  const bf16_t *wp = static_cast<const bf16_t *>(weight);
#define TG_LM(NR)                                                                                          \
  if (n_rows == NR)                                                                                        \
    hipLaunchKernelGGL(lm_head_kernel<NR>, dim3((unsigned)blocks), dim3(256), 0, stream, xp, x_row_stride, wp, \
                       vocab, dim, out, out_row_stride);
  TG_LM(1) TG_LM(2) TG_LM(3) TG_LM(4) TG_LM(5) TG_LM(6) TG_LM(7) TG_LM(8)
#undef TG_LM
  TG_HIP_CHECK(hipGetLastError());
  return 0;
}
