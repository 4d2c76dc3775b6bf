// Shared device helpers for the gfx950 kernels: vector types, MFMA wrappers, LDS access,
// cross-lane reductions, and the thread-local error string behind tg_last_error().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

namespace tg {

typedef uint16_t bf16_t;  // raw bf16 bits in global memory

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---- host-side error reporting -------------------------------------------------------------
int set_error(const char *fmt, ...);   // formats into the thread-local buffer, returns 1
void clear_error();
const char *last_error();

#define TG_CHECK(cond, ...)                 \
  do {                                      \
    if (!(cond)) return ::tg::set_error(__VA_ARGS__); \
  } while (0)

#define TG_HIP_CHECK(expr)                                                              \
  do {                                                                                  \
    hipError_t _e = (expr);                                                             \
    if (_e != hipSuccess)                                                               \
      return ::tg::set_error("%s failed: %s", #expr, hipGetErrorString(_e));            \
  } while (0)

// ---- device helpers -----------------------------------------------------------------------

// C = A(32x16) * B(16x32) + C on the bf16 matrix cores.  Lane l holds A[l%32][8*(l/32)+j] and
// B[8*(l/32)+j][l%32] for j=0..7; C value v sits at row 8*(v/4)+4*(l/32)+(v%4), column l%32.
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// 16-byte LDS load / store at a byte offset into a __shared__ buffer.
__device__ __forceinline__ bf16x8 lds_load16(const char *base, uint32_t byte_off) {
  return *reinterpret_cast<const bf16x8 *>(base + byte_off);
}
__device__ __forceinline__ void lds_store16(char *base, uint32_t byte_off, u32x4 v) {
  *reinterpret_cast<u32x4 *>(base + byte_off) = v;
}
__device__ __forceinline__ void lds_store8(char *base, uint32_t byte_off, u32x2 v) {
  *reinterpret_cast<u32x2 *>(base + byte_off) = v;
}

// 16-byte global load with a validity predicate (zero when invalid, no access made).
__device__ __forceinline__ u32x4 gload16(const bf16_t *p, bool valid) {
  u32x4 r = {0u, 0u, 0u, 0u};
  if (valid) r = *reinterpret_cast<const u32x4 *>(p);
  return r;
}

// Combine a value held by lane l and lane l^32 (the two halves of a wave64).
__device__ __forceinline__ float pair_max(float x) { return fmaxf(x, __shfl_xor(x, 32)); }
// Reinterpret a 32-bit value as float.  Use this (or a copy into a scalar) instead of applying
// __builtin_bit_cast to an element of a vector or of a builtin's result pair directly: this
// compiler lowers __builtin_bit_cast(float, v[i]) to element 0 whatever i is.
__device__ __forceinline__ float u32_as_f32(uint32_t u) { return __builtin_bit_cast(float, u); }
// max of the two values a permlane swap returns.  A bare v_max_f32: fmaxf would first
// canonicalise both operands (two more VALU instructions), which only matters for signalling
// NaNs, and the values reduced here are arithmetic results, never signalling NaNs.
template <typename Pair> __device__ __forceinline__ float swap_pair_max(const Pair &sw) {
  const uint32_t lo = sw[0], hi = sw[1];
  float d;
  asm("v_max_f32 %0, %1, %2" : "=v"(d) : "v"(u32_as_f32(lo)), "v"(u32_as_f32(hi)));
  return d;
}
// Same as pair_max without the LDS crossbar: v_permlane32_swap(x, x) returns (lower half in both
// halves, upper half in both halves), so the max of the two is max(x[l], x[l^32]) in every lane.
__device__ __forceinline__ float half_swap_max(float x) {
  return swap_pair_max(__builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x),
                                                        __builtin_bit_cast(uint32_t, x), false, false));
}
__device__ __forceinline__ float pair_sum(float x) { return x + __shfl_xor(x, 32); }
// Max over the four 16-lane groups (lanes l, l^16, l^32, l^48): v_permlane16_swap(x, x) returns
// (rows 0 and 2 in both rows of each pair, rows 1 and 3 likewise), whose max is max(x[l], x[l^16]);
// then the same across the two halves.
__device__ __forceinline__ float quad_swap_max(float x) {
  return half_swap_max(swap_pair_max(__builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x),
                                                                      __builtin_bit_cast(uint32_t, x), false, false)));
}
__device__ __forceinline__ float quad_sum(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}
// C = A(16x32) * B(32x16) + C on the bf16 matrix cores.  Lane l holds A[l%16][8*(l/16)+j] and
// B[8*(l/16)+j][l%16] for j=0..7; C value i sits at row 4*(l/16)+i, column l%16.
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ---- buffer resources and LDS DMA (gfx950) --------------------------------------------------
typedef __amdgpu_buffer_rsrc_t brsrc_t;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) s16x4 lds_s16x4_t;

// Raw buffer descriptor over [base, base + num_bytes): loads past num_bytes return zero and
// make no memory access.
__device__ __forceinline__ brsrc_t make_rsrc(const void *base, uint32_t num_bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)num_bytes, 0x00020000);
}
// Asynchronous 16-byte-per-lane copy global -> LDS: lane i's 16 bytes land at
// lds_wave_base + 16*i.  Completion is tracked by vmcnt.
__device__ __forceinline__ void dma16(brsrc_t rs, void *lds_wave_base, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t *)lds_wave_base, 16, voff, 0, 0, 0);
}
// Same, 4 bytes per lane (lds_wave_base + 4*i).
__device__ __forceinline__ void dma4(brsrc_t rs, void *lds_wave_base, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t *)lds_wave_base, 4, voff, 0, 0, 0);
}
// Transposing LDS read (ds_read_b64_tr_b16): within each group of 16 lanes, lane j receives
// element j%4 of the four 16-bit values addressed by lanes 4k + j/4, for k = 0..3.
__device__ __forceinline__ s16x4 lds_read_tr16(const void *lds_addr) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t *)lds_addr);
}
__device__ __forceinline__ void wait_all_mem() { __builtin_amdgcn_s_waitcnt(0); }
// Wait for this wave's outstanding vector-memory operations down to N (compile-time, 0..63).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is six bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}
// Workgroup barrier for LDS ring buffers filled by LDS DMA: this wave's LDS reads are complete
// (lgkmcnt 0) and every wave has arrived.  Unlike __syncthreads() it does not make the wave wait
// for its own DMA still in flight into other ring slots (those are waited for by count, wait_vm);
// the empty asm statements keep the compiler from moving LDS accesses across the barrier.
__device__ __forceinline__ void ring_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0); vmcnt and expcnt unconstrained
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
// Wait until at most n (0..63) vector-memory operations of this wave are outstanding (vmcnt: low
// four bits in [3:0], high two in [15:14]), leaving the LDS and export counters unconstrained.
__device__ __forceinline__ void wait_vm_outstanding(int n) {
#define TG_VMCNT(N) case N: __builtin_amdgcn_s_waitcnt(((N) & 15) | (((N) >> 4) << 14) | 0x0F70); break;
#define TG_VMCNT8(B) TG_VMCNT(B) TG_VMCNT(B + 1) TG_VMCNT(B + 2) TG_VMCNT(B + 3) TG_VMCNT(B + 4) TG_VMCNT(B + 5) \
  TG_VMCNT(B + 6) TG_VMCNT(B + 7)
  switch (n) {
    TG_VMCNT8(0) TG_VMCNT8(8) TG_VMCNT8(16) TG_VMCNT8(24) TG_VMCNT8(32) TG_VMCNT8(40) TG_VMCNT8(48)
    TG_VMCNT(56) TG_VMCNT(57) TG_VMCNT(58) TG_VMCNT(59) TG_VMCNT(60) TG_VMCNT(61) TG_VMCNT(62)
    default: __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | 0x0F70); break;
  }
#undef TG_VMCNT8
#undef TG_VMCNT
}

// Index of this wave in its workgroup, held in a scalar register.  The compiler cannot prove that
// threadIdx.x / 64 is the same in every lane of a wave, so without this every condition derived
// from the wave index (tile skips, mask checks) is compiled as exec-masked per-lane code that
// runs on every path instead of a scalar branch.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Two floats -> packed bf16 pair (round to nearest even, v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 p;
  p[0] = (__bf16)lo;
  p[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, p);
}

// acc + lo + hi of a packed bf16 pair, in fp32 (v_dot2c_f32_bf16 against (1, 1)).
__device__ __forceinline__ float sum_bf16x2(uint32_t pair, float acc) {
  bf16x2 one;
  one[0] = (__bf16)1.0f;
  one[1] = (__bf16)1.0f;
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pair), one, acc, false);
}

__device__ __forceinline__ float bf16_to_f32(bf16_t x) {
  return __builtin_bit_cast(float, (uint32_t)x << 16);
}

// Compute units of the current device (cached per device id).
inline int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

}  // namespace tg
