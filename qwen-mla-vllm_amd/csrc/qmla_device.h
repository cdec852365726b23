// Device-side building blocks for the gfx950 (CDNA4) MLA decode kernels: vector types, MFMA and
// LDS-transpose wrappers, fp8 conversion, LDS DMA and wave-level reductions.
//
// Operand layouts used throughout (measured on gfx950 for v_mfma_f32_16x16x32_bf16):
//   A[m][k] lives in lane (m + 16*(k/8)), element k%8     (16 rows x 32 k)
//   B[k][n] lives in lane (n + 16*(k/8)), element k%8     (32 k x 16 cols)
//   D[m][n] lives in lane (n + 16*(m/4)), element m%4     (16 x 16 fp32)
// ds_read_b64_tr_b8: within each 16-lane block, lanes 2r and 2r+1 supply row r (8 bytes each,
//   16 bytes per row, 8 rows); lane i receives byte column i of rows 0..7.
// ds_read_b64_tr_b16: within each 16-lane block, lanes 4r..4r+3 supply row r (4 elements each,
//   16 elements per row, 4 rows); lane i receives element column i of rows 0..3.
// global_load_lds_dwordx4: lane l's 16 bytes land at the wave-uniform LDS base + 16*l.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qmla {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;
typedef __attribute__((__vector_size__(8 * sizeof(int)))) int i32x8;
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short i16x4;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(4 * sizeof(_Float16)))) _Float16 f16x4;
typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 f16x2;

#define QMLA_LDS(T, p) ((__attribute__((address_space(3))) T*)(p))

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma16(const f16x8& a, const f16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 8 fp8 bytes -> f16x8, exact (every e4m3fn value is an fp16 value)
__device__ __forceinline__ f16x8 fp8x8_to_f16(const i32x2& raw) {
  f16x8 r;
  f16x2 t;
  t = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(raw[0], 1.0f, false); r[0] = t[0]; r[1] = t[1];
  t = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(raw[0], 1.0f, true);  r[2] = t[0]; r[3] = t[1];
  t = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(raw[1], 1.0f, false); r[4] = t[0]; r[5] = t[1];
  t = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(raw[1], 1.0f, true);  r[6] = t[0]; r[7] = t[1];
  return r;
}

// 16 fp8 e4m3fn bytes -> two bf16x8 (bytes 0-7, bytes 8-15), exact (scale 1.0 is a no-op).
__device__ __forceinline__ void fp8x16_to_bf16(const i32x4& raw, bf16x8& lo, bf16x8& hi) {
  bf16x2 t;
  t = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[0], 1.0f, false); lo[0] = t[0]; lo[1] = t[1];
  t = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[0], 1.0f, true);  lo[2] = t[0]; lo[3] = t[1];
  t = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[1], 1.0f, false); lo[4] = t[0]; lo[5] = t[1];
  t = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[1], 1.0f, true);  lo[6] = t[0]; lo[7] = t[1];
  t = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[2], 1.0f, false); hi[0] = t[0]; hi[1] = t[1];
  t = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[2], 1.0f, true);  hi[2] = t[0]; hi[3] = t[1];
  t = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[3], 1.0f, false); hi[4] = t[0]; hi[5] = t[1];
  t = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[3], 1.0f, true);  hi[6] = t[0]; hi[7] = t[1];
}

// 8 fp8 bytes -> bf16x8
__device__ __forceinline__ bf16x8 fp8x8_to_bf16(const i32x2& raw) {
  bf16x8 r;
  bf16x2 t;
  t = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[0], 1.0f, false); r[0] = t[0]; r[1] = t[1];
  t = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[0], 1.0f, true);  r[2] = t[0]; r[3] = t[1];
  t = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[1], 1.0f, false); r[4] = t[0]; r[5] = t[1];
  t = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[1], 1.0f, true);  r[6] = t[0]; r[7] = t[1];
  return r;
}

__device__ __forceinline__ float fp8_to_f32(uint32_t byte) {
  return __builtin_amdgcn_cvt_f32_fp8((int)byte, 0);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

__device__ __forceinline__ i32x4 lds_read_b128(const char* p) {
  return *reinterpret_cast<const i32x4*>(p);
}

__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return (uint32_t)(uintptr_t)QMLA_LDS(const char, p);
}

// Transposed LDS reads issued as inline asm: through the builtin the compiler cannot tell them
// apart from the LDS-DMA writes still in flight and waits for vmcnt(0) before each one, which
// drains the prefetch ring mid-tile. The result is NOT ready on return: pass it through
// lds_wait() before use.
__device__ __forceinline__ i32x2 lds_read_tr8_async(const char* p) {
  i32x2 r;
  asm volatile("ds_read_b64_tr_b8 %0, %1" : "=v"(r) : "v"(lds_addr(p)));
  return r;
}
__device__ __forceinline__ i32x2 lds_read_tr16_async(const char* p) {
  i32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"(lds_addr(p)));
  return r;
}
// wait for all outstanding LDS reads of this wave; `v` is threaded through so its consumers
// cannot be scheduled before the wait
template <class T>
__device__ __forceinline__ void lds_wait(T& v) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v));
}
template <class T, class U>
__device__ __forceinline__ void lds_wait(T& v, U& w) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v), "+v"(w));
}

// Cache policy of the loads that stream cached rows into LDS. Non-temporal (nt) by default: a row is
// read once per call, and keeping it cached only displaces other lines (measured, alternating runs
// on one box: the FP8 B 128 decode kernel 237-239 us with nt against 245-248 us without, the bf16
// B 64 one 269 against 274 us, the GLA-g2 and 24-head verify ones 1-2% faster). The column-split
// wide kernel keeps the default policy (with nt it measured 1720 us against 1600 us).
constexpr int kCpolStream = 2, kCpolDefault = 0;
// 16 bytes per lane, global -> LDS (wave-uniform LDS base; lane l writes base + 16*l)
template <int CPOL = kCpolStream>
__device__ __forceinline__ void dma16(const void* gsrc, char* lds_base) {
  __builtin_amdgcn_global_load_lds(gsrc, QMLA_LDS(void, lds_base), 16, 0, CPOL);
}
// 16 bytes per lane from a buffer resource (base in SGPRs, per-lane byte offset voff); lanes
// whose offset falls outside the resource read zeros
template <int CPOL = kCpolStream>
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff, char* lds_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, QMLA_LDS(void, lds_base), 16, voff, 0, 0, CPOL);
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// 4 bytes per lane (lane l writes base + 4*l)
__device__ __forceinline__ void dma4(const void* gsrc, char* lds_base) {
  __builtin_amdgcn_global_load_lds(gsrc, QMLA_LDS(void, lds_base), 4, 0, 0);
}
// 4 bytes per lane from a buffer resource (lane l writes base + 4*l; outside the resource: zeros)
__device__ __forceinline__ void dma4_buf(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff, char* lds_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, QMLA_LDS(void, lds_base), 4, voff, 0, 0, 0);
}

// s_waitcnt vmcnt(N) with expcnt/lgkmcnt left unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// max / sum over the 4 lanes {l, l^16, l^32, l^48} (the 4 lane groups of a 16-lane column), with
// VALU lane swaps: permlane16_swap pairs rows r and r^1 of 16 lanes, permlane32_swap the two
// 32-lane halves; whichever element of the returned pair is the lane's own value, the other is
// its partner's.
__device__ __forceinline__ float max_lg(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum_lg(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// max / sum over the 16 lanes that share (lane / 16)
__device__ __forceinline__ float max16(float v) {
  v = fmaxf(v, __shfl_xor(v, 1));
  v = fmaxf(v, __shfl_xor(v, 2));
  v = fmaxf(v, __shfl_xor(v, 4));
  v = fmaxf(v, __shfl_xor(v, 8));
  return v;
}
__device__ __forceinline__ float sum16(float v) {
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 4);
  v += __shfl_xor(v, 8);
  return v;
}

// Workgroup barrier for LDS traffic only. Both __syncthreads() and an LDS-scoped fence make the
// compiler wait for every outstanding global load first (LDS-DMA writes are counted by vmcnt),
// which would drain the DMA prefetch ring at every barrier. This waits for the wave's own LDS
// reads/writes (lgkmcnt) and the barrier; the "memory" clobber keeps the compiler from moving
// memory accesses across it. DMA data is published by an explicit vmcnt wait before it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// A row's softmax sum is exactly +0 when the row saw no token (it is a sum of exponentials, each
// >= +0) and NaN when one of its scores was. The empty-row results (zero output, lse -inf) are keyed
// on the bits, so a NaN sum reaches the output and the lse as NaN, as in the reference's decode,
// whatever a translation unit built without NaN semantics assumes about comparisons.
__device__ __forceinline__ bool empty_sum(float l) { return __float_as_uint(l) == 0u; }
__device__ __forceinline__ bool is_neg_inf(float x) { return __float_as_uint(x) == 0xff800000u; }
// num / l, or 0 for an empty row
__device__ __forceinline__ float inv_sum(float num, float l) { return empty_sum(l) ? 0.f : num / l; }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }
// natural-log lse of a row from its log2-domain reference max and its sum (-inf for an empty row)
__device__ __forceinline__ float row_lse(float m_log2, float l) {
  return empty_sum(l) ? kNegInf : (m_log2 + fast_log2(l)) * kLn2;
}

// How far a row's tile maximum may exceed its softmax reference before the reference moves, given
// the row's running sum l (relative to the reference). A token that does not move it has
// P <= 2^shift <= l / 4, so it holds at most 1/5 of the row's mass and the rounding of its P to
// 16 bits before P.V moves the output by at most 1/5 of that rounding; a token above that share
// moves the reference to itself and gets P = 1 exactly, as the running max of the reference's
// online softmax does (qwen_mla/ops/mla_decode_attention.py:553-560). While a row has little mass
// (its first tokens, a peaked softmax) the shift is 0, i.e. an exact running max; it grows to
// `cap` as the mass accumulates, so the reference rarely moves in long rows.
__device__ __forceinline__ float ref_shift(float l, float cap) {
  return fminf(cap, fmaxf(0.f, fast_log2(l) - 2.0f));
}

}  // namespace qmla
