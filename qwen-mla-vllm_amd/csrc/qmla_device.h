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
typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short i16x4;

#define QMLA_LDS(T, p) ((__attribute__((address_space(3))) T*)(p))

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
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

__device__ __forceinline__ i32x2 lds_read_tr8(const char* p) {
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32(QMLA_LDS(i32x2, p));
}

__device__ __forceinline__ i16x4 lds_read_tr16(const char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(QMLA_LDS(i16x4, p));
}

// 16 bytes per lane, global -> LDS (wave-uniform LDS base; lane l writes base + 16*l)
__device__ __forceinline__ void dma16(const void* gsrc, char* lds_base) {
  __builtin_amdgcn_global_load_lds(gsrc, QMLA_LDS(void, lds_base), 16, 0, 0);
}
// 4 bytes per lane (lane l writes base + 4*l)
__device__ __forceinline__ void dma4(const void* gsrc, char* lds_base) {
  __builtin_amdgcn_global_load_lds(gsrc, QMLA_LDS(void, lds_base), 4, 0, 0);
}

// s_waitcnt vmcnt(N) with expcnt/lgkmcnt left unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
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

// Workgroup barrier that orders LDS only. __syncthreads() also waits for every outstanding global
// load (vmcnt(0)), which would drain the LDS-DMA prefetch ring at every barrier.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

}  // namespace qmla
