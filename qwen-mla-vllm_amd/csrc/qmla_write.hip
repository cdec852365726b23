// qmla_write.hip -- gfx950 cache-row writer: one new token per input row into its paged cache slot.
//
// Reference: qwen_mla/mla_impl.py:309-342 (QwenMLATritonImpl.do_kv_cache_update, the FP8 writer
// with log8 or bf16-byte rms tails) and vLLM's concat_and_cache_mla for the rows the plugin hands
// to it (bf16 caches; FP8 caches whose rms is e4m3). One wave per row: lane l converts latent
// elements [8l, 8l+8) (and further 512-column blocks for wider latents), lanes 0.. the rope in 8s
// and the rms tail one head each. Rows are independent, so the grid is rows / 4 workgroups of 256.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qmla.h"
#include "qmla_device.h"

namespace qmla {
namespace wr {

constexpr int ROWS_PER_WG = 4;

struct WParams {
  const uint16_t* kv_c;
  int64_t kv_c_stride;
  const uint16_t* k_pe;
  int64_t k_pe_stride;
  const int64_t* slots;
  int n, d_c, rope_w, rms_heads, kv_dtype, rms_mode;
  const float* k_scale;
  char* cache;
  int64_t page_stride, token_stride;
  int page_size;
  int64_t num_slots;
};

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// clamp(x * inv, -448, 448) in fp32 (NaN stays NaN, as torch.clamp leaves it)
__device__ __forceinline__ float sat448(float x, float inv) {
  const float v = x * inv;
  return v > 448.0f ? 448.0f : (v < -448.0f ? -448.0f : v);
}

// four fp32 values -> four e4m3fn bytes, round to nearest even (v_cvt_pk_fp8_f32, OCP e4m3 on gfx950)
__device__ __forceinline__ uint32_t pack_e4m3(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

// 8 bf16 inputs -> 8 e4m3 bytes
__device__ __forceinline__ uint2 quant8(const uint16_t* src, float inv) {
  const uint4 raw = *reinterpret_cast<const uint4*>(src);
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  float f[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = sat448(bf16_to_f32((uint16_t)(w[i] & 0xFFFF)), inv);
    f[2 * i + 1] = sat448(bf16_to_f32((uint16_t)(w[i] >> 16)), inv);
  }
  return make_uint2(pack_e4m3(f[0], f[1], f[2], f[3]), pack_e4m3(f[4], f[5], f[6], f[7]));
}

// log8 code of one rms value: round-half-even((log2(max(r, 1e-30)) + 3) * (255 / 6)), clamped to
// [0, 255]; the logarithm is evaluated in double and rounded once to fp32, the rest in fp32
__device__ __forceinline__ uint32_t log8_code(float r) {
  const float rc = r < 1e-30f ? 1e-30f : r;   // clamp_min keeps NaN
  const float lg = (float)log2((double)rc);
  const float c = rintf((lg - (-3.0f)) * 42.5f);
  return (uint32_t)(c < 0.0f ? 0.0f : (c > 255.0f ? 255.0f : c));
}

__global__ __launch_bounds__(64 * ROWS_PER_WG) void write_kernel(const WParams p) {
  const int lane = threadIdx.x & 63;
  const int row = (int)blockIdx.x * ROWS_PER_WG + (int)(threadIdx.x >> 6);
  if (row >= p.n) return;
  int64_t slot = p.slots[row];
  if (slot < 0) slot = 0;
  if (slot >= p.num_slots) return;
  const int64_t page = slot / p.page_size, tok = slot - page * p.page_size;
  char* dst = p.cache + page * p.page_stride + tok * p.token_stride;
  const uint16_t* kc = p.kv_c + (int64_t)row * p.kv_c_stride;
  const uint16_t* kp = p.k_pe + (int64_t)row * p.k_pe_stride;

  if (p.kv_dtype == QMLA_KV_FP8) {
    const float inv = 1.0f / *p.k_scale;
    for (int c = 8 * lane; c < p.d_c; c += 512)
      *reinterpret_cast<uint2*>(dst + c) = quant8(kc + c, inv);
    for (int c = 8 * lane; c < p.rope_w; c += 512)
      *reinterpret_cast<uint2*>(dst + p.d_c + c) = quant8(kp + c, inv);
    char* rt = dst + p.d_c + p.rope_w;
    for (int h = lane; h < p.rms_heads; h += 64) {
      const uint16_t rb = kp[p.rope_w + h];
      if (p.rms_mode == QMLA_RMS_LOG8) {
        rt[h] = (char)log8_code(bf16_to_f32(rb));
      } else if (p.rms_mode == QMLA_RMS_BF16_BYTES) {
        rt[2 * h] = (char)(rb & 0xFF);
        rt[2 * h + 1] = (char)(rb >> 8);
      } else if (p.rms_mode == QMLA_RMS_E4M3) {
        rt[h] = (char)(pack_e4m3(sat448(bf16_to_f32(rb), inv), 0.f, 0.f, 0.f) & 0xFF);
      }
    }
  } else {
    uint16_t* d16 = reinterpret_cast<uint16_t*>(dst);
    for (int c = 8 * lane; c < p.d_c; c += 512)
      *reinterpret_cast<uint4*>(d16 + c) = *reinterpret_cast<const uint4*>(kc + c);
    const int pe = p.rope_w + (p.rms_mode == QMLA_RMS_BF16 ? p.rms_heads : 0);
    for (int c = lane; c < pe; c += 64) d16[p.d_c + c] = kp[c];
  }
}

}  // namespace wr
}  // namespace qmla

extern "C" int qmla_cache_write(const qmla_cache_write_params* p, void* stream) {
  using namespace qmla;
  if (!p) return QMLA_ERR_NULL;
  if (p->n == 0) return QMLA_OK;
  if (!p->kv_c || !p->k_pe || !p->slots || !p->cache) return QMLA_ERR_NULL;
  if (p->n < 0 || p->d_c <= 0 || p->d_c % 8 || p->rope_w < 0 || p->rms_heads < 0 || p->page_size <= 0 ||
      p->num_slots <= 0 || p->kv_c_stride < p->d_c)
    return QMLA_ERR_SHAPE;
  const bool fp8 = p->kv_dtype == QMLA_KV_FP8;
  if (!fp8 && p->kv_dtype != QMLA_KV_BF16) return QMLA_ERR_MODE;
  const int rb = fp8 ? (p->rms_mode == QMLA_RMS_BF16_BYTES ? 2 : (p->rms_mode == QMLA_RMS_NONE ? 0 : 1))
                     : (p->rms_mode == QMLA_RMS_BF16 ? 2 : 0);
  if (fp8 && p->rms_mode != QMLA_RMS_LOG8 && p->rms_mode != QMLA_RMS_BF16_BYTES && p->rms_mode != QMLA_RMS_E4M3 &&
      p->rms_mode != QMLA_RMS_NONE)
    return QMLA_ERR_MODE;
  if (!fp8 && p->rms_mode != QMLA_RMS_BF16 && p->rms_mode != QMLA_RMS_NONE) return QMLA_ERR_MODE;
  if (fp8 && (p->rope_w % 8 || !p->k_scale)) return fp8 && !p->k_scale ? QMLA_ERR_NULL : QMLA_ERR_SHAPE;
  const int pe_elems = p->rope_w + (rb ? p->rms_heads : 0);
  if (p->k_pe_stride < pe_elems) return QMLA_ERR_SHAPE;
  // the written bytes must fit one token slot
  const int64_t row_bytes = fp8 ? (int64_t)p->d_c + p->rope_w + (int64_t)rb * p->rms_heads
                                : 2 * ((int64_t)p->d_c + p->rope_w + (rb ? p->rms_heads : 0));
  if (row_bytes > p->token_stride || p->page_stride < p->token_stride * p->page_size) return QMLA_ERR_SHAPE;
  // 16-byte vector loads of kv_c and k_pe rows, 8- or 16-byte stores into the row
  if (((uintptr_t)p->kv_c | (uintptr_t)p->k_pe | (uintptr_t)p->cache) % 16 ||
      (p->kv_c_stride * 2) % 16 || (fp8 && (p->k_pe_stride * 2) % 16) || p->token_stride % 16 || p->page_stride % 16)
    return QMLA_ERR_ALIGN;
  wr::WParams k;
  k.kv_c = static_cast<const uint16_t*>(p->kv_c);
  k.kv_c_stride = p->kv_c_stride;
  k.k_pe = static_cast<const uint16_t*>(p->k_pe);
  k.k_pe_stride = p->k_pe_stride;
  k.slots = p->slots;
  k.n = p->n;
  k.d_c = p->d_c;
  k.rope_w = p->rope_w;
  k.rms_heads = p->rms_heads;
  k.kv_dtype = p->kv_dtype;
  k.rms_mode = p->rms_mode;
  k.k_scale = p->k_scale;
  k.cache = static_cast<char*>(p->cache);
  k.page_stride = p->page_stride;
  k.token_stride = p->token_stride;
  k.page_size = p->page_size;
  k.num_slots = p->num_slots;
  void* args[] = {&k};
  const unsigned grid = (unsigned)((p->n + wr::ROWS_PER_WG - 1) / wr::ROWS_PER_WG);
  const hipError_t e = hipLaunchKernel((const void*)wr::write_kernel, dim3(grid), dim3(64 * wr::ROWS_PER_WG), args,
                                       0, (hipStream_t)stream);
  return e == hipSuccess ? QMLA_OK : QMLA_ERR_LAUNCH;
}
