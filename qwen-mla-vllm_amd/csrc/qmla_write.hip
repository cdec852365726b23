// qmla_write.hip -- gfx950 cache-row kernels: the writer (one new token per input row into its paged
// cache slot) and the prefill context gather (paged rows back into a dense bf16 workspace).
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
// rows from which the writer and the gather take several rows a wave (measured on MI355X: at 16384
// rows one row a wave is as fast or faster, at 262144 several rows a wave 23% / 37% faster)
constexpr int kMultiRowMin = 65536;
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
__device__ __forceinline__ uint2 quant8r(const uint4 raw, float inv) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  float f[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = sat448(bf16_to_f32((uint16_t)(w[i] & 0xFFFF)), inv);
    f[2 * i + 1] = sat448(bf16_to_f32((uint16_t)(w[i] >> 16)), inv);
  }
  return make_uint2(pack_e4m3(f[0], f[1], f[2], f[3]), pack_e4m3(f[4], f[5], f[6], f[7]));
}
__device__ __forceinline__ uint2 quant8(const uint16_t* src, float inv) {
  return quant8r(*reinterpret_cast<const uint4*>(src), inv);
}

// log8 code of one rms value: round-half-even((log2(max(r, 1e-30)) + 3) * (255 / 6)), clamped to
// [0, 255]; the logarithm is evaluated in double and rounded once to fp32, the rest in fp32
__device__ __forceinline__ uint32_t log8_code(float r) {
  const float rc = r < 1e-30f ? 1e-30f : r;   // clamp_min keeps NaN
  const float lg = (float)log2((double)rc);
  const float c = rintf((lg - (-3.0f)) * 42.5f);
  return (uint32_t)(c < 0.0f ? 0.0f : (c > 255.0f ? 255.0f : c));
}
// The same code from the hardware log2 (within 2 ulp of the rounded double one): (lg + 3) * 42.5
// then moves by less than 2e-4 inside the code range, so wherever it lies 1e-3 or more from a
// rounding midpoint it rounds as the double path does; the few values nearer one take that path.
__device__ __forceinline__ uint32_t log8_code_fast(float r) {
  const float rc = r < 1e-30f ? 1e-30f : r;
  const float y = (__builtin_amdgcn_logf(rc) - (-3.0f)) * 42.5f;
  if (fabsf(y - floorf(y) - 0.5f) < 1e-3f) return log8_code(r);
  const float c = rintf(y);
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
    // the rope in 8-element groups, then the 1-7 elements before an rms tail that is not 8-aligned
    // one by one (the plugin's rope 116): a group must not spill into the tail other lanes write
    const int r8 = p.rope_w & ~7;
    for (int c = 8 * lane; c < r8; c += 512)
      *reinterpret_cast<uint2*>(dst + p.d_c + c) = quant8(kp + c, inv);
    if (lane < p.rope_w - r8) {
      const int c = r8 + lane;
      dst[p.d_c + c] = (char)(pack_e4m3(sat448(bf16_to_f32(kp[c]), inv), 0.f, 0.f, 0.f) & 0xFF);
    }
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

// FP8 rows with latents up to 512 * NCL columns, a rope up to 512 and up to 64 rms heads: one wave
// writes WROWS rows, all of their input loads in flight before the first conversion (a lone row's
// load latency would otherwise bound a wave), the same bytes as write_kernel.
constexpr int WROWS = 4;
template <int NCL>
__global__ __launch_bounds__(256) void write_fp8_kernel(const WParams p) {
  const int lane = threadIdx.x & 63;
  const int r0 = ((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6)) * WROWS;
  if (r0 >= p.n) return;
  const float inv = 1.0f / *p.k_scale;
  const int r8 = p.rope_w & ~7;
  uint4 lat[WROWS][NCL], rp[WROWS];
  uint16_t rt[WROWS], rm[WROWS];
  int64_t slot[WROWS];
#pragma unroll
  for (int i = 0; i < WROWS; ++i) {
    const int row = r0 + i < p.n ? r0 + i : p.n - 1;   // past the end: a valid row, not written
    const uint16_t* kc = p.kv_c + (int64_t)row * p.kv_c_stride;
    const uint16_t* kp = p.k_pe + (int64_t)row * p.k_pe_stride;
    slot[i] = p.slots[row];
#pragma unroll
    for (int k = 0; k < NCL; ++k) {
      const int c = 8 * lane + 512 * k;
      lat[i][k] = c < p.d_c ? *reinterpret_cast<const uint4*>(kc + c) : make_uint4(0u, 0u, 0u, 0u);
    }
    rp[i] = 8 * lane < r8 ? *reinterpret_cast<const uint4*>(kp + 8 * lane) : make_uint4(0u, 0u, 0u, 0u);
    rt[i] = lane < p.rope_w - r8 ? kp[r8 + lane] : (uint16_t)0;
    rm[i] = lane < p.rms_heads ? kp[p.rope_w + lane] : (uint16_t)0;
  }
#pragma unroll
  for (int i = 0; i < WROWS; ++i) {
    if (r0 + i >= p.n) break;
    int64_t sl = slot[i];
    if (sl < 0) sl = 0;
    if (sl >= p.num_slots) continue;
    const int64_t page = sl / p.page_size, tok = sl - page * p.page_size;
    char* dst = p.cache + page * p.page_stride + tok * p.token_stride;
#pragma unroll
    for (int k = 0; k < NCL; ++k) {
      const int c = 8 * lane + 512 * k;
      if (c < p.d_c) *reinterpret_cast<uint2*>(dst + c) = quant8r(lat[i][k], inv);
    }
    if (8 * lane < r8) *reinterpret_cast<uint2*>(dst + p.d_c + 8 * lane) = quant8r(rp[i], inv);
    if (lane < p.rope_w - r8)
      dst[p.d_c + r8 + lane] = (char)(pack_e4m3(sat448(bf16_to_f32(rt[i]), inv), 0.f, 0.f, 0.f) & 0xFF);
    if (lane < p.rms_heads) {
      char* rtl = dst + p.d_c + p.rope_w;
      if (p.rms_mode == QMLA_RMS_LOG8) {
        rtl[lane] = (char)log8_code_fast(bf16_to_f32(rm[i]));
      } else if (p.rms_mode == QMLA_RMS_BF16_BYTES) {
        rtl[2 * lane] = (char)(rm[i] & 0xFF);
        rtl[2 * lane + 1] = (char)(rm[i] >> 8);
      } else if (p.rms_mode == QMLA_RMS_E4M3) {
        rtl[lane] = (char)(pack_e4m3(sat448(bf16_to_f32(rm[i]), inv), 0.f, 0.f, 0.f) & 0xFF);
      }
    }
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
  if (fp8 && !p->k_scale) return QMLA_ERR_NULL;
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
  // large batches (a long prefill): WROWS rows a wave; smaller ones keep one row a wave, which
  // spreads them over more waves
  if (fp8 && p->n >= kMultiRowMin && p->d_c <= 1024 && p->rope_w <= 512 && p->rms_heads <= 64) {
    const unsigned grid = (unsigned)((p->n + 4 * wr::WROWS - 1) / (4 * wr::WROWS));
    const void* fn = p->d_c <= 512 ? (const void*)wr::write_fp8_kernel<1> : (const void*)wr::write_fp8_kernel<2>;
    const hipError_t e = hipLaunchKernel(fn, dim3(grid), dim3(256), args, 0, (hipStream_t)stream);
    return e == hipSuccess ? QMLA_OK : QMLA_ERR_LAUNCH;
  }
  const unsigned grid = (unsigned)((p->n + wr::ROWS_PER_WG - 1) / wr::ROWS_PER_WG);
  const hipError_t e = hipLaunchKernel((const void*)wr::write_kernel, dim3(grid), dim3(64 * wr::ROWS_PER_WG), args,
                                       0, (hipStream_t)stream);
  return e == hipSuccess ? QMLA_OK : QMLA_ERR_LAUNCH;
}

// ---- prefill context gather (qwen_mla/ops/mla_gather.py:28-76) -----------------------------------
// One wave per destination row: the row's sequence, token and page from the chunk metadata, then the
// cached row copied (bf16 caches) or dequantized into the destination dtype (FP8 caches).
namespace qmla {
namespace ga {

constexpr int ROWS_PER_WG = 4;

struct GParams {
  const char* cache;
  int64_t page_stride, token_stride;
  int page_size, num_pages, kv_dtype, rms_mode, rms_offset, rms_heads, row_elems;
  const float* scale;
  const int32_t* block_table;
  int64_t bt_stride;
  int num_seqs, bt_cols;
  const int32_t* cu_seq_lens;
  const int32_t* token_to_seq;
  const int32_t* seq_starts;
  int num_tokens;
  char* dst;
  int64_t dst_stride;
  int dst_dtype;
};

// one e4m3 byte (byte k of w) -> fp32; the conversion returns +0 for the negative zero 0x80, so the
// sign bit is put back (torch decodes 0x80 as -0.0, which survives the scale and the rounding)
__device__ __forceinline__ float e4m3_f32(int w, int k) {
  float f;
  switch (k) {
    case 0: f = __builtin_amdgcn_cvt_f32_fp8(w, 0); break;
    case 1: f = __builtin_amdgcn_cvt_f32_fp8(w, 1); break;
    case 2: f = __builtin_amdgcn_cvt_f32_fp8(w, 2); break;
    default: f = __builtin_amdgcn_cvt_f32_fp8(w, 3); break;
  }
  return __uint_as_float(__float_as_uint(f) | (((uint32_t)w >> (8 * k + 7)) & 1u) << 31);
}

// fp32 -> the destination dtype, round to nearest even; the sign bit is carried over explicitly so a
// negative zero stays negative whatever instruction the conversion compiles to
__device__ __forceinline__ uint16_t to_out(float x, int dt) {
  const uint16_t sign = (uint16_t)((__float_as_uint(x) >> 16) & 0x8000u);
  if (dt == QMLA_DT_F16) return (uint16_t)(__builtin_bit_cast(uint16_t, (_Float16)x) | sign);
  return (uint16_t)(__builtin_bit_cast(uint16_t, (__bf16)x) | sign);
}

__global__ __launch_bounds__(64 * ROWS_PER_WG) void gather_kernel(const GParams p) {
  const int lane = threadIdx.x & 63;
  const int j = (int)blockIdx.x * ROWS_PER_WG + (int)(threadIdx.x >> 6);
  if (j >= p.num_tokens) return;
  const int s = p.token_to_seq[j];
  if (s < 0 || s >= p.num_seqs) return;
  int64_t tok = (int64_t)j - p.cu_seq_lens[s];
  if (p.seq_starts) tok += p.seq_starts[s];
  if (tok < 0) return;
  const int64_t pi = tok / p.page_size;
  if (pi >= p.bt_cols) return;
  const int blk = p.block_table[(int64_t)s * p.bt_stride + pi];
  if (blk < 0 || blk >= p.num_pages) return;
  const char* row = p.cache + (int64_t)blk * p.page_stride + (tok - pi * p.page_size) * p.token_stride;
  uint16_t* out = reinterpret_cast<uint16_t*>(p.dst) + (int64_t)j * p.dst_stride;

  if (p.kv_dtype == QMLA_KV_BF16) {
    const uint16_t* src = reinterpret_cast<const uint16_t*>(row);
    if (p.dst_dtype == QMLA_DT_BF16) {
      const int nv = p.row_elems / 8;
      for (int c = lane; c < nv; c += 64)
        reinterpret_cast<uint4*>(out)[c] = reinterpret_cast<const uint4*>(src)[c];
      for (int c = 8 * nv + lane; c < p.row_elems; c += 64) out[c] = src[c];
    } else {
      for (int c = lane; c < p.row_elems; c += 64) out[c] = to_out(__uint_as_float((uint32_t)src[c] << 16), p.dst_dtype);
    }
    return;
  }
  const float sc = *p.scale;
  // latent + rope: e4m3 * scale in fp32, rounded to the destination dtype; whole 8-byte groups as
  // vectors, the 1-7 bytes before an rms tail that is not 8-aligned one by one (the plugin's 12-head
  // rope-116 rows put the tail at 4 mod 8)
  const int c8 = p.rms_offset & ~7;
  for (int c = 8 * lane; c < c8; c += 512) {
    const uint2 raw = *reinterpret_cast<const uint2*>(row + c);
    const uint32_t w[2] = {raw.x, raw.y};
    uint32_t o[4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int wv = (int)w[h];
      const float f0 = e4m3_f32(wv, 0) * sc, f1 = e4m3_f32(wv, 1) * sc;
      const float f2 = e4m3_f32(wv, 2) * sc, f3 = e4m3_f32(wv, 3) * sc;
      o[2 * h] = (uint32_t)to_out(f0, p.dst_dtype) | ((uint32_t)to_out(f1, p.dst_dtype) << 16);
      o[2 * h + 1] = (uint32_t)to_out(f2, p.dst_dtype) | ((uint32_t)to_out(f3, p.dst_dtype) << 16);
    }
    *reinterpret_cast<uint4*>(out + c) = make_uint4(o[0], o[1], o[2], o[3]);
  }
  if (lane < p.rms_offset - c8) {
    const int c = c8 + lane;
    out[c] = to_out(e4m3_f32((int)(unsigned char)row[c], 0) * sc, p.dst_dtype);
  }
  // the rms tail: one element per head at rms_offset
  const unsigned char* tail = reinterpret_cast<const unsigned char*>(row) + p.rms_offset;
  for (int h = lane; h < p.rms_heads; h += 64) {
    float v;
    if (p.rms_mode == QMLA_RMS_LOG8) {
      v = (float)exp2(-3.0 + (double)tail[h] * (6.0 / 255.0));   // 2^(-3 + code*6/255)
    } else if (p.rms_mode == QMLA_RMS_BF16_BYTES) {
      const uint32_t bits = (uint32_t)tail[2 * h] | ((uint32_t)tail[2 * h + 1] << 8);
      if (p.dst_dtype == QMLA_DT_BF16) {
        out[p.rms_offset + h] = (uint16_t)bits;
        continue;
      }
      v = __uint_as_float(bits << 16);
    } else {
      v = e4m3_f32((int)tail[h], 0) * sc;
    }
    out[p.rms_offset + h] = to_out(v, p.dst_dtype);
  }
}

// FP8 rows whose latent + rope span at most 1024 bytes and whose rms tail holds at most 64 heads:
// one wave gathers GROWS destination rows. Lanes 0 .. GROWS-1 resolve the rows' sequence, token and
// page together (the per-row kernel waits for that chain of dependent loads once per row). The
// rows' 8-byte chunks are then dealt out flat, chunk q of the wave to lane q % 64, so every issued
// conversion is a full one (a row of 72 chunks would leave 56 lanes idle in its second pass), and
// all their loads are in flight before the first conversion; likewise the rms elements. The same
// values as gather_kernel.
constexpr int GROWS = 8;
template <int DT>
__global__ __launch_bounds__(256) void gather_fp8_kernel(const GParams p) {
  constexpr int NQ = GROWS * 128 / 64;   // chunk passes at most (1024-byte rows)
  constexpr int NT = GROWS * 64 / 64;    // rms passes at most (64 heads)
  const int lane = threadIdx.x & 63;
  const int j0 = ((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6)) * GROWS;
  // the 256 log8 divisors, 2^(-3 + code*6/255) rounded once from double, one per thread (every
  // thread of the workgroup takes part, before any leaves)
  __shared__ float l8[256];
  if (p.rms_mode == QMLA_RMS_LOG8) {
    l8[threadIdx.x] = (float)exp2(-3.0 + (double)threadIdx.x * (6.0 / 255.0));
    __syncthreads();
  }
  if (j0 >= p.num_tokens) return;
  // lane r < GROWS: byte offset of row j0 + r in the cache, or -1 (nothing to write)
  int64_t roff = -1;
  if (lane < GROWS && j0 + lane < p.num_tokens) {
    const int j = j0 + lane;
    const int s = p.token_to_seq[j];
    if (s >= 0 && s < p.num_seqs) {
      int64_t tok = (int64_t)j - p.cu_seq_lens[s];
      if (p.seq_starts) tok += p.seq_starts[s];
      if (tok >= 0) {
        const int64_t pi = tok / p.page_size;
        if (pi < p.bt_cols) {
          const int blk = p.block_table[(int64_t)s * p.bt_stride + pi];
          if (blk >= 0 && blk < p.num_pages)
            roff = (int64_t)blk * p.page_stride + (tok - pi * p.page_size) * p.token_stride;
        }
      }
    }
  }
  const int roff_lo = (int)(uint32_t)roff, roff_hi = (int)(uint32_t)((uint64_t)roff >> 32);
  const int c8 = p.rms_offset & ~7, nch = c8 >> 3, npre = p.rms_offset - c8;
  const int rb = p.rms_mode == QMLA_RMS_BF16_BYTES ? 2 : 1;
  const int nel = nch + (npre > 0 ? 1 : 0);            // chunk slots a row: whole chunks + the pre-tail
  const int total = GROWS * nel, nt = GROWS * p.rms_heads;
  // q / nel and t / rms_heads from 24-bit multiplies (q, t < 2^11; exact below 2^20 / divisor)
  const uint32_t mq = ((1u << 20) + nel - 1) / nel, mt = p.rms_heads > 0 ? ((1u << 20) + p.rms_heads - 1) / p.rms_heads : 0u;
  uint2 raw[NQ];
  uint32_t tb[NT];
  uint32_t live = 0u;   // bit i: this lane's chunk slot of pass i belongs to a row to write
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    raw[i] = make_uint2(0u, 0u);
    if (64 * i < total) {   // wave-uniform
      const int q = lane + 64 * i;
      const int r = (int)(__umul24((uint32_t)(q < total ? q : 0), mq) >> 20);
      const uint32_t lo = (uint32_t)__shfl(roff_lo, r), hi = (uint32_t)__shfl(roff_hi, r);
      const int64_t ro = (int64_t)(((uint64_t)hi << 32) | lo);
      if (q < total && ro >= 0) {
        live |= 1u << i;
        const int c = q - (int)__umul24((uint32_t)r, (uint32_t)nel);
        if (c < nch) raw[i] = *reinterpret_cast<const uint2*>(p.cache + ro + 8 * c);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    tb[i] = 0u;
    if (64 * i < nt) {
      const int t = lane + 64 * i;
      const int r = (int)(__umul24((uint32_t)(t < nt ? t : 0), mt) >> 20);
      const uint32_t lo = (uint32_t)__shfl(roff_lo, r), hi = (uint32_t)__shfl(roff_hi, r);
      const int64_t ro = (int64_t)(((uint64_t)hi << 32) | lo);
      if (t < nt && ro >= 0) {
        const int h = t - (int)__umul24((uint32_t)r, (uint32_t)p.rms_heads);
        const unsigned char* tail = reinterpret_cast<const unsigned char*>(p.cache + ro) + p.rms_offset;
        tb[i] = rb == 2 ? ((uint32_t)tail[2 * h] | ((uint32_t)tail[2 * h + 1] << 8)) : (uint32_t)tail[h];
      }
    }
  }
  const float sc = *p.scale;
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    if (64 * i >= total) break;
    const int q = lane + 64 * i;
    if (!(live & (1u << i))) continue;
    const int r = (int)(__umul24((uint32_t)q, mq) >> 20);
    const int c = q - (int)__umul24((uint32_t)r, (uint32_t)nel);
    uint16_t* out = reinterpret_cast<uint16_t*>(p.dst) + (int64_t)(j0 + r) * p.dst_stride;
    if (c < nch) {
      const uint32_t w[2] = {raw[i].x, raw[i].y};
      uint32_t o[4];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int wv = (int)w[h];
        const float f0 = e4m3_f32(wv, 0) * sc, f1 = e4m3_f32(wv, 1) * sc;
        const float f2 = e4m3_f32(wv, 2) * sc, f3 = e4m3_f32(wv, 3) * sc;
        o[2 * h] = (uint32_t)to_out(f0, DT) | ((uint32_t)to_out(f1, DT) << 16);
        o[2 * h + 1] = (uint32_t)to_out(f2, DT) | ((uint32_t)to_out(f3, DT) << 16);
      }
      *reinterpret_cast<uint4*>(out + 8 * c) = make_uint4(o[0], o[1], o[2], o[3]);
    } else {
      // the 1-7 bytes between the last whole chunk and the rms tail (the plugin's rope-116 rows)
      const uint32_t lo = (uint32_t)__shfl(roff_lo, r), hi = (uint32_t)__shfl(roff_hi, r);
      const unsigned char* row = reinterpret_cast<const unsigned char*>(p.cache + (int64_t)(((uint64_t)hi << 32) | lo));
      for (int e = 0; e < npre; ++e) out[c8 + e] = to_out(e4m3_f32((int)row[c8 + e], 0) * sc, DT);
    }
  }
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    if (64 * i >= nt) break;
    const int t = lane + 64 * i;
    const int r = (int)(__umul24((uint32_t)(t < nt ? t : 0), mt) >> 20);
    const uint32_t lo = (uint32_t)__shfl(roff_lo, r), hi = (uint32_t)__shfl(roff_hi, r);
    const int64_t ro = (int64_t)(((uint64_t)hi << 32) | lo);
    if (t >= nt || ro < 0) continue;
    const int h = t - (int)__umul24((uint32_t)r, (uint32_t)p.rms_heads);
    uint16_t* out = reinterpret_cast<uint16_t*>(p.dst) + (int64_t)(j0 + r) * p.dst_stride + p.rms_offset;
    float v;
    if (p.rms_mode == QMLA_RMS_LOG8) {
      v = l8[tb[i]];
    } else if (p.rms_mode == QMLA_RMS_BF16_BYTES) {
      if (DT == QMLA_DT_BF16) {
        out[h] = (uint16_t)tb[i];
        continue;
      }
      v = __uint_as_float(tb[i] << 16);
    } else {
      v = e4m3_f32((int)tb[i], 0) * sc;
    }
    out[h] = to_out(v, DT);
  }
}

}  // namespace ga
}  // namespace qmla

extern "C" int qmla_gather(const qmla_gather_params* p, void* stream) {
  using namespace qmla;
  if (!p) return QMLA_ERR_NULL;
  if (p->num_tokens == 0) return QMLA_OK;
  if (!p->cache || !p->block_table || !p->cu_seq_lens || !p->token_to_seq || !p->dst) return QMLA_ERR_NULL;
  if (p->num_tokens < 0 || p->page_size <= 0 || p->num_pages <= 0 || p->num_seqs <= 0 || p->bt_cols <= 0 ||
      p->bt_stride < p->bt_cols)
    return QMLA_ERR_SHAPE;
  if (p->dst_dtype != QMLA_DT_BF16 && p->dst_dtype != QMLA_DT_F16) return QMLA_ERR_MODE;
  const bool fp8 = p->kv_dtype == QMLA_KV_FP8;
  if (!fp8 && p->kv_dtype != QMLA_KV_BF16) return QMLA_ERR_MODE;
  int64_t width;
  if (fp8) {
    if (p->rms_mode != QMLA_RMS_LOG8 && p->rms_mode != QMLA_RMS_BF16_BYTES && p->rms_mode != QMLA_RMS_E4M3)
      return QMLA_ERR_MODE;
    if (!p->scale) return QMLA_ERR_NULL;
    if (p->rms_offset <= 0 || p->rms_heads < 0) return QMLA_ERR_SHAPE;
    const int64_t rb = p->rms_mode == QMLA_RMS_BF16_BYTES ? 2 : 1;
    if (p->rms_offset + rb * p->rms_heads > p->token_stride) return QMLA_ERR_SHAPE;
    width = (int64_t)p->rms_offset + p->rms_heads;
  } else {
    if (p->row_elems <= 0 || 2 * (int64_t)p->row_elems > p->token_stride) return QMLA_ERR_SHAPE;
    width = p->row_elems;
  }
  if (p->dst_stride < width || p->page_stride < p->token_stride * p->page_size) return QMLA_ERR_SHAPE;
  if (((uintptr_t)p->cache | (uintptr_t)p->dst) % 16 || p->token_stride % 16 || p->page_stride % 16 ||
      (p->dst_stride * 2) % 16)
    return QMLA_ERR_ALIGN;
  ga::GParams k;
  k.cache = static_cast<const char*>(p->cache);
  k.page_stride = p->page_stride;
  k.token_stride = p->token_stride;
  k.page_size = p->page_size;
  k.num_pages = p->num_pages;
  k.kv_dtype = p->kv_dtype;
  k.rms_mode = p->rms_mode;
  k.rms_offset = p->rms_offset;
  k.rms_heads = p->rms_heads;
  k.row_elems = p->row_elems;
  k.scale = p->scale;
  k.block_table = p->block_table;
  k.bt_stride = p->bt_stride;
  k.num_seqs = p->num_seqs;
  k.bt_cols = p->bt_cols;
  k.cu_seq_lens = p->cu_seq_lens;
  k.token_to_seq = p->token_to_seq;
  k.seq_starts = p->seq_starts;
  k.num_tokens = p->num_tokens;
  k.dst = static_cast<char*>(p->dst);
  k.dst_stride = p->dst_stride;
  k.dst_dtype = p->dst_dtype;
  void* args[] = {&k};
  if (fp8 && p->num_tokens >= kMultiRowMin && p->rms_offset <= 1024 && p->rms_heads <= 64) {
    const unsigned grid = (unsigned)((p->num_tokens + 4 * ga::GROWS - 1) / (4 * ga::GROWS));
    const void* fn = p->dst_dtype == QMLA_DT_F16 ? (const void*)ga::gather_fp8_kernel<QMLA_DT_F16>
                                                 : (const void*)ga::gather_fp8_kernel<QMLA_DT_BF16>;
    const hipError_t e = hipLaunchKernel(fn, dim3(grid), dim3(256), args, 0, (hipStream_t)stream);
    return e == hipSuccess ? QMLA_OK : QMLA_ERR_LAUNCH;
  }
  const unsigned grid = (unsigned)((p->num_tokens + ga::ROWS_PER_WG - 1) / ga::ROWS_PER_WG);
  const hipError_t e = hipLaunchKernel((const void*)ga::gather_kernel, dim3(grid), dim3(64 * ga::ROWS_PER_WG), args,
                                       0, (hipStream_t)stream);
  return e == hipSuccess ? QMLA_OK : QMLA_ERR_LAUNCH;
}
