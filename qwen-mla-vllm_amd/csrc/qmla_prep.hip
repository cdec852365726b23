// qmla_prep.hip -- gfx950 decode q / k_pe prep: the per-token work between the attention module's
// projections and the attention call, in one launch.
//
// Reference: qwen_mla/qwen3_5_mla.py:262-301 (rms from the raw up-projection and the raw rope key,
// one neox rotation of q and the rope keys, q_pe scattered into the head's group slot, k_pe =
// [rope window | rms | pad]), the rotation arithmetic of :341-354 (cos/sin rows rounded to the
// query dtype, x1*cos - x2*sin | x2*cos + x1*sin in bf16), the rope table of
// qwen_mla/partial_rope.py:52-76 (an input here).
//
// One launch, two kinds of 512-thread blocks, so the work spreads over every CU:
// * rms blocks, 16 tokens x one head: k_nope = latent . k_up^T for the head (16 x nope x d_c, bf16
//   MFMA 16x16x32 with fp32 accumulation); wave w takes K quarter (w % 4) and column half (w / 4)
//   with its first two 64-wide k blocks in flight at once; the quarters meet in LDS, the sums are
//   rounded to bf16 (the GEMM's output dtype in the reference), squared and summed per token, and
//   the raw rope key's squares are added. Blocks are mapped so a head's token tiles share an XCD.
// * row blocks, one wave per output row: a q_out row (token, head) gets its rotated rope part from
//   one lane per element (through LDS) and is written 8 elements per lane (16-byte stores where
//   aligned); a k_pe rope window (token, cached group) is rotated one element per lane, and the
//   group-0 wave also writes the row's padding.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qmla.h"
#include "qmla_device.h"

namespace qmla {
namespace prep {

constexpr int TM = 16;          // tokens per rms block
constexpr int NTHREADS = 512;   // 8 waves: 4 K quarters x 2 column halves of the up-projection GEMM
constexpr int KSPLIT = 4;
constexpr int RPARTS = 8;       // lanes per token summing the rope key's squares (128 lanes, 16 tokens)
constexpr int MAX_RD = 256;
#define RED_BYTES(nth) ((KSPLIT - 1) * 2 * (nth) * 64 * 16)
// LDS of a block: the rms blocks' partials and sums, or the row blocks' rotated parts (8 * MAX_RD * 2)
#define LDS_BYTES(nth) (RED_BYTES(nth) + 3 * TM * 4 > 8 * MAX_RD * 2 ? RED_BYTES(nth) + 3 * TM * 4 : 8 * MAX_RD * 2)

struct PParams {
  const uint16_t* q;
  int64_t q_ts, q_hs;
  const uint16_t* latent;
  int64_t lat_s;
  const uint16_t* k_rope;
  int64_t kr_s;
  const uint16_t* k_up;
  const float* k_gain;
  const void* cos_sin;
  int cs_dtype;
  int64_t max_pos;
  const int64_t* positions;
  int64_t pos_rs;
  int pos_rows;
  const int32_t* rope_sec;
  int n, heads, head_dim, rd, kv_heads, d_c;
  int head_offset, rope_group, rope_first, rope_span, declared_rope;
  float eps;
  uint16_t* q_out;
  int64_t qo_ts, qo_hs;
  uint16_t* k_pe;
  int64_t kp_s;
  int vec_in, vec_out;     // q / q_out rows and strides 16-byte aligned: 16-byte loads / stores
  int tiles, xcd_map;      // token tiles of the rms blocks; heads % 8 == 0: a head's tiles share one XCD
  int rms_blocks, row_blocks;
};

// fp32 -> bf16 bits, round to nearest even, sign carried explicitly (negative zero stays negative)
__device__ __forceinline__ uint16_t bf16r(float x) {
  const uint16_t sign = (uint16_t)((__float_as_uint(x) >> 16) & 0x8000u);
  return (uint16_t)(__builtin_bit_cast(uint16_t, (__bf16)x) | sign);
}
__device__ __forceinline__ float f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// the cos or sin entry i of the table, rounded to bf16 as the rotation uses it
__device__ __forceinline__ float table(const PParams& p, int64_t i) {
  if (p.cs_dtype == QMLA_DT_BF16) return f32(static_cast<const uint16_t*>(p.cos_sin)[i]);
  if (p.cs_dtype == QMLA_DT_F32) return f32(bf16r(static_cast<const float*>(p.cos_sin)[i]));
  return f32(bf16r((float)__builtin_bit_cast(_Float16, static_cast<const uint16_t*>(p.cos_sin)[i])));
}

// The two 8-element MFMA fragments of a 64-wide k block for lane group q = lane / 16: k = 8q..8q+7
// (first MFMA) and 32+8q..32+8q+7 (second), so each load instruction reads 64 contiguous bytes of
// every row it touches. ptr = the block's first element of the lane's row (16-byte aligned, always
// a valid address); zeroed when !ok. The loads are unconditional and the zeroing is a select, so no
// branch (and no wait) separates them from the loads issued next to them.
__device__ __forceinline__ void load16(const uint16_t* ptr, int q, bool ok, bf16x8& lo, bf16x8& hi) {
  uint4 a = *reinterpret_cast<const uint4*>(ptr + 8 * q);
  uint4 b = *reinterpret_cast<const uint4*>(ptr + 32 + 8 * q);
  const uint32_t m = ok ? 0xffffffffu : 0u;
  a.x &= m; a.y &= m; a.z &= m; a.w &= m;
  b.x &= m; b.y &= m; b.z &= m; b.w &= m;
  lo = __builtin_bit_cast(bf16x8, a);
  hi = __builtin_bit_cast(bf16x8, b);
}

// ---- role 1: the rms of 16 tokens x one head ---------------------------------------------------
template <int NT>   // 16-column tiles covering nope
__device__ __forceinline__ void rms_block(const PParams& p, int b, char* lds) {
  constexpr int NTH = (NT + 1) / 2;                                  // tiles per column half
  auto red = reinterpret_cast<f32x4(*)[2][NTH][64]>(lds);            // K quarters 1..3: [column half][tile][lane]
  float* ssum = reinterpret_cast<float*>(lds + RED_BYTES(NTH));      // [2][TM]
  float* rsq = ssum + 2 * TM;                                        // [TM]

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int kq = w & (KSPLIT - 1), ch = w / KSPLIT;
  // block -> (token tile, head). Blocks are dealt to the 8 XCDs round robin; with heads % 8 == 0 the
  // token tiles of one head all land on one XCD, so its up-projection rows are read into one L2.
  int tile, h;
  if (p.xcd_map) {
    const int s = b >> 3;
    tile = s % p.tiles;
    h = (s / p.tiles) * 8 + (b & 7);
  } else {
    tile = b % p.tiles;
    h = b / p.tiles;
  }
  const int t0 = tile * TM;
  const int tn = min(TM, p.n - t0);
  const int rd = p.rd, nope = p.head_dim - rd;
  const int g = (p.head_offset + h) / p.rope_group;

  // the up-projection GEMM operands of this wave's K quarter, the first two 64-wide k blocks in
  // flight at once
  const int klen = p.d_c / KSPLIT, nblk = klen >> 6, kb = kq * klen, lq = lane >> 4;
  const int t = t0 + (lane & 15);
  const bool aok = t < p.n;
  const uint16_t* ap = p.latent + (int64_t)(aok ? t : 0) * p.lat_s + kb;
  const uint16_t* bp[NTH];
  bool bok[NTH];
#pragma unroll
  for (int j = 0; j < NTH; ++j) {
    const int tl = ch * NTH + j;
    const int col = 16 * tl + (lane & 15);
    bok[j] = tl < NT && col < nope;
    bp[j] = p.k_up + ((int64_t)h * nope + (bok[j] ? col : 0)) * p.d_c + kb;
  }
  bf16x8 a[2][2], bb[2][NTH][2];                                     // [k block][..][fragment]
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const bool ok = s < nblk;
    const int off = ok ? 64 * s : 0;                                 // stays inside the row
    load16(ap + off, lq, aok && ok, a[s][0], a[s][1]);
#pragma unroll
    for (int j = 0; j < NTH; ++j) load16(bp[j] + off, lq, bok[j] && ok, bb[s][j][0], bb[s][j][1]);
  }
  // the raw rope key of the head's group, for its sum of squares (waves of K quarter 1)
  float rv = 0.f;
  const int ridx = ch * 64 + lane, rt = ridx / RPARTS, rpart = ridx % RPARTS;
  if (kq == 1) {
    // RU unconditional loads in flight at once (rope dims up to RU * RPARTS; addresses clamped into
    // the row, values past it dropped by a select), a plain loop beyond
    const uint16_t* kr = p.k_rope + (int64_t)(t0 + min(rt, tn - 1)) * p.kr_s + (int64_t)g * rd;
    constexpr int RU = 8;
    uint16_t x[RU];
#pragma unroll
    for (int u = 0; u < RU; ++u) x[u] = kr[min(rpart + RPARTS * u, rd - 1)];
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const float v = (rt < tn && rpart + RPARTS * u < rd) ? f32(x[u]) : 0.f;
      rv += v * v;
    }
    if (rt < tn)
      for (int i = rpart + RPARTS * RU; i < rd; i += RPARTS) {
        const float v = f32(kr[i]);
        rv += v * v;
      }
  }
  f32x4 acc[NTH];
#pragma unroll
  for (int j = 0; j < NTH; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
      for (int j = 0; j < NTH; ++j) acc[j] = mfma16(a[s][f], bb[s][j][f], acc[j]);
  for (int blk = 2; blk < nblk; ++blk) {
    bf16x8 an[2], bn[NTH][2];
    load16(ap + 64 * blk, lq, aok, an[0], an[1]);
#pragma unroll
    for (int j = 0; j < NTH; ++j) load16(bp[j] + 64 * blk, lq, bok[j], bn[j][0], bn[j][1]);
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
      for (int j = 0; j < NTH; ++j) acc[j] = mfma16(an[f], bn[j][f], acc[j]);
  }
  if (kq > 0) {
#pragma unroll
    for (int j = 0; j < NTH; ++j) red[kq - 1][ch][j][lane] = acc[j];
  }
  if (kq == 1) {
#pragma unroll
    for (int o = 1; o < RPARTS; o <<= 1) rv += __shfl_xor(rv, o);
    if (rpart == 0 && rt < TM) rsq[rt] = rv;
  }
  __syncthreads();
  if (kq == 0) {
    // the K quarters meet; bf16(k_nope)^2 summed per token
    float sq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NTH; ++j) {
      const f32x4 o1 = red[0][ch][j][lane], o2 = red[1][ch][j][lane], o3 = red[2][ch][j][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = f32(bf16r(((acc[j][i] + o1[i]) + o2[i]) + o3[i]));   // columns past nope are 0
        sq[i] += v * v;
      }
    }
    // D[row][col] sits in lane col + 16*(row/4), element row%4: sum over the 16 column lanes
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = sq[i];
      v += __shfl_xor(v, 1);
      v += __shfl_xor(v, 2);
      v += __shfl_xor(v, 4);
      v += __shfl_xor(v, 8);
      if ((lane & 15) == 0) ssum[ch * TM + 4 * (lane >> 4) + i] = v;
    }
  }
  __syncthreads();
  if ((int)threadIdx.x < tn) {
    const int tt = threadIdx.x;
    const float total = ssum[tt] + ssum[TM + tt] + rsq[tt];
    const float rms = sqrtf(total / (float)p.head_dim + p.eps);
    p.k_pe[(int64_t)(t0 + tt) * p.kp_s + p.rope_span * rd + h] = bf16r(rms);
  }
}

// the cos | sin pair of frequency i for token t (bf16-rounded; NaN outside the table). The loads
// are unconditional (a position outside the table reads row 0) and the NaN a select.
__device__ __forceinline__ void cos_sin(const PParams& p, int t, int i, float& c, float& s) {
  const int row = p.pos_rows == 3 ? min(max(p.rope_sec[i], 0), 2) : 0;   // rows 0..2 only
  const int64_t pos = p.positions[(int64_t)row * p.pos_rs + t];
  const bool ok = pos >= 0 && pos < p.max_pos;
  const int64_t base = (ok ? pos : 0) * p.rd;
  const float c0 = table(p, base + i), s0 = table(p, base + (p.rd >> 1) + i);
  c = ok ? c0 : __builtin_nanf("");
  s = ok ? s0 : __builtin_nanf("");
}

// ---- role 2: one wave per q_out row (token, head) or per k_pe rope window (token, cached group) --
__device__ __forceinline__ void row_block(const PParams& p, int b, char* lds) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  uint16_t* rot = reinterpret_cast<uint16_t*>(lds) + w * MAX_RD;     // this wave's rotated rope part
  const int rd = p.rd, half = rd >> 1, hd = p.head_dim, nope = hd - rd;
  const int64_t task = (int64_t)b * (NTHREADS / 64) + w;
  const int64_t nq = (int64_t)p.n * p.heads;
  int t = -1, h = 0, gi = 0;
  bool qrow = false;
  if (task < nq) {
    t = (int)(task / p.heads);
    h = (int)(task - (int64_t)t * p.heads);
    qrow = true;
  } else if (task < nq + (int64_t)p.n * p.rope_span) {
    const int64_t k = task - nq;
    t = (int)(k / p.rope_span);
    gi = (int)(k - (int64_t)t * p.rope_span);
  }
  const uint16_t* qr = p.q + (int64_t)(t < 0 ? 0 : t) * p.q_ts + (int64_t)h * p.q_hs;
  // rotated rope elements, one per lane. The source row is q's rope part or the cached group's raw
  // rope key (times its gain; bf16(x * 1) == x for the query), so both kinds load the same way.
  if (t >= 0) {
    const uint16_t* src = qrow ? qr : p.k_rope + (int64_t)t * p.kr_s + (int64_t)(p.rope_first + gi) * rd;
    for (int r = lane; r < rd; r += 64) {
      const int i = r < half ? r : r - half;
      float c, s;
      cos_sin(p, t, i, c, s);
      const float g1 = p.k_gain[i], g2 = p.k_gain[half + i];
      const float x1 = f32(bf16r(f32(src[i]) * (qrow ? 1.f : g1)));
      const float x2 = f32(bf16r(f32(src[half + i]) * (qrow ? 1.f : g2)));
      const uint16_t v = r < half ? bf16r(f32(bf16r(x1 * c)) - f32(bf16r(x2 * s)))
                                  : bf16r(f32(bf16r(x2 * c)) + f32(bf16r(x1 * s)));
      if (qrow) rot[r] = v;
      else p.k_pe[(int64_t)t * p.kp_s + gi * rd + r] = v;
    }
    if (!qrow && gi == 0) {
      // the padding after the rms elements
      const int packed = p.rope_span * rd, pad0 = packed + p.heads;
      for (int e = pad0 + lane; e < p.declared_rope; e += 64) p.k_pe[(int64_t)t * p.kp_s + e] = 0;
    }
  }
  __syncthreads();
  if (!qrow) return;
  // q_out[t, h] = [ q[t, h, rd:] | q_pe zero but the group's slot ], 8 elements per lane
  const int g = (p.head_offset + h) / p.rope_group;
  const int slot = nope + (g - p.rope_first) * rd;          // first q_pe element of the slot
  const int width = nope + p.declared_rope;
  const int nch = (width + 7) >> 3;
  uint16_t* orow = p.q_out + (int64_t)t * p.qo_ts + (int64_t)h * p.qo_hs;
  for (int c = lane; c < nch; c += 64) {
    const int k = 8 * c;
    uint32_t o[4];
    if (k + 8 <= nope) {
      if (p.vec_in) {
        const uint4 v = *reinterpret_cast<const uint4*>(qr + rd + k);
        o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) o[u] = *reinterpret_cast<const uint32_t*>(qr + rd + k + 2 * u);
      }
    } else if (k >= nope && (k + 8 <= slot || k >= slot + rd)) {
      o[0] = o[1] = o[2] = o[3] = 0u;
    } else {
      uint16_t e[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int kk = k + u;
        e[u] = kk < nope ? qr[rd + kk] : ((kk >= slot && kk < slot + rd) ? rot[kk - slot] : (uint16_t)0);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) o[u] = (uint32_t)e[2 * u] | ((uint32_t)e[2 * u + 1] << 16);
    }
    if (p.vec_out) {
      *reinterpret_cast<uint4*>(orow + k) = make_uint4(o[0], o[1], o[2], o[3]);
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (k + 2 * u < width) *reinterpret_cast<uint32_t*>(orow + k + 2 * u) = o[u];
    }
  }
}

template <int NT>
__global__ __launch_bounds__(NTHREADS) void prep_kernel(const PParams p) {
  __shared__ __attribute__((aligned(16))) char lds[LDS_BYTES((NT + 1) / 2)];
  const int b = blockIdx.x;
  if (b < p.rms_blocks) rms_block<NT>(p, b, lds);
  else row_block(p, b - p.rms_blocks, lds);
}

template <int NT>
hipError_t launch(const PParams& k, hipStream_t stream) {
  void* args[] = {const_cast<PParams*>(&k)};
  return hipLaunchKernel((const void*)prep_kernel<NT>, dim3((unsigned)(k.rms_blocks + k.row_blocks)),
                         dim3(NTHREADS), args, 0, stream);
}

}  // namespace prep
}  // namespace qmla

extern "C" int qmla_prep(const qmla_prep_params* p, void* stream) {
  using namespace qmla;
  if (!p) return QMLA_ERR_NULL;
  if (p->n < 0) return QMLA_ERR_SHAPE;
  if (p->n == 0) return QMLA_OK;
  if (!p->q || !p->latent || !p->k_rope || !p->k_up || !p->k_gain || !p->cos_sin || !p->positions ||
      !p->q_out || !p->k_pe)
    return QMLA_ERR_NULL;
  if (p->pos_rows != 1 && p->pos_rows != 3) return QMLA_ERR_SHAPE;
  if (p->pos_rows == 3 && !p->rope_sec) return QMLA_ERR_NULL;
  if (p->cos_sin_dtype != QMLA_DT_BF16 && p->cos_sin_dtype != QMLA_DT_F32 && p->cos_sin_dtype != QMLA_DT_F16)
    return QMLA_ERR_MODE;
  const int nope = p->head_dim - p->rope_dim;
  if (p->heads <= 0 || p->rope_dim <= 0 || p->rope_dim % 2 || nope <= 0 || nope % 2 || nope > 256 ||
      p->kv_heads <= 0 || p->d_c <= 0 || p->d_c % 256 || p->max_pos <= 0 || p->rope_group <= 0 ||
      p->head_offset < 0 || p->rope_first < 0 || p->rope_span <= 0 ||
      p->rope_first + p->rope_span > p->kv_heads || p->declared_rope % 2 ||
      p->declared_rope < p->rope_span * p->rope_dim + p->heads)
    return QMLA_ERR_SHAPE;
  // every head's group must be one of the cached groups, and exist in k_rope
  const int g_lo = p->head_offset / p->rope_group, g_hi = (p->head_offset + p->heads - 1) / p->rope_group;
  if (g_lo < p->rope_first || g_hi >= p->rope_first + p->rope_span) return QMLA_ERR_SHAPE;
  if (p->q_head_stride < p->head_dim || p->q_token_stride < (int64_t)p->heads * p->q_head_stride ||
      p->latent_stride < p->d_c || p->k_rope_stride < (int64_t)p->kv_heads * p->rope_dim ||
      p->q_out_head_stride < nope + p->declared_rope ||
      p->q_out_token_stride < (int64_t)p->heads * p->q_out_head_stride || p->k_pe_stride < p->declared_rope ||
      (p->pos_rows == 3 && p->pos_row_stride < p->n))
    return QMLA_ERR_SHAPE;
  // 16-byte MFMA operand loads; 4-byte pair loads/stores of q and q_out (16-byte where aligned)
  if (((uintptr_t)p->latent | (uintptr_t)p->k_up) % 16 || p->latent_stride % 8 ||
      ((uintptr_t)p->q | (uintptr_t)p->q_out) % 4 || p->q_token_stride % 2 || p->q_head_stride % 2 ||
      p->q_out_token_stride % 2 || p->q_out_head_stride % 2 || (uintptr_t)p->k_pe % 2 ||
      (uintptr_t)p->k_rope % 2)
    return QMLA_ERR_ALIGN;
  if (p->rope_dim > prep::MAX_RD || p->k_rope_stride % 2) return p->rope_dim > prep::MAX_RD ? QMLA_ERR_SHAPE : QMLA_ERR_ALIGN;
  // blocks: rms blocks of 16 tokens x one head, then row blocks of 8 waves, one q_out row
  // (token, head) or one k_pe rope window (token, cached group) per wave
  const int64_t tiles = (p->n + prep::TM - 1) / prep::TM;
  const int64_t rows = (int64_t)p->n * (p->heads + p->rope_span);
  const int64_t row_blocks = (rows + prep::NTHREADS / 64 - 1) / (prep::NTHREADS / 64);
  if (tiles * p->heads + row_blocks > 0x7fffffff) return QMLA_ERR_SHAPE;
  prep::PParams k;
  k.q = static_cast<const uint16_t*>(p->q);
  k.q_ts = p->q_token_stride;
  k.q_hs = p->q_head_stride;
  k.latent = static_cast<const uint16_t*>(p->latent);
  k.lat_s = p->latent_stride;
  k.k_rope = static_cast<const uint16_t*>(p->k_rope);
  k.kr_s = p->k_rope_stride;
  k.k_up = static_cast<const uint16_t*>(p->k_up);
  k.k_gain = p->k_gain;
  k.cos_sin = p->cos_sin;
  k.cs_dtype = p->cos_sin_dtype;
  k.max_pos = p->max_pos;
  k.positions = p->positions;
  k.pos_rs = p->pos_rows == 3 ? p->pos_row_stride : 0;
  k.pos_rows = p->pos_rows;
  k.rope_sec = p->rope_sec;
  k.n = p->n;
  k.heads = p->heads;
  k.head_dim = p->head_dim;
  k.rd = p->rope_dim;
  k.kv_heads = p->kv_heads;
  k.d_c = p->d_c;
  k.head_offset = p->head_offset;
  k.rope_group = p->rope_group;
  k.rope_first = p->rope_first;
  k.rope_span = p->rope_span;
  k.declared_rope = p->declared_rope;
  k.eps = p->eps;
  k.q_out = static_cast<uint16_t*>(p->q_out);
  k.qo_ts = p->q_out_token_stride;
  k.qo_hs = p->q_out_head_stride;
  k.k_pe = static_cast<uint16_t*>(p->k_pe);
  k.kp_s = p->k_pe_stride;
  k.tiles = (int)tiles;
  k.xcd_map = p->heads % 8 == 0;
  k.rms_blocks = (int)(tiles * p->heads);
  k.row_blocks = (int)row_blocks;
  const int width = nope + p->declared_rope;
  k.vec_out = width % 8 == 0 && p->q_out_token_stride % 8 == 0 && p->q_out_head_stride % 8 == 0 &&
              (uintptr_t)p->q_out % 16 == 0;
  k.vec_in = p->rope_dim % 8 == 0 && p->q_token_stride % 8 == 0 && p->q_head_stride % 8 == 0 &&
             (uintptr_t)p->q % 16 == 0;
  const int nt = (nope + 15) / 16;
  hipError_t e;
  const hipStream_t s = (hipStream_t)stream;
  if (nt <= 4) e = prep::launch<4>(k, s);
  else if (nt <= 8) e = prep::launch<8>(k, s);
  else if (nt <= 12) e = prep::launch<12>(k, s);
  else if (nt <= 13) e = prep::launch<13>(k, s);
  else e = prep::launch<16>(k, s);
  return e == hipSuccess ? QMLA_OK : QMLA_ERR_LAUNCH;
}
