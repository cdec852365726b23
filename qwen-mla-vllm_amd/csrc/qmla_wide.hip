// qmla_wide.hip -- gfx950 single-pass decode for wide latents (d_c = 1792, bf16 cache).
//
// At d_c = 1792 a workgroup's output accumulator is 32 rows x 1792 fp32 (224 KB) and the query
// fragments another 32 x 1856 bf16 (116 KB): together they only fit in the register files of all
// four SIMDs, so this kernel splits COLUMNS across 8 waves (two per SIMD) rather than tokens. Wave
// w owns latent columns [w*DCW, (w+1)*DCW) (DCW = d_c/8) for both the score product and P.V, waves
// 0-3 also rope columns [16w, 16w+16); each stages only its slice of every row in a private LDS
// ring and waits for its own DMA; wave 0 also stages the rms tail for everyone. Per 16-token tile:
//   QK       S_w^T = K_w . Q_w^T on MFMA (16x16x32 over the latent slice, 16x16x16 over the rope
//            slice): partial scores of 16 tokens x 32 query rows, query fragments in VGPRs.
//   sum      the eight partials meet in LDS; every wave adds them in the same order, so all waves
//            hold bit-identical scores and take identical softmax decisions.
//   softmax  redundantly in every wave (8 scores per lane): rms divide, scale, mask, a lazily moving
//            reference max; P (bf16) is already in the A-operand layout of the 16x16x16 P.V product.
//   PV       acc_w[32 x DCW] += P . V_w on MFMA, V^T fragments read with ds_read_b64_tr_b16.
// The reference runs these widths as two passes (scores into an fp32 scratch, then P.V over column
// slices, qwen_mla/ops/mla_decode_attention.py:602-849) and reads the latent twice; here every row
// is read from HBM once and the scores never leave the chip. Output format and split bounds are
// those of the d_c <= 1024 kernel (attn_logits partials or the balanced plan, then the combine).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qmla.h"
#include "qmla_common.h"
#include "qmla_device.h"

namespace qmla {
namespace wide {

typedef __attribute__((__vector_size__(4 * sizeof(short)))) short s16x4;

constexpr int NW = 8;
constexpr int NTHR = NW * 64;
constexpr int T = 16;        // tokens per tile
constexpr int PIDN = 1024;   // page ids staged per sub-range

__device__ __forceinline__ f32x4 mfma16k16(const s16x4& a, const s16x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// LDS reads issued as inline asm (the builtins make the compiler wait for every LDS-DMA in flight
// first); results are valid after lds_wait().
__device__ __forceinline__ i32x4 lds_b128_async(const char* p) {
  i32x4 r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(lds_addr(p)));
  return r;
}
__device__ __forceinline__ i32x2 lds_b64_async(const char* p) {
  i32x2 r;
  asm volatile("ds_read_b64 %0, %1" : "=v"(r) : "v"(lds_addr(p)));
  return r;
}
__device__ __forceinline__ uint32_t lds_u16_async(const char* p) {
  uint32_t r;
  asm volatile("ds_read_u16 %0, %1" : "=v"(r) : "v"(lds_addr(p)));
  return r;
}

// Compile-time shape: bf16 cache, latent DC (8 column slices), rope 64, rms tail of at most 8*CRM
// heads (CRM 16-byte chunks, staged once per tile by wave 0), S-stage rings.
template <int RMS_, int DC_, int CRM_, int S_>
struct WCfg {
  static constexpr int RMS = RMS_, DC = DC_, CRM = CRM_, S = S_;
  static constexpr int EB = 2;
  static constexpr int DCW = DC / NW;                    // latent columns per wave
  static constexpr int KS = DCW / 32;                    // latent k-steps of the score product
  static constexpr int CB = DCW / 16;                    // 16-column output blocks per wave
  static constexpr int MB = 2, ROWS = 32;
  static constexpr int CL = DCW * EB / 16;               // latent chunks of a row slice
  static constexpr int CR = 16 * EB / 16;                // rope chunks
  static constexpr int CPW = (CL + CR) | 1;              // odd: the 16 rows of a K read hit distinct banks
  static constexpr int RS = 16 * CPW;                    // LDS row stride (bytes)
  static constexpr int NCH = T * CPW;                    // chunks per tile per wave
  static constexpr int NI = (NCH + 63) / 64;             // DMA instructions per tile per wave
  static constexpr int SB = NCH * 16;                    // stage bytes per wave
  static constexpr int NR = CRM > 0 ? 1 : 0;             // wave 0's extra rms DMA per tile
  static_assert(DC % 256 == 0, "8 column slices of whole 32-column k-steps");
  static_assert(T * CRM <= 64, "rms tail in one DMA instruction");
  static_assert((S - 1) * (NI + NR) < 64, "vmcnt range");
};

template <class C>
struct Smem {
  char ring[C::S][NW][C::SB];
  char rms[2 * C::S][T * 16 * (C::CRM > 0 ? C::CRM : 1)];   // 2S deep: read after the exchange
  f32x4 xb[NW][C::MB][64];   // partial scores
  int pid[PIDN];
};

template <class C>
__device__ __forceinline__ void wait_tile(bool steady, int w) {
  if (!steady) wait_vmcnt<0>();
  else if (w == 0) wait_vmcnt<(C::S - 1) * (C::NI + C::NR)>();
  else wait_vmcnt<(C::S - 1) * C::NI>();
}

// One contiguous token range [ta, te) of request `req` (length L), all query rows.
template <class C>
__device__ __forceinline__ void segment(const KParams& p, Smem<C>& sm, int req, int ta, int te, int L,
                                        const SegOut& so) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln16 = lane & 15, lg = lane >> 4;
  const int H = p.heads;
  const int nrows = p.qrows * H;
  const int row0 = req * p.qrows;
  const int P = p.page_size;
  const int64_t TS = p.token_stride_b, PS = p.page_stride_b;
  const int* btrow = p.bt + (int64_t)row0 * p.bt_stride;
  const float csc = p.sm_scale * kLog2e;

  // ---- query fragments (B operands), zero for padding rows ----
  bf16x8 qf[C::KS][C::MB];
  s16x4 qr[C::MB];
  int lim[C::MB];
#pragma unroll
  for (int mb = 0; mb < C::MB; ++mb) {
    const int r = ln16 + 16 * mb;
    const bool ok = r < nrows;
    const int jq = ok ? r / H : 0, h = ok ? r - jq * H : 0;
    // verify row jq of the request sees its first L - (qrows-1-jq) tokens (mla_impl.py:628-662)
    const int lr = L - (p.qrows - 1 - jq);
    lim[mb] = ok ? (lr < te ? lr : te) : 0;
    const __bf16* qn = p.q_nope + (int64_t)(row0 + jq) * p.qn_sr + (int64_t)h * p.qn_sh + w * C::DCW + 8 * lg;
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
      bf16x8 v = *reinterpret_cast<const bf16x8*>(qn + 32 * ks);
      if (!ok) v = bf16x8{};
      qf[ks][mb] = v;
    }
    const __bf16* qp = p.q_pe + (int64_t)(row0 + jq) * p.qp_sr + (int64_t)h * p.qp_sh + 16 * (w & 3) + 4 * lg;
    s16x4 v = *reinterpret_cast<const s16x4*>(qp);
    if (!ok || w >= 4) v = s16x4{};
    qr[mb] = v;
  }

  // ---- per-lane DMA sources: instruction k, lane l -> chunk i = 64k + l of the wave's tile slice:
  //      token i / CPW, chunk i % CPW of [latent slice | rope slice | pad]; lanes past the tile idle.
  //      Wave 0's extra instruction stages the rms tail: lane l -> token l / CRM, chunk l % CRM.
  //      Recomputed at every issue (a few integer ops) rather than held in registers. ----
  auto src_off = [&](int k, int ln, int& tt) {
    const int i = 64 * k + ln;
    const int t = i / C::CPW, c = i - t * C::CPW;
    int off;
    if (c < C::CL) off = w * C::DCW * C::EB + 16 * c;
    else if (c < C::CL + C::CR) off = C::DC * C::EB + (w & 3) * 16 * C::EB + 16 * (c - C::CL);
    else off = 0;
    tt = i < C::NCH ? t : 0;
    return off;
  };
  const int rtok = C::CRM > 0 ? lane / (C::CRM > 0 ? C::CRM : 1) : 0;
  const int roff = C::CRM > 0 ? rtok * (int)TS + p.rms_off_b + 16 * (lane - rtok * C::CRM) : 0;
  const bool rlane = lane < T * C::CRM;

  // byte offset of each softmax row's head inside a staged rms row (row = ln16 + 16*mb)
  int hb[C::MB];
#pragma unroll
  for (int mb = 0; mb < C::MB; ++mb) {
    const int r = ln16 + 16 * mb;
    hb[mb] = r < nrows ? 2 * (r - (r / H) * H) : 0;
  }

  float mref[C::MB], lpart[C::MB];
  f32x4 acc[C::MB][C::CB];
#pragma unroll
  for (int mb = 0; mb < C::MB; ++mb) {
    mref[mb] = kNegInf;
    lpart[mb] = 0.f;
#pragma unroll
    for (int cb = 0; cb < C::CB; ++cb) acc[mb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // sub-ranges of at most PIDN pages, in whole tiles
  int sub = (PIDN - 1) * P;
  sub = sub < T ? T : sub / T * T;
  const bool uni = (P % T) == 0 && (ta % T) == 0;   // every tile within one page
  for (int sa = ta; sa < te; sa += sub) {
    const int se = te - sa < sub ? te : sa + sub;
    const int pbase = sa / P;
    const int np = (se - 1) / P - pbase + 1;
    wait_vmcnt<0>();
    lds_barrier();   // every wave is done with the previous sub-range's page ids
    for (int i = tid; i < np; i += NTHR) sm.pid[i] = btrow[pbase + i];
    __syncthreads();
    const int nt = (se - sa + T - 1) / T;

    auto issue = [&](int t) {
      const int tok0 = sa + t * T;
      const int nvalid = se - tok0 < T ? se - tok0 : T;
      char* dst = sm.ring[t % C::S][w];
      char* rdst = sm.rms[t % (2 * C::S)];
      int ln = lane;
      asm volatile("" : "+v"(ln));   // keep the offsets from being hoisted out of the tile loop
      if (uni) {
        const int pg = __builtin_amdgcn_readfirstlane(sm.pid[tok0 / P - pbase]);
        const char* base = p.kv + (int64_t)pg * PS + (int64_t)(tok0 % P) * TS;
        // rows past the segment end read as zeros (outside the resource)
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(base, (uint32_t)(nvalid * TS));
#pragma unroll
        for (int k = 0; k < C::NI; ++k) {
          int tt;
          const int off = src_off(k, ln, tt);
          if (64 * k + 64 <= C::NCH || 64 * k + ln < C::NCH)
            dma16_buf(rs, (uint32_t)(tt * (int)TS + off), dst + k * 1024);
        }
        if (C::NR && w == 0 && rlane) dma16_buf(rs, (uint32_t)roff, rdst);
      } else {
        // pages change inside a tile: per-lane page lookup; rows past the end repeat the last row
#pragma unroll
        for (int k = 0; k < C::NI; ++k) {
          int tt;
          const int off = src_off(k, ln, tt);
          if (64 * k + 64 <= C::NCH || 64 * k + ln < C::NCH) {
            const int tok = tok0 + (tt < nvalid ? tt : nvalid - 1);
            const int q = tok / P;
            const int pg = sm.pid[q - pbase];
            dma16(p.kv + (int64_t)pg * PS + (int64_t)(tok - q * P) * TS + off, dst + k * 1024);
          }
        }
        if (C::NR && w == 0 && rlane) {
          const int tok = tok0 + (rtok < nvalid ? rtok : nvalid - 1);
          const int q = tok / P;
          const int pg = sm.pid[q - pbase];
          dma16(p.kv + (int64_t)pg * PS + (int64_t)(tok - q * P) * TS + (roff - rtok * (int)TS), rdst);
        }
      }
    };

    for (int t = 0; t < C::S && t < nt; ++t) issue(t);

#pragma clang loop unroll(disable)
    for (int t = 0; t < nt; ++t) {
      wait_tile<C>(t + C::S - 1 < nt, w);
      const char* st = sm.ring[t % C::S][w];
      const int tok0 = sa + t * T;

      // ---- partial scores over this wave's columns ----
      f32x4 sp[C::MB];
#pragma unroll
      for (int mb = 0; mb < C::MB; ++mb) sp[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
      {
        const char* kr = st + ln16 * C::RS + 16 * lg;
        i32x2 rope = lds_b64_async(st + ln16 * C::RS + 16 * C::CL + 8 * lg);
        constexpr int KB = 4;   // k-steps per batch of LDS reads
#pragma unroll
        for (int k0 = 0; k0 < C::KS; k0 += KB) {
          i32x4 kv[KB];
#pragma unroll
          for (int j = 0; j < KB; ++j)
            if (k0 + j < C::KS) kv[j] = lds_b128_async(kr + 64 * (k0 + j));
#pragma unroll
          for (int j = 0; j < KB; ++j)
            if (k0 + j < C::KS) {
              lds_wait(kv[j]);
              const bf16x8 kf = __builtin_bit_cast(bf16x8, kv[j]);
#pragma unroll
              for (int mb = 0; mb < C::MB; ++mb) sp[mb] = mfma16(kf, qf[k0 + j][mb], sp[mb]);
            }
        }
        lds_wait(rope);
        if (w < 4) {
          const s16x4 rf = __builtin_bit_cast(s16x4, rope);
#pragma unroll
          for (int mb = 0; mb < C::MB; ++mb) sp[mb] = mfma16k16(rf, qr[mb], sp[mb]);
        }
      }

      // ---- sum the eight partials (same order in every wave); the rms codes of the tile are read
      //      before the second barrier, after which wave 0 may refill their stage ----
#pragma unroll
      for (int mb = 0; mb < C::MB; ++mb) sm.xb[w][mb][lane] = sp[mb];
      lds_barrier();
      f32x4 s[C::MB];
#pragma unroll
      for (int mb = 0; mb < C::MB; ++mb) {
        // four partials in flight at a time; summed in wave order 0..7 in every wave
        f32x4 a;
#pragma unroll
        for (int v0 = 0; v0 < NW; v0 += 4) {
          i32x4 x[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) x[j] = lds_b128_async(reinterpret_cast<const char*>(&sm.xb[v0 + j][mb][lane]));
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            lds_wait(x[j]);
            const f32x4 y = __builtin_bit_cast(f32x4, x[j]);
            a = (v0 + j == 0) ? y : a + y;
          }
        }
        s[mb] = a;
      }
      lds_barrier();   // the partial-score buffer is free again

      // this tile's rms codes (staged by wave 0; its wait preceded the first barrier). The rms ring
      // is 2S deep, so wave 0 refills this stage only S tiles after every wave has passed the
      // first barrier of the next tile.
      uint32_t rraw[C::MB][4];
      if constexpr (C::RMS == QMLA_RMS_BF16) {
        const char* rs = sm.rms[t % (2 * C::S)] + (4 * lg) * (16 * C::CRM);
#pragma unroll
        for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
          for (int e = 0; e < 4; ++e) rraw[mb][e] = lds_u16_async(rs + e * (16 * C::CRM) + hb[mb]);
#pragma unroll
        for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
          for (int e = 0; e < 4; ++e) lds_wait(rraw[mb][e]);
      }

      // ---- rms divide, scale, mask, lazy online softmax; P in the A layout of 16x16x16 ----
      s16x4 pb[C::MB];
      float tmax[C::MB];
#pragma unroll
      for (int mb = 0; mb < C::MB; ++mb) {
        float m = kNegInf;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int tok = tok0 + 4 * lg + e;
          float rinv = 1.0f;
          if constexpr (C::RMS == QMLA_RMS_BF16) {
            const float rv = bf16_bits_to_f32(rraw[mb][e]);
            rinv = rv > 0.f ? __builtin_amdgcn_rcpf(rv) : 1.0f;
          }
          float v = s[mb][e] * rinv * csc;
          if (tok >= lim[mb]) v = kNegInf;
          s[mb][e] = v;
          m = fmaxf(m, v);
        }
        tmax[mb] = max_lg(m);
      }
      // the reference max moves only when a tile max exceeds it by more than 8 (P <= 2^8 in bf16);
      // the rescale is applied unconditionally (alpha = 1 when it does not move): no branch, so the
      // accumulator keeps one register assignment through the loop
#pragma unroll
      for (int mb = 0; mb < C::MB; ++mb) {
        const float mn = tmax[mb] > mref[mb] + 8.0f ? tmax[mb] : mref[mb];
        const float alpha = mref[mb] == kNegInf ? 0.f : fast_exp2(mref[mb] - mn);
        lpart[mb] *= alpha;
        mref[mb] = mn;
        // accumulator rows 4*lg + i live in lanes 4*lg + i of the softmax layout
        float al[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * lg + i);
#pragma unroll
        for (int cb = 0; cb < C::CB; ++cb)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[mb][cb][i] *= al[i];
      }
#pragma unroll
      for (int mb = 0; mb < C::MB; ++mb) {
        const float mu = mref[mb] == kNegInf ? 0.f : mref[mb];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float pv = fast_exp2(s[mb][e] - mu);
          lpart[mb] += pv;
          pb[mb][e] = __builtin_bit_cast(short, (__bf16)pv);
        }
      }

      // ---- P.V over this wave's columns ----
      {
        const char* vb = st + (4 * lg + (ln16 >> 2)) * C::RS + 8 * (ln16 & 3);
        constexpr int VB = 7;
#pragma unroll
        for (int c0 = 0; c0 < C::CB; c0 += VB) {
          i32x2 vr[VB];
#pragma unroll
          for (int j = 0; j < VB; ++j)
            if (c0 + j < C::CB) vr[j] = lds_read_tr16_async(vb + 32 * (c0 + j));
#pragma unroll
          for (int j = 0; j < VB; ++j)
            if (c0 + j < C::CB) {
              lds_wait(vr[j]);
              const s16x4 vf = __builtin_bit_cast(s16x4, vr[j]);
#pragma unroll
              for (int mb = 0; mb < C::MB; ++mb) acc[mb][c0 + j] = mfma16k16(pb[mb], vf, acc[mb][c0 + j]);
            }
        }
      }
      if (t + C::S < nt) issue(t + C::S);
    }
  }
  wait_vmcnt<0>();

  // ---- epilogue: row sums across the 4 lanes of a row, normalize, write ----
#pragma unroll
  for (int mb = 0; mb < C::MB; ++mb) {
    const float l = sum_lg(lpart[mb]);
    const float lse_v = l > 0.f ? (mref[mb] + fast_log2(l)) * kLn2 : kNegInf;
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    float iv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) iv[i] = __shfl(inv, 4 * lg + i);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * mb + 4 * lg + i;
      if (r >= nrows) continue;
      const int jq = r / H, h = r - jq * H;
      const int col = w * C::DCW + ln16;
      if (so.final_out) {
        const int64_t ob = (int64_t)(row0 + jq) * p.o_sr + (int64_t)h * p.o_sh + col;
        if (p.out_dt == QMLA_DT_BF16) {
          __bf16* o = reinterpret_cast<__bf16*>(p.out) + ob;
#pragma unroll
          for (int cb = 0; cb < C::CB; ++cb) o[16 * cb] = (__bf16)(acc[mb][cb][i] * iv[i]);
        } else if (p.out_dt == QMLA_DT_F16) {
          _Float16* o = reinterpret_cast<_Float16*>(p.out) + ob;
#pragma unroll
          for (int cb = 0; cb < C::CB; ++cb) o[16 * cb] = (_Float16)(acc[mb][cb][i] * iv[i]);
        } else {
          float* o = reinterpret_cast<float*>(p.out) + ob;
#pragma unroll
          for (int cb = 0; cb < C::CB; ++cb) o[16 * cb] = acc[mb][cb][i] * iv[i];
        }
      } else {
        float* ob = so.po + (int64_t)jq * so.po_sr + (int64_t)h * so.po_sh + col;
#pragma unroll
        for (int cb = 0; cb < C::CB; ++cb) ob[16 * cb] = acc[mb][cb][i] * iv[i];
      }
    }
    // lse from the softmax layout (row ln16 + 16mb), one lane per row
    const int r = ln16 + 16 * mb;
    if (w == 0 && lg == 0 && r < nrows) {
      const int jq = r / H, h = r - jq * H;
      if (so.final_out) {
        if (p.lse) store_out(p.lse, p.lse_dt, (int64_t)(row0 + jq) * p.lse_sr + h, lse_v);
      } else if (so.plse) {
        so.plse[(int64_t)jq * so.plse_sr + h] = lse_v;
      } else {
        so.po[(int64_t)jq * so.po_sr + (int64_t)h * so.po_sh + C::DC] = lse_v;
      }
    }
  }
}

template <class C>
__global__ __launch_bounds__(NTHR, 1) void wide_kernel(const KParams p) {
  __shared__ __attribute__((aligned(16))) Smem<C> sm;
  for_each_segment<C::DC>(p, [&](int req, int a, int e, int L, const SegOut& so) {
    segment<C>(p, sm, req, a, e, L, so);
  });
}

struct WInst {
  int rms, dc, crm;
  void (*fn)(const KParams);
};

#define QMLA_WINST(RMS, DC, CRM, S) {RMS, DC, CRM, &wide_kernel<WCfg<RMS, DC, CRM, S>>}

static const WInst kWInst[] = {
    // bf16 cache, d_c 1792, rope 64, up to 24 heads of bf16 rms (3 chunks): 2 x 7.75 KB ring per wave
    QMLA_WINST(QMLA_RMS_BF16, 1792, 3, 2),
    QMLA_WINST(QMLA_RMS_NONE, 1792, 0, 2),
};

}  // namespace wide

int wide_select(const qmla_decode_params* p) {
  if (p->kv_dtype != QMLA_KV_BF16 || p->groups != 1 || p->rope_w != 64 || p->logit_cap > 0.f) return -1;
  if ((int64_t)p->qrows * p->heads > 32) return -1;
  const int64_t ts = p->token_stride * 2;
  for (int i = 0; i < (int)(sizeof(wide::kWInst) / sizeof(wide::kWInst[0])); ++i) {
    const wide::WInst& in = wide::kWInst[i];
    if (in.rms != p->rms_mode || in.dc != p->d_c) continue;
    if ((int64_t)in.dc * 2 + 128 > ts) continue;
    if (in.crm > 0) {
      const int64_t roff = (int64_t)p->rms_offset * 2;
      if (p->heads * 2 > 16 * in.crm || roff % 16 || roff + 16 * in.crm > ts) continue;
    }
    return i;
  }
  return -1;
}

int wide_launch(int inst, const qmla_decode_params* p, const KParams& k, int nwg, hipStream_t st) {
  KParams kk = k;
  void* args[] = {&kk};
  dim3 grid = p->num_splits > 0 ? dim3(p->num_splits, k.n_req, 1) : dim3(nwg, 1, 1);
  if (grid.x == 0 || grid.y == 0) return QMLA_OK;
  hipError_t e = hipLaunchKernel((const void*)wide::kWInst[inst].fn, grid, dim3(wide::NTHR, 1, 1), args, 0, st);
  return e == hipSuccess ? QMLA_OK : QMLA_ERR_LAUNCH;
}

}  // namespace qmla
