// qmla_ws.hip -- gfx950 warp-specialized MLA decode for one latent group (d_c 512, rope 64, <= 32
// query rows per request: 24 heads, one token each).
//
// A workgroup owns a contiguous token range of one request and all its query rows (every cached row
// is read from HBM once per call). Its 8 waves take two roles, one of each on every SIMD:
//   score waves (0-3): wave (tb, mb) scores 16 tokens x 16 rows over all 576 columns of a 32-token
//                      tile (S^T = K . Q^T on MFMA, its query fragments resident in VGPRs), divides
//                      by the rms, applies the mask and the softmax shift, and writes P (bf16) for
//                      the tile into LDS;
//   value waves (4-7): wave v accumulates P . V over latent columns [128v, 128v+128) for all rows,
//                      one tile behind the score waves, with V^T fragments read by ds_read_b64_tr_b8.
// So on every SIMD an MFMA+conversion-heavy score step of tile t+1 runs beside the MFMA P.V step of
// tile t, and the workgroup meets once per tile at a single barrier (P double-buffered in LDS).
// Rows stream global -> LDS by LDS-DMA through a deep ring (a tile is reused by the value waves one
// step after the score waves), issued by all 8 waves, each waiting only for its own loads.
//
// Softmax: every row keeps one reference max shared by its two score waves. P = exp2(s - ref) is
// written optimistically; if some row's tile max exceeds its reference by more than SHIFT (or the
// row had none yet), the workgroup takes a rare extra step: the score waves agree on the new
// reference, rewrite P, and publish the factor by which the value waves rescale their accumulators
// before they use the tile.
//
// Reference semantics: qwen_mla/ops/mla_decode_attention.py:297-586 (stage 1: tile loop, fp8
// dequant :451-463, rms divide :466-507, softmax :553-560, partial store :562-586).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qmla.h"
#include "qmla_common.h"
#include "qmla_device.h"

namespace qmla {
namespace ws {

constexpr int NW = 8, NTHR = 512;
constexpr int TILE = 32;          // tokens per tile
constexpr int PIDN = 512;         // page ids staged per sub-range
constexpr float SHIFT = 16.0f;    // P <= 2^16 before the reference max moves

__device__ __forceinline__ i32x4 ldsr128(const char* p) {
  i32x4 r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(lds_addr(p)));
  return r;
}
__device__ __forceinline__ uint32_t ldsr8(const char* p) {
  uint32_t r;
  asm volatile("ds_read_u8 %0, %1" : "=v"(r) : "v"(lds_addr(p)));
  return r;
}
__device__ __forceinline__ uint32_t ldsr16(const char* p) {
  uint32_t r;
  asm volatile("ds_read_u16 %0, %1" : "=v"(r) : "v"(lds_addr(p)));
  return r;
}

// Compile-time shape: EB cache element bytes (1 fp8, 2 bf16), RMS tail format, DCG latent columns,
// S ring stages, CPR 16-byte chunks staged per row, CAP tanh logit cap, RTR rms codes read
// transposed (query rows are the heads of one token).
template <int EB_, int RMS_, int DCG_, int S_, int CPR_, bool CAP_, bool RTR_>
struct WS {
  static constexpr int EB = EB_, RMS = RMS_, DCG = DCG_, S = S_, CPR = CPR_;
  static constexpr bool CAP = CAP_, RTR = RTR_;
  static constexpr int RB = 16 * CPR;                 // staged row bytes
  static constexpr int STAGE = TILE * RB;
  static constexpr int NCH = TILE * CPR;              // 16-byte chunks per tile
  static constexpr int NI = (NCH + 63) / 64;          // DMA instructions per tile
  static constexpr int DPW = (NI + NW - 1) / NW;      // ... per wave (at most)
  static constexpr int KQ = (DCG + 64) / 32;          // k-steps of the score product (latent + rope 64)
  static constexpr int KP = KQ / 2;                   // 64-column pairs
  static constexpr int VC = DCG / 4;                  // latent columns per value wave
  static constexpr int CB = VC / 16;
  static constexpr int RMS_EB = (RMS == QMLA_RMS_BF16 || RMS == QMLA_RMS_BF16_BYTES) ? 2 : 1;
  static constexpr int PST = TILE * 2 + 16;           // P row stride in LDS (bytes)
  static_assert(DCG % 64 == 0 && CPR * 16 >= (DCG + 64) * EB, "row slice");
  static_assert(S >= 4 && (S - 3) * (DPW + 1) < 64, "ring depth / vmcnt range");
};

template <class C>
struct Smem {
  char kv[C::S][C::STAGE];
  char p[2][32][C::PST];        // P (bf16) of a tile, double-buffered
  float tmax[2][2][32];         // [parity][score token block][row] tile max
  float alpha[2][32];           // [parity][row] accumulator rescale of the rare step
  int flag[2][4];               // [parity][score wave]
  float fin[2][2][32];          // epilogue: [max, sum][token block][row]
  int pid[PIDN];
};

// rotated row layout: chunk c of staged row r at position (c + (r & 15)) mod CPR
template <int CPR>
__device__ __forceinline__ int rot(int c, int r) {
  const int p = c + (r & 15);
  return p >= CPR ? p - CPR : p;
}
template <int CPR>
__device__ __forceinline__ int lbyte(int r, int b) {
  return r * (16 * CPR) + 16 * rot<CPR>(b >> 4, r) + (b & 15);
}

// DMA instructions wave w issues per tile (instructions w, w+8, ... < NI)
template <class C>
__device__ __forceinline__ constexpr int dpw(int w) { return (C::NI - w + NW - 1) / NW; }

// wait until this wave's loads of tile t landed: at most `ahead` later tiles of its loads remain
template <class C>
__device__ __forceinline__ void wait_own(int w, int ahead) {
  if (ahead <= 0) { wait_vmcnt<0>(); return; }
  const bool big = dpw<C>(w) == dpw<C>(0);
  if (ahead >= C::S - 3) {
    if (big) wait_vmcnt<(C::S - 3) * dpw<C>(0)>();
    else wait_vmcnt<(C::S - 3) * dpw<C>(NW - 1)>();
  } else {
    wait_vmcnt<0>();   // short tail: drain
  }
}

// One contiguous token range [ta, te) of request `req` (length L), all query rows, seen from one
// role. Both roles run the same sub-range / tile / barrier sequence; only the work between the
// barriers differs, so each role keeps only its own registers live (score waves the query
// fragments, value waves the accumulators).
template <class C, bool SCORER>
__device__ __forceinline__ void segment_role(const KParams& p, Smem<C>& sm, int req, int ta, int te, int L,
                                             const SegOut& so, float kscale) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tb = (w >> 1) & 1, smb = w & 1;   // score wave: token block, row block
  const int vw = w & 3;                        // value wave: column slice
  const int ln16 = lane & 15, lg = lane >> 4;
  const int qrows = p.qrows, hpg = p.hpg;
  const int nrows = qrows * hpg;
  const int row0 = req * qrows;
  const int P = p.page_size;
  const int* btrow = p.bt + (int64_t)row0 * p.bt_stride;
  const float c2 = p.sm_scale * kscale * kLog2e;

  // ---- score wave: query fragments for rows 16*smb + ln16 (pair jj, lane group lg: columns
  //      64jj + 16lg .. +16 of [latent | rope]); row limit and rms byte offset ----
  bf16x8 qf[SCORER ? C::KQ : 1];
  int lim = 0, rms_b = 0;
  float mref = kNegInf, lpart = 0.f;
  if constexpr (SCORER) {
    const int r = 16 * smb + ln16;
    const bool ok = r < nrows;
    const int jq = ok ? r / hpg : 0, h = ok ? r - jq * hpg : 0;
    const int lr = L - (qrows - 1 - jq);
    lim = ok ? (lr < te ? lr : te) : 0;
    rms_b = p.rms_off_b + h * C::RMS_EB;
    const __bf16* qn = p.q_nope + (int64_t)(row0 + jq) * p.qn_sr + (int64_t)h * p.qn_sh;
    const __bf16* qp = p.q_pe + (int64_t)(row0 + jq) * p.qp_sr + (int64_t)h * p.qp_sh;
#pragma unroll
    for (int k = 0; k < C::KQ; ++k) {
      const int col = 64 * (k >> 1) + 16 * lg + 8 * (k & 1);
      bf16x8 v = col < C::DCG ? *reinterpret_cast<const bf16x8*>(qn + col)
                              : *reinterpret_cast<const bf16x8*>(qp + (col - C::DCG));
      if (!ok) v = bf16x8{};
      qf[k] = v;
    }
  }
  // ---- value wave: accumulator of rows (16mb + 4lg + i) x columns VC*vw + 16cb + ln16 ----
  f32x4 acc[2][SCORER ? 1 : C::CB];
  if constexpr (!SCORER) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int cb = 0; cb < C::CB; ++cb) acc[mb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // DMA sources: instruction i = w + 8j covers LDS chunks 64i .. 64i+63 of a stage: staged row
  // q / CPR, position q % CPR, i.e. row chunk (position - (row & 15)) mod CPR
  uint32_t doff[C::DPW];
  int drow[C::DPW];
#pragma unroll
  for (int j = 0; j < C::DPW; ++j) {
    int q = (w + NW * j) * 64 + lane;
    q = q < C::NCH ? q : C::NCH - 1;
    const int r = q / C::CPR, pp = q - r * C::CPR;
    int c = pp - (r & 15);
    c = c < 0 ? c + C::CPR : c;
    doff[j] = (uint32_t)(r * C::RB + 16 * c);
    drow[j] = r;
  }

  int sub = (PIDN - 1) * P;
  sub = sub < TILE ? TILE : sub / TILE * TILE;
  for (int sa = ta; sa < te; sa += sub) {
    const int se = te - sa < sub ? te : sa + sub;
    const int pbase = sa / P;
    const int np = (se - 1) / P - pbase + 1;
    wait_vmcnt<0>();
    lds_barrier();   // previous sub-range finished with the page ids and the ring
    for (int i = tid; i < np; i += NTHR) sm.pid[i] = btrow[pbase + i];
    __syncthreads();
    const int nt = (se - sa + TILE - 1) / TILE;
    const bool contig = p.token_stride_b == C::RB;

    // issue cursor: tiles are issued in order, so the page of the next tile is tracked
    // incrementally (no divisions in the tile loop)
    int ipg = sa / P - pbase, ioff = sa % P;   // page index (staged) and offset of tile `inext`
    auto issue = [&](int t) {
      const int tok0 = sa + t * TILE;
      const int nvalid = se - tok0 < TILE ? se - tok0 : TILE;
      char* dst = sm.kv[t % C::S];
      if (contig && ioff + TILE <= P) {
        // the tile's rows are consecutive in one page; rows past the range end read as zeros
        const int pg = __builtin_amdgcn_readfirstlane(sm.pid[ipg]);
        const char* base = p.kv + (int64_t)pg * p.page_stride_b + (int64_t)ioff * p.token_stride_b;
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(base, (uint32_t)(nvalid * C::RB));
#pragma unroll
        for (int j = 0; j < C::DPW; ++j) {
          const int i = w + NW * j;
          if (i < C::NI && (i * 64 + 64 <= C::NCH || i * 64 + lane < C::NCH)) dma16_buf(rs, doff[j], dst + i * 1024);
        }
      } else {
        // per-lane page lookup; rows past the range end repeat the last row
#pragma unroll
        for (int j = 0; j < C::DPW; ++j) {
          const int i = w + NW * j;
          if (i < C::NI && (i * 64 + 64 <= C::NCH || i * 64 + lane < C::NCH)) {
            const int rr = drow[j] < nvalid ? drow[j] : nvalid - 1;
            const int tok = tok0 + rr;
            const int q = tok / P;
            const int pg = sm.pid[q - pbase];
            const uint32_t cb = doff[j] - (uint32_t)(drow[j] * C::RB);
            dma16(p.kv + (int64_t)pg * p.page_stride_b + (int64_t)(tok - q * P) * p.token_stride_b + cb,
                  dst + i * 1024);
          }
        }
      }
      ioff += TILE;
      while (ioff >= P) {
        ioff -= P;
        ++ipg;
      }
    };

    // prologue: tiles 0 .. S-3 in flight, tile 0 landed everywhere
    for (int t = 0; t < C::S - 2 && t < nt; ++t) issue(t);
    wait_own<C>(w, nt - 1 < C::S - 3 ? nt - 1 : C::S - 3);
    lds_barrier();

    // iteration it: score waves take tile it, value waves tile it-1; one barrier per iteration
    // (two when the reference max of some row moves)
#pragma clang loop unroll(disable)
    for (int it = 0; it <= nt; ++it) {
      if (it + C::S - 2 < nt) issue(it + C::S - 2);
      const int par = it & 1;
      const int ahead = nt - 1 - (it + 1) < C::S - 3 ? nt - 1 - (it + 1) : C::S - 3;
      if constexpr (SCORER) {
        if (it < nt) {
          const char* kvs = sm.kv[it % C::S];
          const int tok0 = sa + it * TILE;
          // ---- scores for tokens tok0 + 16tb + (4lg + i), rows 16smb + ln16 ----
          const int krow = 16 * tb + ln16;
          const char* rowp = kvs + krow * C::RB;
          i32x4 kr0[C::KP], kr1[C::EB == 2 ? C::KP : 1];
#pragma unroll
          for (int jj = 0; jj < C::KP; ++jj) {
            const int cbyte = (64 * jj + 16 * lg) * C::EB;
            kr0[jj] = ldsr128(rowp + 16 * rot<C::CPR>(cbyte >> 4, krow));
            if constexpr (C::EB == 2) kr1[jj] = ldsr128(rowp + 16 * rot<C::CPR>((cbyte >> 4) + 1, krow));
          }
          // rms codes of the lane's 4 tokens
          uint32_t code[4];
          if constexpr (C::RMS != QMLA_RMS_NONE) {
            if constexpr (C::RTR && C::RMS_EB == 1) {
              // tr_b8: lanes 2r, 2r+1 of block lg supply token row 16tb + 4lg + (r & 3); lane n gets head 16smb + n
              const int rr = 16 * tb + 4 * lg + ((ln16 >> 1) & 3);
              i32x2 raw = lds_read_tr8_async(kvs + lbyte<C::CPR>(rr, p.rms_off_b + 16 * smb + 8 * (ln16 & 1)));
              lds_wait(raw);
#pragma unroll
              for (int i = 0; i < 4; ++i) code[i] = ((uint32_t)raw[0] >> (8 * i)) & 0xFF;
            } else {
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const char* a = kvs + lbyte<C::CPR>(16 * tb + 4 * lg + i, rms_b);
                code[i] = C::RMS_EB == 1 ? ldsr8(a) : ldsr16(a);
              }
#pragma unroll
              for (int i = 0; i < 4; ++i) lds_wait(code[i]);
            }
          }
          f32x4 s2a = f32x4{0.f, 0.f, 0.f, 0.f}, s2b = s2a;
#pragma unroll
          for (int jj = 0; jj < C::KP; ++jj) {
            lds_wait(kr0[jj]);
            bf16x8 ka, kb;
            if constexpr (C::EB == 1) {
              fp8x16_to_bf16(kr0[jj], ka, kb);
            } else {
              lds_wait(kr1[jj]);
              ka = __builtin_bit_cast(bf16x8, kr0[jj]);
              kb = __builtin_bit_cast(bf16x8, kr1[jj]);
            }
            if (jj & 1) {
              s2b = mfma16(ka, qf[2 * jj], s2b);
              s2b = mfma16(kb, qf[2 * jj + 1], s2b);
            } else {
              s2a = mfma16(ka, qf[2 * jj], s2a);
              s2a = mfma16(kb, qf[2 * jj + 1], s2a);
            }
          }
          f32x4 sc = s2a + s2b;
          // ---- rms divide, scale, cap, mask ----
          float tm = kNegInf;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float rinv = 1.0f;
            if constexpr (C::RMS == QMLA_RMS_LOG8) {
              rinv = fast_exp2(fmaf((float)code[i], -6.0f / 255.0f, 3.0f));   // 1 / 2^(-3 + c*6/255)
            } else if constexpr (C::RMS == QMLA_RMS_E4M3) {
              const float rv = fp8_to_f32(code[i]) * kscale;
              rinv = rv > 0.f ? __builtin_amdgcn_rcpf(rv) : 1.0f;
            } else if constexpr (C::RMS == QMLA_RMS_BF16 || C::RMS == QMLA_RMS_BF16_BYTES) {
              const float rv = bf16_bits_to_f32(code[i]);
              rinv = rv > 0.f ? __builtin_amdgcn_rcpf(rv) : 1.0f;
            }
            float v;
            if constexpr (C::CAP) {
              const float sn = sc[i] * (c2 * kLn2) * rinv;
              const float th = 1.0f - 2.0f / (fast_exp2(2.0f * kLog2e * (sn / p.logit_cap)) + 1.0f);
              v = p.logit_cap * th * kLog2e;
            } else {
              v = sc[i] * c2 * rinv;
            }
            v = tok0 + 16 * tb + 4 * lg + i < lim ? v : kNegInf;
            sc[i] = v;
            tm = fmaxf(tm, v);
          }
          tm = max_lg(tm);
          // ---- optimistic P against the current reference; the rare step fixes it ----
          const float mu = mref == kNegInf ? 0.f : mref;
          bf16x4 pk;
          float ps = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float e = fast_exp2(sc[i] - mu);
            ps += e;
            pk[i] = (__bf16)e;
          }
          *reinterpret_cast<bf16x4*>(&sm.p[par][16 * smb + ln16][(16 * tb + 4 * lg) * 2]) = pk;
          if (lg == 0) sm.tmax[par][tb][16 * smb + ln16] = tm;
          const bool any = __builtin_amdgcn_ballot_w64(tm > mref + SHIFT) != 0;
          if (lane == 0) sm.flag[par][w] = any ? 1 : 0;
          wait_own<C>(w, ahead);
          lds_barrier();
          const bool rare = (sm.flag[par][0] | sm.flag[par][1] | sm.flag[par][2] | sm.flag[par][3]) != 0;
          if (!rare) {
            lpart += ps;
          } else {
            const int r = 16 * smb + ln16;
            const float gm = fmaxf(sm.tmax[par][0][r], sm.tmax[par][1][r]);
            const float mn = gm > mref + SHIFT ? gm : mref;
            const float alpha = mref == kNegInf ? 0.f : fast_exp2(mref - mn);
            mref = mn;
            const float mu2 = mref == kNegInf ? 0.f : mref;
            bf16x4 pk2;
            float ps2 = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float e = fast_exp2(sc[i] - mu2);
              ps2 += e;
              pk2[i] = (__bf16)e;
            }
            lpart = lpart * alpha + ps2;
            *reinterpret_cast<bf16x4*>(&sm.p[par][r][(16 * tb + 4 * lg) * 2]) = pk2;
            if (tb == 0 && lg == 0) sm.alpha[par][r] = alpha;
            lds_barrier();
          }
        } else {
          // no tile left for the score waves: meet the value waves (no rare step at it == nt)
          wait_own<C>(w, ahead);
          lds_barrier();
        }
      } else {
        if (it >= 1) {
          // ---- P . V for tile it-1 over columns VC*vw .. +VC ----
          const int pv = (it - 1) & 1;
          const char* kvs = sm.kv[(it - 1) % C::S];
          bf16x8 pf[2];
#pragma unroll
          for (int mb = 0; mb < 2; ++mb)
            pf[mb] = __builtin_bit_cast(bf16x8, ldsr128(&sm.p[pv][16 * mb + ln16][(8 * lg) * 2]));
          i32x2 vraw[C::CB][C::EB];
#pragma unroll
          for (int cb = 0; cb < C::CB; ++cb) {
            const int col0 = C::VC * vw + 16 * cb;
            if constexpr (C::EB == 1) {
              const int vr = 8 * lg + (ln16 >> 1);
              vraw[cb][0] = lds_read_tr8_async(kvs + lbyte<C::CPR>(vr, col0 + 8 * (ln16 & 1)));
            } else {
              const int vr = 8 * lg + (ln16 >> 2);
              const int vb = (col0 + 4 * (ln16 & 3)) * 2;
              vraw[cb][0] = lds_read_tr16_async(kvs + lbyte<C::CPR>(vr, vb));
              vraw[cb][C::EB - 1] = lds_read_tr16_async(kvs + lbyte<C::CPR>(vr + 4, vb));
            }
          }
          lds_wait(pf[0], pf[1]);
#pragma unroll
          for (int cb = 0; cb < C::CB; ++cb) {
            i32x2 c0 = vraw[cb][0], c1 = vraw[cb][C::EB - 1];
            if constexpr (C::EB == 1) lds_wait(c0);
            else lds_wait(c0, c1);
            bf16x8 vf;
            if constexpr (C::EB == 1) {
              vf = fp8x8_to_bf16(c0);
            } else {
              const i32x4 w4 = {c0[0], c0[1], c1[0], c1[1]};
              vf = __builtin_bit_cast(bf16x8, w4);
            }
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) acc[mb][cb] = mfma16(pf[mb], vf, acc[mb][cb]);
          }
        }
        wait_own<C>(w, ahead);
        lds_barrier();
        if (it < nt) {
          const bool rare = (sm.flag[par][0] | sm.flag[par][1] | sm.flag[par][2] | sm.flag[par][3]) != 0;
          if (rare) {
            lds_barrier();   // the score waves published the rescale of tile it
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const float a = sm.alpha[par][16 * mb + 4 * lg + i];
#pragma unroll
                for (int cb = 0; cb < C::CB; ++cb) acc[mb][cb][i] *= a;
              }
          }
        }
      }
    }
  }
  wait_vmcnt<0>();

  // ---- epilogue: score waves publish (reference max, sum) per row and token block; value waves
  //      normalize their columns and write the output (final or partial) and natural-log lse ----
  if constexpr (SCORER) {
    const float l = sum_lg(lpart);
    if (lg == 0) {
      sm.fin[0][tb][16 * smb + ln16] = mref;
      sm.fin[1][tb][16 * smb + ln16] = l;
    }
  }
  lds_barrier();
  if constexpr (!SCORER) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * mb + 4 * lg + i;
        if (r >= nrows) continue;
        const float m = sm.fin[0][0][r];
        const float l = sm.fin[1][0][r] + sm.fin[1][1][r];
        const int jq = r / hpg, h = r - jq * hpg;
        const float inv = l > 0.f ? kscale / l : 0.f;   // fp8 values were accumulated unscaled
        const float lse_v = l > 0.f ? (m + fast_log2(l)) * kLn2 : kNegInf;
        const int col = C::VC * vw + ln16;
        if (so.final_out) {
          const int64_t ob = (int64_t)(row0 + jq) * p.o_sr + (int64_t)h * p.o_sh + col;
#pragma unroll
          for (int cb = 0; cb < C::CB; ++cb) store_out(p.out, p.out_dt, ob + 16 * cb, acc[mb][cb][i] * inv);
          if (vw == 0 && ln16 == 0 && p.lse) store_out(p.lse, p.lse_dt, (int64_t)(row0 + jq) * p.lse_sr + h, lse_v);
        } else {
          float* ob = so.po + (int64_t)jq * so.po_sr + (int64_t)h * so.po_sh + col;
#pragma unroll
          for (int cb = 0; cb < C::CB; ++cb) ob[16 * cb] = acc[mb][cb][i] * inv;
          if (vw == 0 && ln16 == 0) {
            if (so.plse) so.plse[(int64_t)jq * so.plse_sr + h] = lse_v;
            else so.po[(int64_t)jq * so.po_sr + (int64_t)h * so.po_sh + C::DCG] = lse_v;
          }
        }
      }
  }
  lds_barrier();   // LDS free for the next range
}

template <class C>
__device__ __forceinline__ void segment(const KParams& p, Smem<C>& sm, int req, int ta, int te, int L,
                                        const SegOut& so, float kscale) {
  if (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) < 4) segment_role<C, true>(p, sm, req, ta, te, L, so, kscale);
  else segment_role<C, false>(p, sm, req, ta, te, L, so, kscale);
}

template <class C>
__global__ __launch_bounds__(NTHR, 1) void ws_kernel(const KParams p) {
  static_assert(sizeof(Smem<C>) <= 163840, "LDS budget of a workgroup");
  __shared__ __attribute__((aligned(16))) Smem<C> sm;
  const float kscale = (C::EB == 1 && p.k_scale) ? *p.k_scale : 1.0f;
  for_each_segment<C::DCG>(p, [&](int req, int a, int e, int L, const SegOut& so) {
    segment<C>(p, sm, req, a, e, L, so, kscale);
  });
}

struct Inst {
  int eb, rms, dcg, cpr;
  bool cap, rtr;
  void (*fn)(const KParams);
};

#define QMLA_WS(EB, RMS, DCG, S, CPR, CAP, RTR) \
  {EB, RMS, DCG, CPR, CAP, RTR, &ws_kernel<WS<EB, RMS, DCG, S, CPR, CAP, RTR>>}

static const Inst kInst[] = {
    // fp8 e4m3 + log8 codes, d_c 512, rope 64, 24 heads: 608-byte rows, 6-stage ring of 32-token tiles
    QMLA_WS(1, QMLA_RMS_LOG8, 512, 6, 38, false, true),
    QMLA_WS(1, QMLA_RMS_LOG8, 512, 6, 38, false, false),
};

}  // namespace ws

int ws_select(const qmla_decode_params* p) {
  if (p->rope_w != 64 || p->groups != 1 || p->qrows * p->heads > 32) return -1;
  const int eb = p->kv_dtype == QMLA_KV_FP8 ? 1 : 2;
  const bool cap = p->logit_cap > 0.f;
  const int64_t ts = p->token_stride * eb;
  for (int i = 0; i < (int)(sizeof(ws::kInst) / sizeof(ws::kInst[0])); ++i) {
    const ws::Inst& in = ws::kInst[i];
    if (in.eb != eb || in.rms != p->rms_mode || in.dcg != p->d_c || in.cap != cap) continue;
    if (in.rtr && (p->qrows != 1 || p->heads > 32)) continue;
    if ((int64_t)in.cpr * 16 > ts) continue;   // never read past a row
    if (p->rms_mode != QMLA_RMS_NONE) {
      const int rb = (p->rms_mode == QMLA_RMS_BF16 || p->rms_mode == QMLA_RMS_BF16_BYTES) ? 2 : 1;
      const int64_t roff = (int64_t)p->rms_offset * eb;
      // staged bytes cover the rms of every head (transposed reads take 16 heads per 16-byte chunk)
      const int64_t need = in.rtr ? (roff % 16 == 0 ? roff + 32 : 1 << 30) : roff + (int64_t)p->heads * rb;
      if (need > in.cpr * 16) continue;
    }
    return i;
  }
  return -1;
}

int ws_launch(int inst, const qmla_decode_params* p, const KParams& k, int nwg, hipStream_t st) {
  KParams kk = k;
  void* args[] = {&kk};
  dim3 grid = p->num_splits > 0 ? dim3(p->num_splits, k.n_req, 1) : dim3(nwg, 1, 1);
  if (grid.x == 0 || grid.y == 0) return QMLA_OK;
  hipError_t e = hipLaunchKernel((const void*)ws::kInst[inst].fn, grid, dim3(ws::NTHR, 1, 1), args, 0, st);
  return e == hipSuccess ? QMLA_OK : QMLA_ERR_LAUNCH;
}

}  // namespace qmla
