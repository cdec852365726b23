// qmla_ws.hip -- gfx950 warp-specialized MLA decode for one latent group (d_c 512, rope 64, <= 32
// query rows per request: 24 heads, one token each).
//
// A workgroup owns a contiguous range of the concatenated requests' tokens (balanced mode) or one
// split of one request (fixed splits), with all query rows, so every cached row is read from HBM
// once per call. It walks its range as ONE sequence of 32-token tiles across request boundaries:
// the DMA keeps streaming into the next request while the last tiles of the previous one are still
// being scored and accumulated, so a request boundary costs no pipeline fill or drain. The pieces of
// the range (one per request) and their page ids are staged in LDS once per window (a window holds up
// to NSEG pieces and PIDN pages; a range that needs more is walked in several windows).
//
// Its 8 waves take two roles, one of each on every SIMD:
//   score waves (0-3):  wave (tb, mb) scores 16 tokens x 16 rows over all 576 columns of a tile
//                       (S^T = K . Q^T on MFMA, query fragments resident in VGPRs), divides by the
//                       rms, applies the mask and the softmax shift, and writes P into LDS (fp16
//                       for fp8 rows, bf16 for bf16 rows).
//                       With an fp8 cache the K bytes enter the MFMA as stored: the query is split
//                       into two e4m3 parts (hi + lo, 8 significant bits, as bf16), the latent runs
//                       on the 16x16x128 fp8 MFMA and the rope on the 16x16x32 one;
//   value waves (4-7):  wave v accumulates P . V over latent columns [128v, 128v+128) for all rows,
//                       two tiles behind the score waves, with V^T fragments from ds_read_b64_tr_b8
//                       converted exactly to fp16 (fp8 rows; the MFMA is the fp16 one),
//                       writes a request's output when its last tile is in, and streams the tiles
//                       global -> LDS by LDS-DMA, A tiles ahead of the score waves, into a ring of
//                       A+3 stages (each value wave waits only for its own loads).
// The workgroup meets once per tile at one barrier. Inside a step a wave issues all its LDS reads at
// once and waits for them in order with counted lgkmcnt waits, so the MFMAs start as soon as the
// first rows arrive.
//
// Softmax: every row keeps one reference max shared by its two score waves. P = exp2(s - ref) is
// written optimistically. One step later, when the barrier has made both halves' tile maxima
// visible, the score waves check whether some row's tile max exceeds its reference by more than
// SHIFT (or the row had none yet); if so they agree on the new reference, rewrite that tile's P and
// publish the factor by which the value waves rescale their accumulators before they use the tile
// (which they do one step later still, so the check needs no barrier of its own).
//
// Reference semantics: qwen_mla/ops/mla_decode_attention.py:297-586 (stage 1: tile loop, fp8
// dequant :451-463, rms divide :466-507, softmax :553-560, partial store :562-586).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "qmla.h"
#include "qmla_common.h"
#include "qmla_device.h"
#include "qmla_window.h"

namespace qmla {
namespace ws {

constexpr float SHIFT = 15.0f;    // P <= 2^15 before the reference max moves (fp16 P stays finite)
enum Role { SCORE, VALUE };

// Compile-time shape: EB cache element bytes (1 fp8, 2 bf16), RMS tail format, DCG latent columns
// per group, A tiles in flight ahead of the score waves, CPR 16-byte chunks staged per row, CAP tanh
// logit cap, RTR rms codes read transposed (query rows are the heads of one token), ISS who issues a
// tile's DMA and when: 0 the value waves after their step, 1 before it, 3 between issuing their
// LDS reads and waiting for them, 2 all eight waves (value waves before their step, score waves
// after theirs), G latent groups:
//   G 1  up to 32 query rows (2 row blocks); score wave (tb, u) scores row block u over all 576
//        columns, value wave v owns latent columns [128v, 128v+128) of every row;
//   G 2  (GLA) up to 48 rows per group (3 row blocks each); score wave (tb, u) scores the 3 row
//        blocks of group u over the group's 256 latent columns and the shared rope, value wave v
//        owns columns [128(v&1), +128) of group v>>1 for the group's rows. fp8 rows only.
template <int EB_, int RMS_, int DCG_, int A_, int CPR_, bool CAP_, bool RTR_, int ISS_, int G_>
struct WS {
  static constexpr int EB = EB_, RMS = RMS_, DCG = DCG_, A = A_, S = A_ + 3, CPR = CPR_;
  static constexpr bool CAP = CAP_, RTR = RTR_;
  static constexpr int ISS = ISS_, G = G_;
  static constexpr int DC = G * DCG;                  // latent columns of a row
  static constexpr int NRB = G == 1 ? 2 : 6;          // 16-row blocks of a request
  static constexpr int MBG = NRB / 2;                 // row blocks per score wave
  static constexpr int MBV = NRB / G;                 // row blocks per value wave (its group's)
  static constexpr int ROWS = 16 * NRB;
  static constexpr int VPG = 4 / G;                   // value waves per group
  static constexpr int NW = 8, NTHR = 64 * NW;
  static constexpr int NIW = ISS == 2 ? 8 : 4;        // waves sharing a tile's DMA instructions
  static constexpr int RB = 16 * CPR;                 // staged row bytes
  static constexpr int STAGE = TILE * RB;
  static constexpr int NCH = TILE * CPR;              // 16-byte chunks per tile
  static constexpr int NI = (NCH + 63) / 64;          // DMA instructions per tile
  static constexpr int DPW = (NI + NIW - 1) / NIW;    // ... per issuing wave (at most)
  static constexpr int KQ = (DCG + 64) / 32;          // k-steps of the score product (latent + rope 64)
  static constexpr int KP = KQ / 2;                   // 16-byte K reads per lane and tile
  static constexpr int VC = DCG / VPG;                // latent columns per value wave
  static constexpr int CB = VC / 16;
  static constexpr int RMS_EB = (RMS == QMLA_RMS_BF16 || RMS == QMLA_RMS_BF16_BYTES) ? 2 : 1;
  static constexpr int NCODE = RMS == QMLA_RMS_NONE ? 0 : (RTR && RMS_EB == 1) ? 1 : 4;   // rms reads
  static constexpr int NKR = KP * EB;                 // K reads of a score step
  static constexpr int NVR = CB * EB;                 // V reads of a value step
  static constexpr int PST = TILE * 2 + 16;           // P row stride in LDS (bytes)
  // P.V operands: fp8 rows run it in fp16 (every e4m3 value is exact in fp16, and P keeps 11
  // significant bits instead of bf16's 8, so its rounding before P.V is 8x smaller than the
  // reference's bf16 P); bf16 rows in bf16
  using PT = std::conditional_t<EB == 1, _Float16, __bf16>;
  using PX4 = std::conditional_t<EB == 1, f16x4, bf16x4>;
  using PX8 = std::conditional_t<EB == 1, f16x8, bf16x8>;
  static_assert(DCG % 64 == 0 && CPR * 16 >= (DC + 64) * EB, "row slice");
  static_assert(G == 1 || (G == 2 && EB == 1 && !RTR), "latent groups: fp8 rows, rms codes read per row");
  static_assert(A >= 2 && A * DPW < 64, "lookahead / vmcnt range");
  static_assert(EB == 2 || DCG % 128 == 0, "fp8 latent in 128-column MFMA blocks");
  static_assert(CPR == 37 || CPR == 38, "staged row layout of fp8 rows (lbyte)");
};

template <class C>
struct Smem {
  char kv[C::S][C::STAGE];
  alignas(16) char p[3][C::ROWS][C::PST];   // P (C::PT) of tiles g % 3
  alignas(16) int flag[3][C::G][4];         // [g % 3][group][row block of the group]: reference moved at tile g
  alignas(16) float tmax[2][2][C::ROWS];    // [g & 1][token block][row] tile max
  alignas(16) float alpha[3][C::ROWS];      // [g % 3][row] accumulator rescale at tile g
  alignas(16) float fin[2][2][2][C::ROWS];  // [piece & 1][max, sum][token block][row] of a finished request
  alignas(16) SegD seg[NSEG];
  alignas(16) int pid[PIDN];
  int win[4];                          // pieces, tiles, pages of the window; another window follows
};

// DMA instructions issuing wave d issues per tile (instructions d, d+NIW, ... < NI)
template <class C>
__device__ __forceinline__ constexpr int dpw(int d) { return (C::NI - d + C::NIW - 1) / C::NIW; }

// The whole range of this workgroup, seen from one role. All roles run the same window / tile /
// barrier sequence; only the work between the barriers differs, so each role keeps only its own
// registers live (score waves the query fragments, value waves the accumulators).
template <class C, int ROLE>
__device__ __forceinline__ void role_main(const KParams& p, Smem<C>& sm, float kscale, bool fixed, int lo,
                                          int hi, int b0, int c0, int wr, int hz, int& bad) {
  constexpr int NTHR = C::NTHR;
  constexpr bool F8 = C::EB == 1;
  constexpr int NB = C::DCG / 128;       // latent blocks of the fp8 product
  constexpr bool QS = ROLE == SCORE;
  constexpr bool ISSUER = ROLE == VALUE || C::ISS == 2;
  constexpr int ND = ISSUER ? C::DPW : 1;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tb = (w >> 1) & 1, su = w & 1;     // score wave: token block, row-block set
  const int sg = su * C::MBG / C::MBV;         // score wave: latent group of its row blocks
  const int vw = w & 3;                        // value wave
  const int vg = vw / C::VPG, vh = vw % C::VPG;   // value wave: group, column slice of the group
  const int dw = C::NIW == 8 ? w : vw;         // issuing wave: first DMA instruction of a tile
  const int ln16 = lane & 15, lg = lane >> 4;
  const int qrows = p.qrows, hpg = p.hpg;
  // the workgroup's heads of each group: hpw of them from h0 (head split hz of p.hsplit)
  const int hpw = hpg / p.hsplit, h0 = hz * hpw;
  const int nrows = qrows * hpw;               // rows per group
  const int P = p.page_size;
  const float c2b = p.sm_scale * kscale * kLog2e;
  // score wave: the lane's row in each of its row blocks (r indexes the workgroup's row arrays),
  // its verify token and head
  int r[C::MBG], jq[C::MBG], hd[C::MBG], rms_b[C::MBG];
  bool rok[C::MBG];
#pragma unroll
  for (int m = 0; m < C::MBG; ++m) {
    const int rb = su * C::MBG + m;
    const int rg = 16 * (rb - sg * C::MBV) + ln16;   // row within the group
    r[m] = 16 * rb + ln16;
    rok[m] = rg < nrows;
    jq[m] = rok[m] ? rg / hpw : 0;
    hd[m] = sg * hpg + h0 + (rok[m] ? rg - jq[m] * hpw : 0);
    rms_b[m] = p.rms_off_b + hd[m] * C::RMS_EB;
  }
  const bool contig = p.token_stride_b == C::RB;
  // per-lane read offsets within a stage (staged row layout: lbyte). Score wave: K row 16tb + ln16,
  // 16-byte half h of the lane group's 32 columns of each latent block (block b adds 128b bytes), and
  // its rope chunk; value wave: transposed V row 8lg + ln16/2, its 128 columns' latent block, chunks
  // 0..6 and 7 (the flip may wrap the last)
  uint32_t koff[2] = {0u, 0u}, kofr = 0u, vb0 = 0u, vb7 = 0u;
  if constexpr (ROLE == SCORE && C::EB == 1) {
    const int krow = 16 * tb + ln16, fk = lflip<C::CPR>(krow);
#pragma unroll
    for (int h = 0; h < 2; ++h)
      koff[h] = (uint32_t)(krow * C::RB + 16 * (sg * (C::DCG / 16) + ((2 * lg + h + fk) & 7)));
    kofr = (uint32_t)(krow * C::RB + 16 * (C::DC / 16 + ((lg + fk) & 3)));
  }
  if constexpr (ROLE == VALUE && C::EB == 1) {
    const int vr = 8 * lg + (ln16 >> 1), fv = lflip<C::CPR>(vr);
    const int c0 = (vg * C::DCG + C::VC * vh) / 16;
    vb0 = (uint32_t)(vr * C::RB + 16 * (c0 + fv) + 8 * (ln16 & 1));
    vb7 = (uint32_t)(vr * C::RB + 16 * (c0 + ((7 + fv) & 7)) + 8 * (ln16 & 1));
  }

  // ---- score wave: query fragments (fp8 cache: e4m3 hi/lo parts scaled per row by a power of two
  //      folded into c2; the latent in 128-column blocks, lane group lg holding columns
  //      128b + 32lg .. +32, the rope as two 16x16x32 k-steps over rope columns 16lg .. +16;
  //      bf16 cache: bf16, pair jj and lane group lg holding columns 64jj + 16lg .. +16) ----
  bf16x8 qf[!F8 && QS ? C::KQ : 1];
  i32x8 qh8[C::MBG][F8 && QS ? NB : 1], ql8[C::MBG][F8 && QS ? NB : 1];
  long qhr[C::MBG][2], qlr[C::MBG][2];
  bf16x8 qn[QS ? C::KQ : 1];   // the query of one row block of a request, loaded at its first tile
  // per row block: query scale, reference max, sum, own max / optimistic sum / scores (log2 domain,
  // masked) of the last scored tile, verify limit
  float c2[C::MBG], mref[C::MBG], lpart[C::MBG], tmp[C::MBG], ps_pend[C::MBG];
  f32x4 scp[C::MBG];
  int lim[C::MBG];
#pragma unroll
  for (int m = 0; m < C::MBG; ++m) {
    c2[m] = c2b;
    mref[m] = kNegInf;
    lpart[m] = 0.f;
    tmp[m] = kNegInf;
    ps_pend[m] = 0.f;
    scp[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    lim[m] = 0;
  }

  // query row block m of request req into qn (group-local latent columns, then the rope)
  auto load_q = [&](int req, int m) {
    const int row = req * qrows + jq[m];
    const __bf16* qnp = p.q_nope + (int64_t)row * p.qn_sr + (int64_t)hd[m] * p.qn_sh;
    const __bf16* qpp = p.q_pe + (int64_t)row * p.qp_sr + (int64_t)hd[m] * p.qp_sh;
#pragma unroll
    for (int k = 0; k < C::KQ; ++k) {
      const int col = !F8 ? 64 * (k >> 1) + 16 * lg + 8 * (k & 1)
                          : k < 4 * NB ? 128 * (k >> 2) + 32 * lg + 8 * (k & 3) : C::DCG + 16 * lg + 8 * (k - 4 * NB);
      bf16x8 v = load_q8(col < C::DCG ? qnp + col : qpp + (col - C::DCG), p.q_vec);
      if (!rok[m]) v = bf16x8{};
      qn[k] = v;
    }
  };
  // qn -> the MFMA operands of row block m
  auto set_q = [&](int m) {
    if constexpr (F8) {
      float mx = 0.f;
#pragma unroll
      for (int k = 0; k < C::KQ; ++k)
#pragma unroll
        for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf((float)qn[k][e]));
      mx = max_lg(mx);
      // |q| * qs in (112, 448]: e4m3 keeps 4 significant bits in hi and 4 more in lo
      const float ex = mx > 0.f ? fminf(floorf(fast_log2(224.0f / mx)), 126.0f) : 0.0f;
      const float qs = fast_exp2(ex);
      c2[m] = c2b * fast_exp2(-ex);
      int hq[2 * C::KQ], lq[2 * C::KQ];
#pragma unroll
      for (int k = 0; k < C::KQ; ++k) {
#pragma unroll
        for (int hw = 0; hw < 2; ++hw) {
          float v[4], rsd[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (float)qn[k][4 * hw + e] * qs;
          int hb = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], 0, false);
          hb = __builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], hb, true);
          rsd[0] = v[0] - __builtin_amdgcn_cvt_f32_fp8(hb, 0);
          rsd[1] = v[1] - __builtin_amdgcn_cvt_f32_fp8(hb, 1);
          rsd[2] = v[2] - __builtin_amdgcn_cvt_f32_fp8(hb, 2);
          rsd[3] = v[3] - __builtin_amdgcn_cvt_f32_fp8(hb, 3);
          int lb = __builtin_amdgcn_cvt_pk_fp8_f32(rsd[0], rsd[1], 0, false);
          lb = __builtin_amdgcn_cvt_pk_fp8_f32(rsd[2], rsd[3], lb, true);
          hq[2 * k + hw] = hb;
          lq[2 * k + hw] = lb;
        }
      }
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          qh8[m][b][e] = hq[8 * b + e];
          ql8[m][b][e] = lq[8 * b + e];
        }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        qhr[m][t] = __builtin_bit_cast(long, i32x2{hq[8 * NB + 2 * t], hq[8 * NB + 2 * t + 1]});
        qlr[m][t] = __builtin_bit_cast(long, i32x2{lq[8 * NB + 2 * t], lq[8 * NB + 2 * t + 1]});
      }
    } else {
#pragma unroll
      for (int k = 0; k < C::KQ; ++k) qf[k] = qn[k];
    }
  };

  // ---- value wave: accumulator of the group's rows (16mb + 4lg + i) x its columns VC*vh + 16cb + ln16 ----
  f32x4 acc[C::MBV][ROLE == VALUE ? C::CB : 1];
  auto zero_acc = [&]() {
#pragma unroll
    for (int mb = 0; mb < C::MBV; ++mb)
#pragma unroll
      for (int cb = 0; cb < (ROLE == VALUE ? C::CB : 1); ++cb) acc[mb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  };
  zero_acc();

  // ---- value wave DMA: instruction i = vw + 4j covers LDS chunks 64i .. 64i+63 of a stage: staged
  //      row q / CPR, position q % CPR, i.e. row chunk pos_chunk(position, flip of the row) ----
  uint32_t doff[ND];
  int drow[ND];
  if constexpr (ISSUER) {
#pragma unroll
    for (int j = 0; j < ND; ++j) {
      int q = (dw + C::NIW * j) * 64 + lane;
      q = q < C::NCH ? q : C::NCH - 1;
      const int rr = q / C::CPR, pp = q - rr * C::CPR;
      doff[j] = (uint32_t)(rr * C::RB + 16 * pos_chunk<C::CPR>(pp, lflip<C::CPR>(rr)));
      drow[j] = rr;
    }
  }
  const bool big = dpw<C>(dw) == C::DPW;

  // reads one piece descriptor (asm reads: no wait on the LDS-DMA in flight); its fields are
  // wave-uniform, so they live in scalar registers (the DMA's buffer resources are built from them)
  auto read_seg = [&](int k) {
    i32x4 a, b;
    if constexpr (C::G == 1) {
      a = ldsr128(&sm.seg[k].req);
      b = ldsr128(&sm.seg[k].nt);
      lds_wait_n<1>(a);
      lds_wait_n<0>(b);
    } else {
      ldsr128x2_drained(&sm.seg[k].req, &sm.seg[k].nt, a, b);
    }
    SegD d;
    d.req = __builtin_amdgcn_readfirstlane(a[0]);
    d.ta = __builtin_amdgcn_readfirstlane(a[1]);
    d.te = __builtin_amdgcn_readfirstlane(a[2]);
    d.L = __builtin_amdgcn_readfirstlane(a[3]);
    d.nt = __builtin_amdgcn_readfirstlane(b[0]);
    d.pf = __builtin_amdgcn_readfirstlane(b[1]);
    d.fl = __builtin_amdgcn_readfirstlane(b[2]);
    d.pad = 0;
    return d;
  };

  // score step helpers: reference check of the previous tile and its publication
  using PX4 = typename C::PX4;
  using PT = typename C::PT;
  auto fix_decide = [&](int m, float tpart, bool& rare, float& alpha_f, PX4& pk_fix) {
    const float gm = fmaxf(tmp[m], tpart);
    const bool ch = gm > mref[m] + SHIFT;
    rare = __builtin_amdgcn_ballot_w64(ch) != 0;
    if (!rare) {
      lpart[m] += ps_pend[m];
      return;
    }
    const float mn = ch ? gm : mref[m];
    alpha_f = ch ? (mref[m] == kNegInf ? 0.f : fast_exp2(mref[m] - mn)) : 1.0f;
    mref[m] = mn;
    const float mu = mref[m] == kNegInf ? 0.f : mref[m];
    float ps2 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float e = fast_exp2(scp[m][i] - mu);
      ps2 += e;
      pk_fix[i] = (PT)e;
    }
    lpart[m] = lpart[m] * alpha_f + ps2;
  };
  auto fix_publish = [&](int m, int g, bool rare, float alpha_f, const PX4& pk_fix) {
    const int pt = g % 3;
    if (rare) {
      *reinterpret_cast<PX4*>(&sm.p[pt][r[m]][(16 * tb + 4 * lg) * 2]) = pk_fix;
      if (tb == 0 && lg == 0) sm.alpha[pt][r[m]] = alpha_f;
    }
    if (tb == 0 && lane == 0) sm.flag[pt][sg][su * C::MBG + m - sg * C::MBV] = rare ? 1 : 0;
  };
  auto publish_fin = [&](int k, int m) {
    const float l = sum_lg(lpart[m]);
    if (lg == 0) {
      sm.fin[k & 1][0][tb][r[m]] = mref[m];
      sm.fin[k & 1][1][tb][r[m]] = l;
    }
  };
  // value wave: normalize and write the output of request req, whose sums are in fin[k & 1]
  auto finalize = [&](int k, int req, int fl) {
    const SegOut so = seg_out<C::DCG>(p, req, (fl & SEG_FINAL) != 0, wr);
    const int row0 = req * qrows;
#pragma unroll
    for (int mb = 0; mb < C::MBV; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rr = 16 * mb + 4 * lg + i;        // row within the group
        const int rw = 16 * C::MBV * vg + rr;       // row of the workgroup's arrays
        float m, l0, l1;
        if constexpr (C::G == 1) {
          m = ldsr32f(&sm.fin[k & 1][0][0][rw]);
          l0 = ldsr32f(&sm.fin[k & 1][1][0][rw]);
          l1 = ldsr32f(&sm.fin[k & 1][1][1][rw]);
          lds_wait_n<2>(m);
          lds_wait_n<1>(l0);
          lds_wait_n<0>(l1);
        } else {
          ldsr32f3_drained(&sm.fin[k & 1][0][0][rw], &sm.fin[k & 1][1][0][rw], &sm.fin[k & 1][1][1][rw], m, l0, l1);
        }
        if (rr >= nrows) continue;
        const float l = l0 + l1;
        const int jr = rr / hpw, h = vg * hpg + h0 + rr - jr * hpw;
        const float inv = inv_sum(kscale, l);   // fp8 values were accumulated unscaled
        const float lse_v = row_lse(m, l);
        const int col = C::VC * vh + ln16;
        if (so.final_out) {
          const int64_t ob = (int64_t)(row0 + jr) * p.o_sr + (int64_t)h * p.o_sh + col;
#pragma unroll
          for (int cb = 0; cb < C::CB; ++cb) store_out(p.out, p.out_dt, ob + 16 * cb, acc[mb][cb][i] * inv);
          if (vh == 0 && ln16 == 0 && p.lse) store_out(p.lse, p.lse_dt, (int64_t)(row0 + jr) * p.lse_sr + h, lse_v);
        } else if (so.plse && p.part_h) {
          _Float16* ob = reinterpret_cast<_Float16*>(so.po) + (int64_t)jr * so.po_sr + (int64_t)h * so.po_sh + col;
          const float invh = inv_sum(1.0f, l);
#pragma unroll
          for (int cb = 0; cb < C::CB; ++cb) ob[16 * cb] = (_Float16)(acc[mb][cb][i] * invh);
          if (vh == 0 && ln16 == 0) so.plse[(int64_t)jr * so.plse_sr + h] = lse_v;
        } else {
          float* ob = so.po + (int64_t)jr * so.po_sr + (int64_t)h * so.po_sh + col;
#pragma unroll
          for (int cb = 0; cb < C::CB; ++cb) ob[16 * cb] = acc[mb][cb][i] * inv;
          if (vh == 0 && ln16 == 0) {
            if (so.plse) so.plse[(int64_t)jr * so.plse_sr + h] = lse_v;
            else so.po[(int64_t)jr * so.po_sr + (int64_t)h * so.po_sh + C::DCG] = lse_v;
          }
        }
      }
    zero_acc();
  };

  // window planning cursor (wave 0 only): request, token, plan prefix of the request
  int cb = fixed ? (int)blockIdx.y : b0, ctok = 0, cp = c0;

  for (;;) {
    if (w == 0) plan_window<kPlanSwitchWs>(p, sm, fixed, lo, hi, cb, ctok, cp);
    __syncthreads();
    const int nseg = sm.win[0], ntot = sm.win[1], npg = sm.win[2], more = sm.win[3];
    if (nseg == 0) break;
    // page ids of the window: page f belongs to the last piece with pf <= f
    for (int f = tid; f < npg; f += NTHR) {
      int k0 = 0, k1 = nseg - 1;
      while (k0 < k1) {
        const int mid = (k0 + k1 + 1) >> 1;
        if (sm.seg[mid].pf <= f) k0 = mid;
        else k1 = mid - 1;
      }
      const SegD& d = sm.seg[k0];
      // a folded request reads the block-table row of its last verify row, as its length does
      sm.pid[f] = checked_page(p, p.bt[((int64_t)d.req * qrows + qrows - 1) * p.bt_stride + d.ta / P + (f - d.pf)],
                               bad);
    }
    __syncthreads();

    // ---- per-role cursors over the window's pieces ----
    // DMA (value waves): piece ki, tile ti, page cursor (window page index ipg, token offset ioff)
    int ki = 0, ti = 0, i_ta = 0, i_te = 0, i_nt = 0, i_pf = 0, ipg = 0, ioff = 0, pidv = 0;
    auto enter_i = [&]() {
      const SegD d = read_seg(ki);
      i_ta = d.ta;
      i_te = d.te;
      i_nt = d.nt;
      i_pf = d.pf;
      ipg = d.pf;
      ioff = d.ta % P;
    };
    // issues tile g (the cursor's) into ring stage g % S and advances the cursor
    // (pid_landed: the page id was read before the last barrier, so no LDS read issued since needs
    // to complete before it is used)
    auto issue = [&](int g, bool pid_landed) {
      const int tok0 = i_ta + ti * TILE;
      const int nvalid = i_te - tok0 < TILE ? i_te - tok0 : TILE;
      char* dst = sm.kv[g % C::S];
      if (contig && ioff + TILE <= P) {
        // the tile's rows are consecutive in one page; rows past the piece end read as zeros
        if (pid_landed) lds_wait_n<15>(pidv);
        else lds_wait_n<0>(pidv);
        const int pg = __builtin_amdgcn_readfirstlane(pidv);
        const char* base = p.kv + (int64_t)pg * p.page_stride_b + (int64_t)ioff * p.token_stride_b;
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(base, (uint32_t)(nvalid * C::RB));
#pragma unroll
        for (int j = 0; j < ND; ++j) {
          const int i = dw + C::NIW * j;
          if (i < C::NI && (i * 64 + 64 <= C::NCH || i * 64 + lane < C::NCH)) dma16_buf(rs, doff[j], dst + i * 1024);
        }
      } else {
        // per-lane page lookup; rows past the piece end repeat its last row
#pragma unroll
        for (int j = 0; j < ND; ++j) {
          const int i = dw + C::NIW * j;
          if (i < C::NI && (i * 64 + 64 <= C::NCH || i * 64 + lane < C::NCH)) {
            const int rr = drow[j] < nvalid ? drow[j] : nvalid - 1;
            const int tok = tok0 + rr;
            const int q = tok / P;
            int pg = ldsr32(&sm.pid[i_pf + q - i_ta / P]);
            lds_wait_n<0>(pg);
            const uint32_t cbo = doff[j] - (uint32_t)(drow[j] * C::RB);
            dma16(p.kv + (int64_t)pg * p.page_stride_b + (int64_t)(tok - q * P) * p.token_stride_b + cbo,
                  dst + i * 1024);
          }
        }
      }
      ioff += TILE;
      while (ioff >= P) {
        ioff -= P;
        ++ipg;
      }
      if (++ti == i_nt) {
        ti = 0;
        if (++ki < nseg) enter_i();
      }
      pidv = ldsr32(&sm.pid[ipg < npg ? ipg : npg - 1]);
    };
    // wait until tile t landed, with tiles t+1 .. last issued after it
    auto wait_tile = [&](int t, int last) {
      const int ahead = last - t;
      if (big) wait_tiles<C::DPW, C::A - 1>(ahead);
      else wait_tiles<(C::NI % C::NIW == 0 ? C::DPW : C::DPW - 1), C::A - 1>(ahead);
    };
    // score: piece ks, tile ts; value: piece kv, tile tv
    int ks = 0, ts = 0, s_ta = 0, s_nt = 0, s_fl = 0, fl_prev = 0;
    int kv = 0, tv = 0, v_req = 0, v_nt = 0, v_fl = 0;
    if constexpr (ROLE == VALUE) {
      const SegD d = read_seg(0);
      v_req = d.req;
      v_nt = d.nt;
      v_fl = d.fl;
    }
    if constexpr (ISSUER) {
      enter_i();
      pidv = ldsr32(&sm.pid[ipg]);
      // prologue: tiles 0 .. A-1 in flight, tile 0 landed
      for (int t = 0; t < C::A && t < ntot; ++t) issue(t, false);
      wait_tile(0, (C::A < ntot ? C::A : ntot) - 1);
    }
    lds_barrier();

    // iteration g: value waves issue tile g+A, wait for tile g+1 and take tile g-2; score waves fix
    // tile g-1 and score tile g
#pragma clang loop unroll(disable)
    for (int g = 0; g <= ntot + 1; ++g) {
      if constexpr (ROLE == SCORE) {
        if (g < ntot) {
          if (ts == 0) {
            const SegD d = read_seg(ks);
            s_ta = d.ta;
            s_nt = d.nt;
            s_fl = d.fl;
            if (d.fl & SEG_FIRST) {
              if constexpr (C::G == 1) {
                load_q(d.req, 0);   // in flight during the reads below, converted after them
              } else {
                // three row blocks: the query switches here, before this tile's reads (the previous
                // request's softmax state does not depend on the query or its scale)
#pragma unroll
                for (int m = 0; m < C::MBG; ++m) {
                  load_q(d.req, m);
                  set_q(m);
                }
              }
            }
#pragma unroll
            for (int m = 0; m < C::MBG; ++m) {
              const int lr = d.L - (qrows - 1 - jq[m]);
              lim[m] = rok[m] ? (lr < d.te ? lr : d.te) : 0;
            }
          }
          const char* kvs = sm.kv[g % C::S];
          const int tok0 = s_ta + ts * TILE;
          // ---- LDS reads, in this order: partner maxima of tile g-1, rms codes, K rows ----
          float tpart[C::MBG];   // unused at g == 0
#pragma unroll
          for (int m = 0; m < C::MBG; ++m) tpart[m] = ldsr32f(&sm.tmax[(g + 1) & 1][tb ^ 1][r[m]]);
          uint32_t code[C::MBG][4];
#pragma unroll
          for (int m = 0; m < C::MBG; ++m)
#pragma unroll
            for (int i = 0; i < 4; ++i) code[m][i] = 0u;
          i32x2 craw = {0, 0};
          if constexpr (C::RMS != QMLA_RMS_NONE) {
            if constexpr (C::RTR && C::RMS_EB == 1) {
              // tr_b8: lanes 2r', 2r'+1 of block lg supply token row 16tb + 4lg + (r' & 3); lane n gets head 16su + n
              const int rr = 16 * tb + 4 * lg + ((ln16 >> 1) & 3);
              craw = lds_read_tr8_async(kvs + lbyte<C::CPR>(rr, p.rms_off_b + 16 * su + 8 * (ln16 & 1)));
            } else {
#pragma unroll
              for (int m = 0; m < C::MBG; ++m)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                  const char* a = kvs + lbyte<C::CPR>(16 * tb + 4 * lg + i, rms_b[m]);
                  code[m][i] = C::RMS_EB == 1 ? ldsr8(a) : ldsr16(a);
                }
            }
          }
          i32x4 kr0[C::KP], kr1[C::EB == 2 ? C::KP : 1];
          if constexpr (F8) {
            // latent block b of the wave's group (halves h = 0, 1 at one base each), then the rope
            // after the whole latent
            const uint32_t sb = lds_addr(kvs);
            const uint32_t a0 = sb + koff[0], a1 = sb + koff[1];
            static_for<0, NB>([&](auto bc) {
              constexpr int b = decltype(bc)::value;
              kr0[2 * b] = ldsr128_at<128 * b>(a0);
              kr0[2 * b + 1] = ldsr128_at<128 * b>(a1);
            });
            kr0[2 * NB] = ldsr128_at<0>(sb + kofr);
          } else {
#pragma unroll
            for (int jj = 0; jj < C::KP; ++jj) {
              const int cbyte = (64 * jj + 16 * lg) * C::EB;
              kr0[jj] = ldsr128(kvs + lbyte<C::CPR>(16 * tb + ln16, cbyte));
              kr1[jj] = ldsr128(kvs + lbyte<C::CPR>(16 * tb + ln16, cbyte + 16));
            }
          }
          // ---- reference check of tile g-1 (its writes follow the score product); at the first
          //      tile of a request: publish the previous request's sums, switch the query ----
#pragma unroll
          for (int m = 0; m < C::MBG; ++m) lds_wait_n<cmin15(C::MBG * C::NCODE + C::NKR)>(tpart[m]);
          bool rare[C::MBG];
          float alpha_f[C::MBG];
          PX4 pk_fix[C::MBG];
#pragma unroll
          for (int m = 0; m < C::MBG; ++m) {
            rare[m] = false;
            alpha_f[m] = 1.0f;
            if (g >= 1) fix_decide(m, tpart[m], rare[m], alpha_f[m], pk_fix[m]);
          }
          if (ts == 0) {
            if (g >= 1 && (fl_prev & SEG_LAST)) {
#pragma unroll
              for (int m = 0; m < C::MBG; ++m) publish_fin(ks - 1, m);
            }
            if (s_fl & SEG_FIRST) {
#pragma unroll
              for (int m = 0; m < C::MBG; ++m) {
                mref[m] = kNegInf;
                lpart[m] = 0.f;
              }
              if constexpr (C::G == 1) set_q(0);
            }
          }
          // ---- S^T = K . Q^T as the K rows arrive ----
          f32x4 sc[C::MBG];
          if constexpr (C::G == 1) {
            f32x4 s2a = f32x4{0.f, 0.f, 0.f, 0.f}, s2b = s2a, s2c = s2a, s2d = s2a;
            static_for<0, C::KP>([&](auto jc) {
              constexpr int jj = decltype(jc)::value;
              if constexpr (F8) {
                if constexpr (jj < 2 * NB && (jj & 1)) {
                  // latent block jj/2: 32 bytes per lane from reads jj-1, jj
                  lds_wait_n<cmin15(C::KP - 1 - jj)>(kr0[jj]);
                  lds_wait_n<cmin15(C::KP - jj)>(kr0[jj - 1]);
                  const i32x8 ka = {kr0[jj - 1][0], kr0[jj - 1][1], kr0[jj - 1][2], kr0[jj - 1][3],
                                    kr0[jj][0], kr0[jj][1], kr0[jj][2], kr0[jj][3]};
                  s2a = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ka, qh8[0][jj >> 1], s2a, 0, 0, 0, 127, 0, 127);
                  s2b = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ka, ql8[0][jj >> 1], s2b, 0, 0, 0, 127, 0, 127);
                } else if constexpr (jj == 2 * NB) {
                  lds_wait_n<cmin15(C::KP - 1 - jj)>(kr0[jj]);
                  const long k0 = __builtin_bit_cast(long, i32x2{kr0[jj][0], kr0[jj][1]});
                  const long k1 = __builtin_bit_cast(long, i32x2{kr0[jj][2], kr0[jj][3]});
                  s2c = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(k0, qhr[0][0], s2c, 0, 0, 0);
                  s2d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(k0, qlr[0][0], s2d, 0, 0, 0);
                  s2c = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(k1, qhr[0][1], s2c, 0, 0, 0);
                  s2d = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(k1, qlr[0][1], s2d, 0, 0, 0);
                }
              } else {
                lds_wait_n<cmin15(2 * (C::KP - 1 - jj) + 1)>(kr0[jj]);
                lds_wait_n<cmin15(2 * (C::KP - 1 - jj))>(kr1[jj]);
                const bf16x8 ka = __builtin_bit_cast(bf16x8, kr0[jj]);
                const bf16x8 kb = __builtin_bit_cast(bf16x8, kr1[jj]);
                if constexpr (jj & 1) {
                  s2b = mfma16(ka, qf[2 * jj], s2b);
                  s2b = mfma16(kb, qf[2 * jj + 1], s2b);
                } else {
                  s2a = mfma16(ka, qf[2 * jj], s2a);
                  s2a = mfma16(kb, qf[2 * jj + 1], s2a);
                }
              }
            });
            sc[0] = (s2a + s2c) + (s2b + s2d);
          } else {
            // latent groups (fp8): per row block one 16x16x128 chain (hi and lo parts) and one
            // 16x16x32 chain for the rope; the row blocks' chains are independent of each other
            f32x4 sl[C::MBG], sr[C::MBG];
#pragma unroll
            for (int m = 0; m < C::MBG; ++m) sl[m] = sr[m] = f32x4{0.f, 0.f, 0.f, 0.f};
            static_for<0, C::KP>([&](auto jc) {
              constexpr int jj = decltype(jc)::value;
              if constexpr (jj < 2 * NB && (jj & 1)) {
                lds_wait_n<cmin15(C::KP - 1 - jj)>(kr0[jj]);
                lds_wait_n<cmin15(C::KP - jj)>(kr0[jj - 1]);
                const i32x8 ka = {kr0[jj - 1][0], kr0[jj - 1][1], kr0[jj - 1][2], kr0[jj - 1][3],
                                  kr0[jj][0], kr0[jj][1], kr0[jj][2], kr0[jj][3]};
#pragma unroll
                for (int m = 0; m < C::MBG; ++m)
                  sl[m] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ka, qh8[m][jj >> 1], sl[m], 0, 0, 0, 127, 0, 127);
#pragma unroll
                for (int m = 0; m < C::MBG; ++m)
                  sl[m] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ka, ql8[m][jj >> 1], sl[m], 0, 0, 0, 127, 0, 127);
              } else if constexpr (jj == 2 * NB) {
                lds_wait_n<cmin15(C::KP - 1 - jj)>(kr0[jj]);
                const long k0 = __builtin_bit_cast(long, i32x2{kr0[jj][0], kr0[jj][1]});
                const long k1 = __builtin_bit_cast(long, i32x2{kr0[jj][2], kr0[jj][3]});
#pragma unroll
                for (int m = 0; m < C::MBG; ++m) sr[m] = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(k0, qhr[m][0], sr[m], 0, 0, 0);
#pragma unroll
                for (int m = 0; m < C::MBG; ++m) sr[m] = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(k0, qlr[m][0], sr[m], 0, 0, 0);
#pragma unroll
                for (int m = 0; m < C::MBG; ++m) sr[m] = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(k1, qhr[m][1], sr[m], 0, 0, 0);
#pragma unroll
                for (int m = 0; m < C::MBG; ++m) sr[m] = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(k1, qlr[m][1], sr[m], 0, 0, 0);
              }
            });
#pragma unroll
            for (int m = 0; m < C::MBG; ++m) sc[m] = sl[m] + sr[m];
          }
          if constexpr (C::RMS != QMLA_RMS_NONE) {
            if constexpr (C::RTR && C::RMS_EB == 1) {
              lds_wait_n<0>(craw);   // landed before the K rows
#pragma unroll
              for (int i = 0; i < 4; ++i) code[0][i] = ((uint32_t)craw[0] >> (8 * i)) & 0xFF;
            } else {
#pragma unroll
              for (int m = 0; m < C::MBG; ++m)
#pragma unroll
                for (int i = 0; i < 4; ++i) lds_wait_n<0>(code[m][i]);
            }
          }
#pragma unroll
          for (int m = 0; m < C::MBG; ++m) {
            // ---- rms divide, scale, cap, mask ----
            float tm = kNegInf;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float rinv = 1.0f;
              if constexpr (C::RMS == QMLA_RMS_LOG8) {
                rinv = fast_exp2(fmaf((float)code[m][i], -6.0f / 255.0f, 3.0f));   // 1 / 2^(-3 + c*6/255)
              } else if constexpr (C::RMS == QMLA_RMS_E4M3) {
                const float rv = fp8_to_f32(code[m][i]) * kscale;
                rinv = rv > 0.f ? __builtin_amdgcn_rcpf(rv) : 1.0f;
              } else if constexpr (C::RMS == QMLA_RMS_BF16 || C::RMS == QMLA_RMS_BF16_BYTES) {
                const float rv = bf16_bits_to_f32(code[m][i]);
                rinv = rv > 0.f ? __builtin_amdgcn_rcpf(rv) : 1.0f;
              }
              float v;
              if constexpr (C::CAP) {
                const float sn = sc[m][i] * (c2[m] * kLn2) * rinv;
                const float th = 1.0f - 2.0f / (fast_exp2(2.0f * kLog2e * (sn / p.logit_cap)) + 1.0f);
                v = p.logit_cap * th * kLog2e;
              } else {
                v = sc[m][i] * c2[m] * rinv;
              }
              v = tok0 + 16 * tb + 4 * lg + i < lim[m] ? v : kNegInf;
              sc[m][i] = v;
              tm = fmaxf(tm, v);
            }
            tm = max_lg(tm);
            // ---- optimistic P against the current reference ----
            const float mu = mref[m] == kNegInf ? 0.f : mref[m];
            PX4 pk;
            float ps = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float e = fast_exp2(sc[m][i] - mu);
              ps += e;
              pk[i] = (PT)e;
            }
            *reinterpret_cast<PX4*>(&sm.p[g % 3][r[m]][(16 * tb + 4 * lg) * 2]) = pk;
            if (lg == 0) sm.tmax[g & 1][tb][r[m]] = tm;
            if (g >= 1) fix_publish(m, g - 1, rare[m], alpha_f[m], pk_fix[m]);
            scp[m] = sc[m];
            tmp[m] = tm;
            ps_pend[m] = ps;
          }
          if (++ts == s_nt) {
            ts = 0;
            fl_prev = s_fl;
            ++ks;
          }
        } else if (g == ntot) {
          // reference check of the window's last tile
          float tpart[C::MBG];
#pragma unroll
          for (int m = 0; m < C::MBG; ++m) tpart[m] = ldsr32f(&sm.tmax[(g + 1) & 1][tb ^ 1][r[m]]);
#pragma unroll
          for (int m = 0; m < C::MBG; ++m) {
            lds_wait_n<0>(tpart[m]);
            bool rare = false;
            float alpha_f = 1.0f;
            PX4 pk_fix;
            fix_decide(m, tpart[m], rare, alpha_f, pk_fix);
            fix_publish(m, g - 1, rare, alpha_f, pk_fix);
          }
          if (fl_prev & SEG_LAST) {
#pragma unroll
            for (int m = 0; m < C::MBG; ++m) publish_fin(ks - 1, m);
          }
        }
        if constexpr (C::ISS == 2) {
          if (g + C::A < ntot) issue(g + C::A, false);
          if (g + 1 < ntot) wait_tile(g + 1, g + C::A < ntot - 1 ? g + C::A : ntot - 1);
        }
      } else {
        if constexpr (C::ISS == 1 || C::ISS == 2) {
          if (g + C::A < ntot) issue(g + C::A, false);
        }
        // issuing value waves wait for the next tile before their P . V rather than after it (the
        // fp8 B 128 workload measured 0.6% faster so)
        if constexpr (C::ISS == 1) {
          if (g + 1 < ntot) wait_tile(g + 1, g + C::A < ntot - 1 ? g + C::A : ntot - 1);
        }
        // ---- P . V for tile j = g-2 over columns VC*vw .. +VC: reads first ----
        const int j = g - 2, pj = (g + 1) % 3;
        const int vr0 = 16 * C::MBV * vg;   // the group's first row in the workgroup's arrays
        i32x2 fl = {0, 0};                  // one group: the two row blocks' flags
        i32x4 fl4 = {0, 0, 0, 0};           // latent groups: the group's row blocks' flags
        i32x4 pr[C::MBV];
        i32x2 vraw[C::CB][C::EB];
        if (g >= 2) {
          const char* kvs = sm.kv[j % C::S];
          if constexpr (C::G == 1) fl = ldsr64(&sm.flag[pj][0][0]);
          else fl4 = ldsr128(&sm.flag[pj][vg][0]);
#pragma unroll
          for (int mb = 0; mb < C::MBV; ++mb) pr[mb] = ldsr128(&sm.p[pj][vr0 + 16 * mb + ln16][(8 * lg) * 2]);
          if constexpr (C::EB == 1) {
            // 16-column block cb of the wave's 128 columns: chunk position (cb + f) & 7 of their latent block
            const uint32_t a0 = lds_addr(kvs) + vb0, a7 = lds_addr(kvs) + vb7;
            static_for<0, C::CB>([&](auto cc) {
              constexpr int c = decltype(cc)::value;
              if constexpr (c < 7) vraw[c][0] = ldstr8_at<16 * c>(a0);
              else vraw[c][0] = ldstr8_at<0>(a7);
            });
          } else {
#pragma unroll
            for (int cb = 0; cb < C::CB; ++cb) {
              const int col0 = C::VC * vh + 16 * cb;
              const int vr = 8 * lg + (ln16 >> 2);
              const int vb = (col0 + 4 * (ln16 & 3)) * 2;
              vraw[cb][0] = lds_read_tr16_async(kvs + lbyte<C::CPR>(vr, vb));
              vraw[cb][C::EB - 1] = lds_read_tr16_async(kvs + lbyte<C::CPR>(vr + 4, vb));
            }
          }
        }
        // the DMA issue stalls while the memory pipeline is full: let the reads land meanwhile
        if constexpr (C::ISS == 3) {
          if (g + C::A < ntot) issue(g + C::A, true);
        }
        if (g >= 2) {
          int fm[C::MBV];
          if constexpr (C::G == 1) {
            lds_wait_n<cmin15(C::MBV + C::NVR)>(fl);
#pragma unroll
            for (int mb = 0; mb < C::MBV; ++mb) fm[mb] = __builtin_amdgcn_readfirstlane(fl[mb]);
          } else {
            lds_wait_n<cmin15(C::MBV + C::NVR)>(fl4);
#pragma unroll
            for (int mb = 0; mb < C::MBV; ++mb) fm[mb] = __builtin_amdgcn_readfirstlane(fl4[mb]);
          }
          int fany = 0;
#pragma unroll
          for (int mb = 0; mb < C::MBV; ++mb) fany |= fm[mb];
          if (fany) {
            // the reference of some row moved at tile j: rescale before adding it
            i32x4 ar[C::MBV];
#pragma unroll
            for (int mb = 0; mb < C::MBV; ++mb) ar[mb] = ldsr128(&sm.alpha[pj][vr0 + 16 * mb + 4 * lg]);
#pragma unroll
            for (int mb = 0; mb < C::MBV; ++mb) lds_wait_n<0>(ar[mb]);
#pragma unroll
            for (int mb = 0; mb < C::MBV; ++mb) {
              if (fm[mb] == 0) continue;
              const f32x4 al = __builtin_bit_cast(f32x4, ar[mb]);
#pragma unroll
              for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int cb = 0; cb < C::CB; ++cb) acc[mb][cb][i] *= al[i];
            }
          }
          using PX8 = typename C::PX8;
          PX8 pf[C::MBV];
#pragma unroll
          for (int mb = 0; mb < C::MBV; ++mb) {
            lds_wait_n<cmin15(C::NVR)>(pr[mb]);
            pf[mb] = __builtin_bit_cast(PX8, pr[mb]);
          }
          static_for<0, C::CB>([&](auto cc) {
            constexpr int cb = decltype(cc)::value;
            PX8 vf;
            if constexpr (C::EB == 1) {
              lds_wait_n<cmin15(C::CB - 1 - cb)>(vraw[cb][0]);
              vf = fp8x8_to_f16(vraw[cb][0]);
            } else {
              lds_wait_n<cmin15(2 * (C::CB - 1 - cb) + 1)>(vraw[cb][0]);
              lds_wait_n<cmin15(2 * (C::CB - 1 - cb))>(vraw[cb][1]);
              const i32x4 w4 = {vraw[cb][0][0], vraw[cb][0][1], vraw[cb][1][0], vraw[cb][1][1]};
              vf = __builtin_bit_cast(PX8, w4);
            }
#pragma unroll
            for (int mb = 0; mb < C::MBV; ++mb) acc[mb][cb] = mfma16(pf[mb], vf, acc[mb][cb]);
          });
          if (++tv == v_nt) {
            // the request's last tile: its sums were published at the previous step
            if (v_fl & SEG_LAST) finalize(kv, v_req, v_fl);
            tv = 0;
            if (++kv < nseg) {
              const SegD d = read_seg(kv);
              v_req = d.req;
              v_nt = d.nt;
              v_fl = d.fl;
            }
          }
        }
        if constexpr (C::ISS == 0) {
          if (g + C::A < ntot) issue(g + C::A, false);
        }
        if constexpr (C::ISS != 1) {
          if (g + 1 < ntot) wait_tile(g + 1, g + C::A < ntot - 1 ? g + C::A : ntot - 1);
        }
      }
      lds_barrier();
    }
    wait_vmcnt<0>();
    if (!more) break;
  }
}

template <class C>
__global__ __launch_bounds__(C::NTHR, 1) void ws_kernel(const KParams p) {
  static_assert(sizeof(Smem<C>) <= 163840, "LDS budget of a workgroup");
  __shared__ __attribute__((aligned(16))) Smem<C> sm;
  const float kscale = (C::EB == 1 && p.k_scale) ? *p.k_scale : 1.0f;
  const bool fixed = p.num_splits > 0;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // head split: the p.hsplit workgroups of one token range are consecutive on one XCD (workgroup i
  // runs on XCD i % 8), so their shared reads of the range's rows are served by that XCD's L2
  int hz = fixed ? (int)blockIdx.z : 0, wr = blockIdx.x;
  if (!fixed && p.hsplit > 1) {
    if ((p.nwg & 7) == 0) {
      const int slot = (int)blockIdx.x >> 3;
      hz = slot % p.hsplit;
      wr = (slot / p.hsplit) * 8 + ((int)blockIdx.x & 7);
    } else {   // a caller's range count: the split's workgroups are at least adjacent in launch order
      hz = (int)blockIdx.x % p.hsplit;
      wr = (int)blockIdx.x / p.hsplit;
    }
  }
  int lo = 0, hi = 0, b0 = 0, c0 = 0;
  if (!fixed) {
    if (wr == 0 && hz == 0 && wv == 1) store_plan<kPlanSwitchWs>(p);   // for the balanced combine
    const BalRange r = balanced_range<kPlanSwitchWs>(p, wr);
    lo = r.lo;
    hi = r.hi;
    b0 = r.b0;
    c0 = r.c0;
    if (lo >= hi) return;
  }
  int bad = 0;
  if (wv < 4) role_main<C, SCORE>(p, sm, kscale, fixed, lo, hi, b0, c0, wr, hz, bad);
  else role_main<C, VALUE>(p, sm, kscale, fixed, lo, hi, b0, c0, wr, hz, bad);
  report_pages(p, bad);
}

struct Inst {
  int eb, rms, dcg, cpr, g;
  bool cap, rtr;
  int nthr;
  void (*fn)(const KParams);
};

#define QMLA_WS(EB, RMS, DCG, A, CPR, CAP, RTR, ISS, G)                                   \
  {EB, RMS, DCG, CPR, G, CAP, RTR, WS<EB, RMS, DCG, A, CPR, CAP, RTR, ISS, G>::NTHR, \
   &ws_kernel<WS<EB, RMS, DCG, A, CPR, CAP, RTR, ISS, G>>}

static const Inst kInst[] = {
    // fp8 e4m3 + log8 codes, d_c 512, rope 64, 24 heads: 608-byte rows, 32-token tiles 3 ahead (6 stages)
    QMLA_WS(1, QMLA_RMS_LOG8, 512, 3, 38, false, true, 1, 1),
    QMLA_WS(1, QMLA_RMS_LOG8, 512, 3, 38, false, false, 1, 1),
    // ... up to 16 heads (592-byte rows), rms codes read per row
    QMLA_WS(1, QMLA_RMS_LOG8, 512, 3, 37, false, false, 1, 1),
    // (GLA-g2 on these rows runs in the row-owner kernel, qmla_ro.hip; the G = 2 form of this
    // template is kept but not instantiated)
};

}  // namespace ws

// Workgroups per token range for a request's rows: one group holds 32 rows (2 row blocks) per
// workgroup, so more rows split the heads over up to 4 workgroups (24 heads x 4 verify tokens: 3 of
// 8 heads x 4 tokens); latent groups (GLA) hold 48 rows per group in one workgroup. 0: no fit.
int ws_head_split(const qmla_decode_params* p) {
  const int hpg = p->heads / p->groups, rows = p->qrows * hpg;
  if (p->groups == 2) return rows <= 48 ? 1 : 0;
  if (p->groups != 1) return 0;
  for (int hs = 1; hs <= 4; ++hs)
    if (hpg % hs == 0 && p->qrows * (hpg / hs) <= 32) return hs;
  return 0;
}

// Instances past the warp-specialized table are the row-owner kernel's (qmla_ro.hip), which takes
// the GLA-g2 shapes it serves, and the wide-row warp-specialized kernel's (qmla_wsb.hip: bf16 rows,
// the deployed fp8 layouts).
constexpr int kRoBase = 1000, kWsbBase = 2000;

// the fp8 warp-specialized table's instance, or -1
static int ws_table_select(const qmla_decode_params* p) {
  if (p->rope_w != 64 || (p->groups != 1 && p->groups != 2)) return -1;
  const int hs = ws_head_split(p);
  if (hs == 0) return -1;
  const int eb = p->kv_dtype == QMLA_KV_FP8 ? 1 : 2;
  const bool cap = p->logit_cap > 0.f;
  const int64_t ts = p->token_stride * eb;
  for (int i = 0; i < (int)(sizeof(ws::kInst) / sizeof(ws::kInst[0])); ++i) {
    const ws::Inst& in = ws::kInst[i];
    if (in.g != p->groups || in.eb != eb || in.rms != p->rms_mode || in.dcg != p->d_c / p->groups || in.cap != cap)
      continue;
    if (in.rtr && (p->qrows != 1 || p->heads > 32 || hs != 1)) continue;
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

int ws_select(const qmla_decode_params* p) {
  if (!rows16(p)) return -1;
  const int ri = ro_select(p);
  if (ri >= 0) return kRoBase + ri;
  const int wi = ws_table_select(p);
  if (wi >= 0) return wi;
  const int bi = wsb_select(p);
  return bi >= 0 ? kWsbBase + bi : -1;
}

int ws_launch(int inst, const qmla_decode_params* p, const KParams& k, int nwg, hipStream_t st) {
  if (inst >= kWsbBase) return wsb_launch(inst - kWsbBase, p, k, nwg, st);
  if (inst >= kRoBase) return ro_launch(inst - kRoBase, p, k, nwg, st);
  KParams kk = k;
  kk.hsplit = ws_head_split(p);
  void* args[] = {&kk};
  dim3 grid = p->num_splits > 0 ? dim3(p->num_splits, k.n_req, kk.hsplit) : dim3(nwg * kk.hsplit, 1, 1);
  if (grid.x == 0 || grid.y == 0) return QMLA_OK;
  hipError_t e = hipLaunchKernel((const void*)ws::kInst[inst].fn, grid, dim3(ws::kInst[inst].nthr, 1, 1), args, 0, st);
  return e == hipSuccess ? QMLA_OK : QMLA_ERR_LAUNCH;
}

}  // namespace qmla
