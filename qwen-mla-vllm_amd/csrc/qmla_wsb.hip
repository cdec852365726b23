// qmla_wsb.hip -- gfx950 warp-specialized MLA decode of wide rows, <= 32 query rows per workgroup
// (24 heads, one token each; 24 heads x 4 verify tokens split over 3 workgroups of 8 heads):
//   bf16 rows: d_c 512, rope 64, one bf16 rms per head (or none): 1200 staged bytes;
//   fp8 rows (the plugin's deployed layouts): latent d_c 768 or 256, a partial rope of 232 columns
//   read as a 256-column window, one rms code per head: 1024 or 512 bytes.
//
// A workgroup owns a contiguous range of the concatenated requests' tokens (balanced mode) or one
// split of one request (fixed splits), with all of its query rows, and walks it as one sequence of
// 32-token tiles across request boundaries (the window walk of qmla_window.h). A 32-token tile of
// these rows is 32-37.5 KB, so the LDS holds a ring of four. That decides the split of the work: the
// softmax of a tile has to be final within the step that scores it, so the value waves can take the
// tile one step later and the ring needs only the tiles in flight, the one being scored and the one
// being accumulated (A + 2 stages).
//
// Its 6 waves take two roles:
//   score waves (4, 5): wave 4 + u owns 16 query rows (row block u) for all 32 tokens of a tile. It
//                       computes S^T = K . Q^T on MFMA with the query fragments resident in VGPRs and
//                       the K fragments read from the staged rows: bf16 rows on the 16x16x32 bf16
//                       MFMA; fp8 rows with their bytes as stored on the 16x16x128 fp8 MFMA, the
//                       query split per row into two e4m3 parts (hi + lo, 8 significant bits like
//                       bf16), the rope window's columns past the rope zeroed in K (they hold the rms
//                       codes). It divides by the rms, applies the mask, and runs the rows' online
//                       softmax entirely in its own registers (a
//                       row's tile max is a reduction over its 4 lane groups). The reference max moves
//                       only when a row's tile max exceeds it by more than ref_shift(the row's sum),
//                       so a dominant token gets P = 1 exactly and the bf16 rounding of P costs no
//                       more than in the reference; the wave then publishes the factor by which the
//                       value waves rescale their accumulators. P (bf16) goes to LDS. At a request's
//                       last tile it publishes the rows' max and sum;
//   value waves (0-3):  wave v accumulates P . V over latent columns [v d_c/4, (v+1) d_c/4) for all 32
//                       rows one tile behind the score waves, with V^T fragments read transposed from
//                       the staged rows (ds_read_b64_tr_b16; fp8 rows ds_read_b64_tr_b8, converted
//                       exactly to fp16, P in fp16), writes a request's output when its last tile is
//                       in, and streams the tiles global -> LDS by LDS-DMA, A tiles ahead of the
//                       score waves (each value wave waits only for its own loads).
// The two score waves sit on SIMDs 0 and 1 beside value waves 0 and 1 (waves are placed on SIMDs in
// order); SIMDs 2 and 3 hold one value wave each. The workgroup meets once per tile at one barrier.
// Inside a step a wave issues its LDS reads and waits for them in order with counted lgkmcnt waits.
// fp8 rows are 256 dwords (or 128) long, which puts every staged row on the same LDS banks: they are
// staged with each 16-byte chunk rotated inside its 256-byte region by the row index (chunk c of a
// region of row r at position (c + r) & 15), so the K reads of 16 consecutive rows and the
// transposed V reads of 8 consecutive rows land on distinct banks; 1200-byte bf16 rows need none.
//
// Reference semantics: qwen_mla/ops/mla_decode_attention.py:297-586 (stage 1: tile loop, fp8 dequant
// :451-463, rms divide :466-507, softmax :553-560, partial store :562-586); the deployed fp8 layouts
// (partial rope, rms codes after it) of qwen_mla/mla_impl.py:125-145, 261-271.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "qmla.h"
#include "qmla_common.h"
#include "qmla_device.h"
#include "qmla_window.h"

namespace qmla {
namespace wsb {
using namespace ws;   // TILE, NSEG, SegD, the counted LDS reads, plan_window, wait_tiles

constexpr float SHIFT_CAP = 8.0f;   // P = exp2(s - ref) <= 2^8 before a row's reference moves
constexpr int PIDB = 256;        // page ids per window (the ring leaves no room for more)
enum Role { SCORE, VALUE };

// Compile-time shape: EB cache element bytes (2 bf16, 1 fp8 e4m3), RMS tail format, DC latent
// columns, RW rope columns read as a window of WIN (the columns past RW are masked), CPR 16-byte
// chunks staged per row, A tiles in flight ahead of the score waves, CAP tanh logit cap, CP cache
// policy of the row loads (non-temporal, or the default for launches whose workgroups share a
// token range and read its rows from L2).
template <int EB_, int RMS_, int DC_, int RW_, int WIN_, int CPR_, int A_, bool CAP_, int CP_ = kCpolStream>
struct WB {
  static constexpr int EB = EB_, RMS = RMS_, DC = DC_, RW = RW_, WIN = WIN_, CPR = CPR_, A = A_, S = A_ + 2;
  static constexpr bool CAP = CAP_;
  static constexpr int CP = CP_;
  // fp8 rows are rotated inside whole 256-byte regions, and inside the 128-byte block that follows
  // them when the row has one (the rope window's last block of 896-byte rows); the rest is unrotated
  static constexpr bool ROT = EB == 1;
  static constexpr int FULL = CPR & ~15;                          // chunks in whole regions
  static constexpr int TAIL8 = (ROT && CPR - FULL >= 8) ? 8 : 0;  // rotated chunks past them
  static constexpr int RB = 16 * CPR, STAGE = TILE * RB;
  static constexpr int NW = 6, NTHR = 64 * NW;   // value waves 0-3, score waves 4-5
  static constexpr int ROWS = 32;
  static constexpr int NCH = TILE * CPR;          // 16-byte chunks per tile
  static constexpr int NI = (NCH + 63) / 64;      // DMA instructions per tile
  static constexpr int NIW = 4;                   // issuing waves
  static constexpr int DPW = (NI + NIW - 1) / NIW;
  // bf16 rows: 32-column k-steps of the score product (pairs: two 16-byte K reads per lane)
  static constexpr int KQ = EB == 2 ? (DC + WIN) / 32 : 1;
  static constexpr int KP = KQ / 2;
  // fp8 rows: 128-column blocks (latent, then the rope window); KW blocks of K reads in flight
  static constexpr int NBT = EB == 1 ? (DC + WIN) / 128 : 1;
  static constexpr int KW = 2;
  static constexpr int VC = DC / 4, CB = VC / 16; // columns per value wave, 16-column blocks
  static constexpr int PST = TILE * 2 + 16;       // P row stride in LDS (bytes)
  static constexpr int RMS_EB = (RMS == QMLA_RMS_BF16 || RMS == QMLA_RMS_BF16_BYTES) ? 2 : 1;
  // P and the P . V operands: fp16 for fp8 rows (every e4m3 value is exact in fp16, P keeps 11
  // significant bits), bf16 for bf16 rows
  using PT = std::conditional_t<EB == 1, _Float16, __bf16>;
  using PX4 = std::conditional_t<EB == 1, f16x4, bf16x4>;
  using PX8 = std::conditional_t<EB == 1, f16x8, bf16x8>;
  static_assert(EB == 1 || (RW == WIN && WIN % 64 == 0 && DC % 64 == 0 &&
                            (RMS == QMLA_RMS_NONE || RMS == QMLA_RMS_BF16) && CPR * 16 >= (DC + WIN) * 2),
                "bf16 rows: whole 64-column pairs, one bf16 rms per head or none");
  static_assert(EB == 2 || (DC % 128 == 0 && WIN % 128 == 0 && RW <= WIN && RW > WIN - 128 &&
                            (DC + WIN) / 16 <= FULL + TAIL8 && RMS != QMLA_RMS_NONE && RMS != QMLA_RMS_BF16),
                "fp8 rows: 128-column blocks inside the rotated chunks, rms codes after the rope");
  static_assert(DC % 64 == 0 && CB >= 1, "column split of the value waves");
  static_assert(A >= 2 && A * DPW < 64, "lookahead / vmcnt range");
};

// staged position (16-byte chunk) of chunk c of row r, and the inverse
template <class C>
__device__ __forceinline__ int stage_pos(int c, int r) {
  if (!C::ROT) return c;
  if (c < C::FULL) return (c & ~15) + ((c + r) & 15);
  if (c < C::FULL + C::TAIL8) return C::FULL + ((c - C::FULL + r) & 7);
  return c;
}
template <class C>
__device__ __forceinline__ int stage_chunk(int q, int r) {
  if (!C::ROT) return q;
  if (q < C::FULL) return (q & ~15) + ((q - r) & 15);
  if (q < C::FULL + C::TAIL8) return C::FULL + ((q - C::FULL - r) & 7);
  return q;
}

template <class C>
struct Smem {
  char kv[C::S][C::STAGE];
  alignas(16) char p[2][C::ROWS][C::PST];   // P (bf16) of tile g, at g & 1
  alignas(16) float alpha[2][C::ROWS];      // [g & 1][row] accumulator rescale at tile g
  alignas(16) float fin[2][2][C::ROWS];     // [piece & 1][max, sum][row] of a finished request
  alignas(16) int flag[2][4];               // [g & 1][row block]: its reference moved at tile g
  alignas(16) SegD seg[NSEG];
  alignas(16) int pid[PIDB];
  int win[4];
};

template <class C>
__device__ __forceinline__ constexpr int dpw(int d) { return (C::NI - d + C::NIW - 1) / C::NIW; }

// The whole range of this workgroup, seen from one role. All roles run the same window / tile /
// barrier sequence; each keeps only its own registers live.
template <class C, int ROLE>
__device__ __forceinline__ void role_main(const KParams& p, Smem<C>& sm, float kscale, bool fixed, int lo, int hi,
                                          int b0, int c0, int wr, int hz, int& bad) {
  constexpr int NTHR = C::NTHR;
  constexpr bool QS = ROLE == SCORE;
  constexpr bool F8 = C::EB == 1;
  constexpr int ND = QS ? 1 : C::DPW;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int su = w & 1;    // score wave: its row block
  const int vw = w & 3;    // value wave: its columns, its first DMA instruction of a tile
  const int ln16 = lane & 15, lg = lane >> 4;
  const int qrows = p.qrows;
  // the workgroup's heads: hpw of them from h0 (head split hz of p.hsplit)
  const int hpw = p.hpg / p.hsplit, h0 = hz * hpw;
  const int nrows = qrows * hpw;
  const int P = p.page_size;
  const int64_t tsb = p.token_stride_b;
  const float c2b = p.sm_scale * kscale * kLog2e;   // fp8 rows: the values are scaled by kscale
  // score wave: its row (verify token jq, head hd)
  const int rg = 16 * su + ln16;
  const bool rok = rg < nrows;
  const int jq = rok ? rg / hpw : 0;
  const int hd = h0 + (rok ? rg - jq * hpw : 0);

  // ---- score wave: query fragments. bf16 rows: pair jj and lane group lg hold columns
  //      64jj + 16lg .. +16 (k-step 2jj the first 8, 2jj + 1 the next 8). fp8 rows: block b and lane
  //      group lg hold columns 128b + 32lg .. +32 as e4m3 hi and lo parts of the query scaled by a
  //      power of two per row (undone in c2); rope columns past RW are zero ----
  bf16x8 qf[QS && !F8 ? C::KQ : 1];
  i32x8 qh8[QS && F8 ? C::NBT : 1], ql8[QS && F8 ? C::NBT : 1];
  float c2 = c2b;
  // 8 query columns from col (latent, then rope; rope columns past RW read as zero)
  auto q8 = [&](const __bf16* qnp, const __bf16* qpp, int col) {
    if (col < C::DC) return load_q8(qnp + col, p.q_vec);
    const int rc = col - C::DC;
    if (rc + 8 <= C::RW) return load_q8(qpp + rc, p.q_vec);
    bf16x8 v{};
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (rc + e < C::RW) v[e] = qpp[rc + e];
    return v;
  };
  auto load_q = [&](int req) {
    const int row = req * qrows + jq;
    const __bf16* qnp = p.q_nope + (int64_t)row * p.qn_sr + (int64_t)hd * p.qn_sh;
    const __bf16* qpp = p.q_pe + (int64_t)row * p.qp_sr + (int64_t)hd * p.qp_sh;
    if constexpr (!F8) {
#pragma unroll
      for (int k = 0; k < C::KQ; ++k) {
        bf16x8 v = q8(qnp, qpp, 64 * (k >> 1) + 16 * lg + 8 * (k & 1));
        if (!rok) v = bf16x8{};
        qf[k] = v;
      }
    } else {
      bf16x8 qn[4 * C::NBT];
#pragma unroll
      for (int k = 0; k < 4 * C::NBT; ++k) {
        qn[k] = q8(qnp, qpp, 128 * (k >> 2) + 32 * lg + 8 * (k & 3));
        if (!rok) qn[k] = bf16x8{};
      }
      float mx = 0.f;
#pragma unroll
      for (int k = 0; k < 4 * C::NBT; ++k)
#pragma unroll
        for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf((float)qn[k][e]));
      mx = max_lg(mx);
      // |q| * qs in (112, 448]: e4m3 keeps 4 significant bits in hi and 4 more in lo
      const float ex = mx > 0.f ? fminf(floorf(fast_log2(224.0f / mx)), 126.0f) : 0.0f;
      const float qs = fast_exp2(ex);
      c2 = c2b * fast_exp2(-ex);
      // each block's parts are built whole, so the previous request's parts die here
#pragma unroll
      for (int b = 0; b < C::NBT; ++b) {
        int hq[8], lq[8];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
#pragma unroll
          for (int hw = 0; hw < 2; ++hw) {
            float v[4], rsd[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = (float)qn[4 * b + k][4 * hw + e] * qs;
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
        qh8[b] = i32x8{hq[0], hq[1], hq[2], hq[3], hq[4], hq[5], hq[6], hq[7]};
        ql8[b] = i32x8{lq[0], lq[1], lq[2], lq[3], lq[4], lq[5], lq[6], lq[7]};
      }
    }
  };
  // fp8 rows: the K bytes of the last window block's columns past RW (the rms codes) are zeroed:
  // lane group lg keeps the first kvalid of its 32 bytes
  const int kvalid = F8 ? min(32, max(0, C::RW - (C::WIN - 128) - 32 * lg)) : 32;
  float mref = kNegInf, lpart = 0.f;   // the row's reference max (log2 domain) and partial sum
  int lim = 0;                          // the row's token limit in the current piece

  // ---- value wave: accumulator of rows 16mb + 4lg + i x columns VC*vw + 16cb + ln16 ----
  f32x4 acc[2][QS ? 1 : C::CB];
  auto zero_acc = [&]() {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int cb = 0; cb < (QS ? 1 : C::CB); ++cb) acc[mb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  };
  zero_acc();

  // ---- value wave DMA: instruction i = vw + 4j covers chunks 64i .. 64i+63 of a tile, staged in
  //      order (chunk q at LDS byte 16q: row q / CPR, 16-byte chunk q % CPR of the row) ----
  uint32_t goff[ND];
  int drow[ND];
  if constexpr (!QS) {
#pragma unroll
    for (int j = 0; j < ND; ++j) {
      int q = (vw + C::NIW * j) * 64 + lane;
      q = q < C::NCH ? q : C::NCH - 1;
      const int rr = q / C::CPR, pp = q - rr * C::CPR;
      goff[j] = (uint32_t)(rr * tsb + 16 * stage_chunk<C>(pp, rr));
      drow[j] = rr;
    }
  }
  const bool big = dpw<C>(vw) == C::DPW;
  // per-lane LDS offsets within a stage. Score wave: the rms of rows 4lg + i (+16tb); K row ln16
  // (+16tb): bf16 rows at byte 32lg of each 64-column pair, fp8 rows chunk 2lg + h of each block of
  // parity e. Value wave: transposed V reads of its 16-column blocks
  uint32_t coff[4] = {0u, 0u, 0u, 0u}, koff[2][2] = {{0u, 0u}, {0u, 0u}}, kofft[2] = {0u, 0u};
  uint32_t voff[QS ? 1 : C::CB];
  if constexpr (QS) {
    const int rb = p.rms_off_b + C::RMS_EB * hd;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rr = 4 * lg + i;
      coff[i] = (uint32_t)(rr * C::RB + 16 * stage_pos<C>(rb >> 4, rr) + (rb & 15));
    }
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        koff[e][h] = F8 ? (uint32_t)(ln16 * C::RB + 16 * stage_pos<C>(8 * e + 2 * lg + h, ln16))
                        : (uint32_t)(ln16 * C::RB + 32 * lg + 16 * h);
#pragma unroll
    for (int h = 0; h < 2; ++h)   // the block in the rotated 128-byte tail
      kofft[h] = (uint32_t)(ln16 * C::RB + 16 * stage_pos<C>(C::FULL + 2 * lg + h, ln16));
  } else {
    const int vr = F8 ? 8 * lg + (ln16 >> 1) : 8 * lg + (ln16 >> 2);
#pragma unroll
    for (int c = 0; c < C::CB; ++c) {
      const int col = C::VC * vw + 16 * c;
      voff[c] = F8 ? (uint32_t)(vr * C::RB + 16 * stage_pos<C>(col >> 4, vr) + 8 * (ln16 & 1))
                   : (uint32_t)(vr * C::RB + (col + 4 * (ln16 & 3)) * 2);
    }
  }

  // one piece descriptor (drained reads: its fields are wave-uniform and live in scalar registers)
  auto read_seg = [&](int k) {
    i32x4 a, b;
    ldsr128x2_drained(&sm.seg[k].req, &sm.seg[k].nt, a, b);
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

  // value wave: normalize and write the output of request req, whose sums are in fin[k & 1]
  auto finalize = [&](int k, int req, int fl) {
    const SegOut so = seg_out<C::DC>(p, req, (fl & SEG_FINAL) != 0, wr);
    const int row0 = req * qrows;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      i32x4 mr, lr;
      ldsr128x2_drained(&sm.fin[k & 1][0][16 * mb + 4 * lg], &sm.fin[k & 1][1][16 * mb + 4 * lg], mr, lr);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rr = 16 * mb + 4 * lg + i;
        if (rr >= nrows) continue;
        const float m = __int_as_float(mr[i]), l = __int_as_float(lr[i]);
        const int jr = rr / hpw, h = h0 + rr - jr * hpw;
        const float inv = inv_sum(kscale, l);   // fp8 values were accumulated unscaled
        const float lse_v = row_lse(m, l);
        const int col = C::VC * vw + ln16;
        if (so.final_out) {
          const int64_t ob = (int64_t)(row0 + jr) * p.o_sr + (int64_t)h * p.o_sh + col;
#pragma unroll
          for (int cb = 0; cb < C::CB; ++cb) store_out(p.out, p.out_dt, ob + 16 * cb, acc[mb][cb][i] * inv);
          if (vw == 0 && ln16 == 0 && p.lse) store_out(p.lse, p.lse_dt, (int64_t)(row0 + jr) * p.lse_sr + h, lse_v);
        } else if (so.plse && p.part_h) {
          // fp16 partials without the fp8 scale, which the combine applies
          _Float16* ob = reinterpret_cast<_Float16*>(so.po) + (int64_t)jr * so.po_sr + (int64_t)h * so.po_sh + col;
          const float invh = inv_sum(1.0f, l);
#pragma unroll
          for (int cb = 0; cb < C::CB; ++cb) ob[16 * cb] = (_Float16)(acc[mb][cb][i] * invh);
          if (vw == 0 && ln16 == 0) so.plse[(int64_t)jr * so.plse_sr + h] = lse_v;
        } else {
          float* ob = so.po + (int64_t)jr * so.po_sr + (int64_t)h * so.po_sh + col;
#pragma unroll
          for (int cb = 0; cb < C::CB; ++cb) ob[16 * cb] = acc[mb][cb][i] * inv;
          if (vw == 0 && ln16 == 0) {
            if (so.plse) so.plse[(int64_t)jr * so.plse_sr + h] = lse_v;
            else so.po[(int64_t)jr * so.po_sr + (int64_t)h * so.po_sh + C::DC] = lse_v;
          }
        }
      }
    }
    zero_acc();
  };

  // window planning cursor (wave 0 only): request, token, plan prefix of the request
  int cb = fixed ? (int)blockIdx.y : b0, ctok = 0, cp = c0;

  for (;;) {
    if (w == 0) plan_window<kPlanSwitchWs, PIDB>(p, sm, fixed, lo, hi, cb, ctok, cp);
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

    // ---- DMA cursor (value waves): piece ki, tile ti, window page index ipg, token offset ioff ----
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
    // issues tile g (the cursor's) into ring stage g % S and advances the cursor; pidv holds the
    // page id of the cursor's page, read at the previous issue (a barrier has drained it since)
    auto issue = [&](int g) {
      const int tok0 = i_ta + ti * TILE;
      const int nvalid = i_te - tok0 < TILE ? i_te - tok0 : TILE;
      char* dst = sm.kv[g % C::S];
      if (ioff + TILE <= P) {
        // the tile's rows are in one page; rows past the piece end read as zeros
        lds_wait_n<0>(pidv);
        const int pg = __builtin_amdgcn_readfirstlane(pidv);
        const char* base = p.kv + (int64_t)pg * p.page_stride_b + (int64_t)ioff * tsb;
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(base, (uint32_t)(nvalid * tsb));
#pragma unroll
        for (int j = 0; j < ND; ++j) {
          const int i = vw + C::NIW * j;
          if (i < C::NI && (i * 64 + 64 <= C::NCH || i * 64 + lane < C::NCH)) dma16_buf<C::CP>(rs, goff[j], dst + i * 1024);
        }
      } else {
        // per-lane page lookup; rows past the piece end repeat its last row
#pragma unroll
        for (int j = 0; j < ND; ++j) {
          const int i = vw + C::NIW * j;
          if (i < C::NI && (i * 64 + 64 <= C::NCH || i * 64 + lane < C::NCH)) {
            const int rr = drow[j] < nvalid ? drow[j] : nvalid - 1;
            const int tok = tok0 + rr;
            const int q = tok / P;
            int pg = ldsr32(&sm.pid[i_pf + q - i_ta / P]);
            lds_wait_n<0>(pg);
            const uint32_t cbo = goff[j] - (uint32_t)(drow[j] * tsb);
            dma16<C::CP>(p.kv + (int64_t)pg * p.page_stride_b + (int64_t)(tok - q * P) * tsb + cbo,
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
    int ks = 0, ts = 0, s_ta = 0, s_nt = 0, s_fl = 0;
    int kv = 0, tv = 0, v_req = 0, v_nt = 0, v_fl = 0;
    if constexpr (ROLE == VALUE) {
      const SegD d = read_seg(0);
      v_req = d.req;
      v_nt = d.nt;
      v_fl = d.fl;
      enter_i();
      pidv = ldsr32(&sm.pid[ipg]);
      lds_wait_n<0>(pidv);
      // prologue: tiles 0 .. A-1 in flight, tile 0 landed
      for (int t = 0; t < C::A && t < ntot; ++t) issue(t);
      wait_tile(0, (C::A < ntot ? C::A : ntot) - 1);
    }
    lds_barrier();

    // iteration g: value waves issue tile g+A, wait for tile g+1 and accumulate tile g-1; score
    // waves score tile g
#pragma clang loop unroll(disable)
    for (int g = 0; g <= ntot; ++g) {
      if constexpr (ROLE == SCORE) {
        if (g < ntot) {
          if (ts == 0) {
            const SegD d = read_seg(ks);
            s_ta = d.ta;
            s_nt = d.nt;
            s_fl = d.fl;
            if (d.fl & SEG_FIRST) {
              load_q(d.req);
              mref = kNegInf;
              lpart = 0.f;
            }
            const int lr = d.L - (qrows - 1 - jq);
            lim = rok ? (lr < d.te ? lr : d.te) : 0;
          }
          const uint32_t sb = lds_addr(sm.kv[g % C::S]);
          const int tok0 = s_ta + ts * TILE;
          // ---- LDS reads: rms of tokens 16tb + 4lg + i (head hd), then the K rows ----
          uint32_t code[2][4];
          if constexpr (C::RMS != QMLA_RMS_NONE) {
            static_for<0, 2>([&](auto tc) {
              constexpr int tb = decltype(tc)::value;
              static_for<0, 4>([&](auto ic) {
                constexpr int i = decltype(ic)::value;
                if constexpr (C::RMS_EB == 2) code[tb][i] = ldsr16_at<16 * tb * C::RB>(sb + coff[i]);
                else code[tb][i] = ldsr8_off<16 * tb * C::RB>(sb + coff[i]);
              });
            });
          }
          f32x4 sc[2];
          if constexpr (!F8) {
            // K row 16tb + ln16, columns 64jj + 16lg .. +8 and +8 .. +16
            const uint32_t ka = sb + koff[0][0];
            i32x4 kr[C::KQ];
            static_for<0, C::KP>([&](auto jc) {
              constexpr int jj = decltype(jc)::value;
              kr[2 * jj] = ldsr128_at<128 * jj>(ka);
              kr[2 * jj + 1] = ldsr128_at<128 * jj + 16>(ka);
            });
            // S^T = K . Q^T: token block 0 as its rows land, each of its reads followed by the same
            // read of token block 1, whose products run after
            f32x4 sa = f32x4{0.f, 0.f, 0.f, 0.f}, sbb = sa;
            i32x4 kq[C::KQ];
            static_for<0, C::KQ>([&](auto kc) {
              constexpr int kk = decltype(kc)::value;
              // issued after kr[kk]: reads kk+1 .. KQ-1 of block 0 and 0 .. kk-1 of block 1
              lds_wait_n<cmin15(C::KQ - 1)>(kr[kk]);
              if constexpr (kk & 1) sbb = mfma16(__builtin_bit_cast(bf16x8, kr[kk]), qf[kk], sbb);
              else sa = mfma16(__builtin_bit_cast(bf16x8, kr[kk]), qf[kk], sa);
              constexpr int jj = kk >> 1;
              kq[kk] = ldsr128_at<16 * C::RB + 128 * jj + 16 * (kk & 1)>(ka);
            });
            sc[0] = sa + sbb;
            sa = f32x4{0.f, 0.f, 0.f, 0.f};
            sbb = sa;
            static_for<0, C::KQ>([&](auto kc) {
              constexpr int kk = decltype(kc)::value;
              lds_wait_n<cmin15(C::KQ - 1 - kk)>(kq[kk]);
              if constexpr (kk & 1) sbb = mfma16(__builtin_bit_cast(bf16x8, kq[kk]), qf[kk], sbb);
              else sa = mfma16(__builtin_bit_cast(bf16x8, kq[kk]), qf[kk], sa);
            });
            sc[1] = sa + sbb;
          } else {
            // block b of K row 16tb + ln16: chunks 2lg, 2lg + 1 of its 256-byte region's half b & 1,
            // read KW blocks ahead of the products (both token blocks, hi and lo chains each)
            i32x4 kr[C::NBT][2][2];
            auto rd = [&](auto bc) {
              constexpr int b = decltype(bc)::value;
              if constexpr (8 * b < C::FULL) {
                const uint32_t a0 = sb + koff[b & 1][0], a1 = sb + koff[b & 1][1];
                kr[b][0][0] = ldsr128_at<256 * (b >> 1)>(a0);
                kr[b][0][1] = ldsr128_at<256 * (b >> 1)>(a1);
                kr[b][1][0] = ldsr128_at<16 * C::RB + 256 * (b >> 1)>(a0);
                kr[b][1][1] = ldsr128_at<16 * C::RB + 256 * (b >> 1)>(a1);
              } else {
                const uint32_t a0 = sb + kofft[0], a1 = sb + kofft[1];
                kr[b][0][0] = ldsr128_at<0>(a0);
                kr[b][0][1] = ldsr128_at<0>(a1);
                kr[b][1][0] = ldsr128_at<16 * C::RB>(a0);
                kr[b][1][1] = ldsr128_at<16 * C::RB>(a1);
              }
            };
            static_for<0, (C::KW < C::NBT ? C::KW : C::NBT)>(rd);
            f32x4 s0h = f32x4{0.f, 0.f, 0.f, 0.f}, s0l = s0h, s1h = s0h, s1l = s0h;
            static_for<0, C::NBT>([&](auto bc) {
              constexpr int b = decltype(bc)::value;
              constexpr int na = (C::KW - 1 < C::NBT - 1 - b ? C::KW - 1 : C::NBT - 1 - b);   // blocks issued after b
              lds_wait_n<cmin15(3 + 4 * na)>(kr[b][0][0]);
              lds_wait_n<cmin15(2 + 4 * na)>(kr[b][0][1]);
              lds_wait_n<cmin15(1 + 4 * na)>(kr[b][1][0]);
              lds_wait_n<cmin15(4 * na)>(kr[b][1][1]);
              i32x8 k0 = {kr[b][0][0][0], kr[b][0][0][1], kr[b][0][0][2], kr[b][0][0][3],
                          kr[b][0][1][0], kr[b][0][1][1], kr[b][0][1][2], kr[b][0][1][3]};
              i32x8 k1 = {kr[b][1][0][0], kr[b][1][0][1], kr[b][1][0][2], kr[b][1][0][3],
                          kr[b][1][1][0], kr[b][1][1][1], kr[b][1][1][2], kr[b][1][1][3]};
              if constexpr (b == C::NBT - 1 && C::RW < C::WIN) {
#pragma unroll
                for (int d = 0; d < 8; ++d) {
                  const int nb = kvalid - 4 * d;   // valid bytes of dword d
                  const uint32_t m = nb >= 4 ? 0xffffffffu : nb <= 0 ? 0u : (1u << (8 * nb)) - 1u;
                  k0[d] &= (int)m;
                  k1[d] &= (int)m;
                }
              }
              s0h = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(k0, qh8[b], s0h, 0, 0, 0, 127, 0, 127);
              s1h = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(k1, qh8[b], s1h, 0, 0, 0, 127, 0, 127);
              s0l = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(k0, ql8[b], s0l, 0, 0, 0, 127, 0, 127);
              s1l = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(k1, ql8[b], s1l, 0, 0, 0, 127, 0, 127);
              if constexpr (b + C::KW < C::NBT) rd(std::integral_constant<int, b + C::KW>{});
              // the block's products stay here: sunk past later reads they would keep every K
              // fragment of the tile live at once
              __builtin_amdgcn_sched_barrier(0);
            });
            sc[0] = s0h + s0l;
            sc[1] = s1h + s1l;
          }
          if constexpr (C::RMS != QMLA_RMS_NONE) {
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
              for (int i = 0; i < 4; ++i) lds_wait_n<0>(code[tb][i]);
          }
          // ---- rms divide, scale, cap, mask; the rows' tile max ----
          float tm = kNegInf;
#pragma unroll
          for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float rinv = 1.0f;
              if constexpr (C::RMS == QMLA_RMS_LOG8) {
                rinv = fast_exp2(fmaf((float)code[tb][i], -6.0f / 255.0f, 3.0f));   // 1 / 2^(-3 + c*6/255)
              } else if constexpr (C::RMS == QMLA_RMS_E4M3) {
                const float rv = fp8_to_f32(code[tb][i]) * kscale;
                rinv = rv > 0.f ? __builtin_amdgcn_rcpf(rv) : 1.0f;
              } else if constexpr (C::RMS == QMLA_RMS_BF16 || C::RMS == QMLA_RMS_BF16_BYTES) {
                const float rv = bf16_bits_to_f32(code[tb][i]);
                rinv = rv > 0.f ? __builtin_amdgcn_rcpf(rv) : 1.0f;
              }
              float v;
              if constexpr (C::CAP) {
                const float sn = sc[tb][i] * (c2 * kLn2) * rinv;
                const float th = 1.0f - 2.0f / (fast_exp2(2.0f * kLog2e * (sn / p.logit_cap)) + 1.0f);
                v = p.logit_cap * th * kLog2e;
              } else {
                v = sc[tb][i] * c2 * rinv;
              }
              v = tok0 + 16 * tb + 4 * lg + i < lim ? v : kNegInf;
              sc[tb][i] = v;
              tm = fmaxf(tm, v);
            }
          tm = max_lg(tm);
          // ---- the reference moves when a row's tile max exceeds it by more than the shift its
          //      running sum allows ----
          const bool ch = tm > mref + ref_shift(sum_lg(lpart), SHIFT_CAP);
          const bool rare = __builtin_amdgcn_ballot_w64(ch) != 0;
          if (rare) {
            const float mn = ch ? tm : mref;
            const float alpha_f = ch ? (mref == kNegInf ? 0.f : fast_exp2(mref - mn)) : 1.0f;
            mref = mn;
            lpart *= alpha_f;
            if (lg == 0) sm.alpha[g & 1][rg] = alpha_f;
          }
          if (lane == 0) sm.flag[g & 1][su] = rare ? 1 : 0;
          // ---- P against the reference ----
          const float mu = mref == kNegInf ? 0.f : mref;
          float ps = 0.f;
#pragma unroll
          for (int tb = 0; tb < 2; ++tb) {
            typename C::PX4 pk;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float e = fast_exp2(sc[tb][i] - mu);
              ps += e;
              pk[i] = (typename C::PT)e;
            }
            *reinterpret_cast<typename C::PX4*>(&sm.p[g & 1][rg][(16 * tb + 4 * lg) * 2]) = pk;
          }
          lpart += ps;
          if (++ts == s_nt) {
            // the piece's last tile: publish its rows' max and sum for the value waves
            if (s_fl & SEG_LAST) {
              const float l = sum_lg(lpart);
              if (lg == 0) {
                sm.fin[ks & 1][0][rg] = mref;
                sm.fin[ks & 1][1][rg] = l;
              }
            }
            ts = 0;
            ++ks;
          }
        }
      } else {
        if (g + C::A < ntot) issue(g + C::A);
        if (g + 1 < ntot) wait_tile(g + 1, g + C::A < ntot - 1 ? g + C::A : ntot - 1);
        if (g >= 1) {
          // ---- P . V of tile j = g - 1 over columns VC*vw .. +VC: reads first ----
          const int j = g - 1, pj = j & 1;
          const i32x2 fl = ldsr64(&sm.flag[pj][0]);
          i32x4 pr[2];
#pragma unroll
          for (int mb = 0; mb < 2; ++mb) pr[mb] = ldsr128(&sm.p[pj][16 * mb + ln16][16 * lg]);
          // V^T: lane (ln16, lg) gets column VC*vw + 16cb + ln16 of rows 8lg .. 8lg+7 (bf16 rows: two
          // reads of 4 rows each)
          constexpr int NVR = F8 ? 1 : 2;   // V reads per 16-column block
          const uint32_t sj = lds_addr(sm.kv[j % C::S]);
          i32x2 vraw[C::CB][NVR];
          static_for<0, C::CB>([&](auto cc) {
            constexpr int c = decltype(cc)::value;
            if constexpr (F8) {
              vraw[c][0] = ldstr8_at<0>(sj + voff[c]);
            } else {
              vraw[c][0] = ldstr16_at<0>(sj + voff[c]);
              vraw[c][NVR - 1] = ldstr16_at<4 * C::RB>(sj + voff[c]);
            }
          });
          i32x2 flw = fl;
          lds_wait_n<cmin15(2 + NVR * C::CB)>(flw);
          const int f0 = __builtin_amdgcn_readfirstlane(flw[0]), f1 = __builtin_amdgcn_readfirstlane(flw[1]);
          if (f0 | f1) {
            // some row's reference moved at tile j: rescale before adding it
            i32x4 ar[2];
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) ar[mb] = ldsr128(&sm.alpha[pj][16 * mb + 4 * lg]);
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) lds_wait_n<0>(ar[mb]);
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) {
              if ((mb == 0 ? f0 : f1) == 0) continue;
              const f32x4 al = __builtin_bit_cast(f32x4, ar[mb]);
#pragma unroll
              for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int cb = 0; cb < C::CB; ++cb) acc[mb][cb][i] *= al[i];
            }
          }
          using PX8 = typename C::PX8;
          PX8 pf[2];
          lds_wait_n<cmin15(1 + NVR * C::CB)>(pr[0]);
          lds_wait_n<cmin15(NVR * C::CB)>(pr[1]);
          pf[0] = __builtin_bit_cast(PX8, pr[0]);
          pf[1] = __builtin_bit_cast(PX8, pr[1]);
          static_for<0, C::CB>([&](auto cc) {
            constexpr int c = decltype(cc)::value;
            PX8 vf;
            if constexpr (F8) {
              lds_wait_n<cmin15(C::CB - 1 - c)>(vraw[c][0]);
              vf = fp8x8_to_f16(vraw[c][0]);
            } else {
              lds_wait_n<cmin15(2 * (C::CB - 1 - c) + 1)>(vraw[c][0]);
              lds_wait_n<cmin15(2 * (C::CB - 1 - c))>(vraw[c][NVR - 1]);
              const i32x4 w4 = {vraw[c][0][0], vraw[c][0][1], vraw[c][NVR - 1][0], vraw[c][NVR - 1][1]};
              vf = __builtin_bit_cast(PX8, w4);
            }
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) acc[mb][c] = mfma16(pf[mb], vf, acc[mb][c]);
          });
          if (++tv == v_nt) {
            // the request's last tile: its sums were published with it
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
      }
      lds_barrier();
    }
    wait_vmcnt<0>();
    if (!more) break;
  }
}

template <class C>
__global__ __launch_bounds__(C::NTHR, 1) void wsb_kernel(const KParams p) {
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
  if (wv >= 4) role_main<C, SCORE>(p, sm, kscale, fixed, lo, hi, b0, c0, wr, hz, bad);
  else role_main<C, VALUE>(p, sm, kscale, fixed, lo, hi, b0, c0, wr, hz, bad);
  report_pages(p, bad);
}

struct Inst {
  int eb, rms, dc, rw, cpr;
  bool cap, shared;   // shared: default cache policy, for launches whose ranges have several workgroups
  int nthr;
  void (*fn)(const KParams);
};

#define QMLA_WSB(EB, RMS, DC, RW, WIN, CPR, A, CAP)                                                        \
  {EB, RMS, DC, RW, CPR, CAP, false, WB<EB, RMS, DC, RW, WIN, CPR, A, CAP>::NTHR,                       \
   &wsb_kernel<WB<EB, RMS, DC, RW, WIN, CPR, A, CAP>>}
#define QMLA_WSB_SHARED(EB, RMS, DC, RW, WIN, CPR, A, CAP)                                                 \
  {EB, RMS, DC, RW, CPR, CAP, true, WB<EB, RMS, DC, RW, WIN, CPR, A, CAP, kCpolDefault>::NTHR,          \
   &wsb_kernel<WB<EB, RMS, DC, RW, WIN, CPR, A, CAP, kCpolDefault>>}

static const Inst kInst[] = {
    // bf16 rows [latent 512 | rope 64 | 24 bf16 rms]: 1200 bytes staged, 2 tiles ahead (4 stages)
    QMLA_WSB(2, QMLA_RMS_BF16, 512, 64, 64, 75, 2, false),
    QMLA_WSB(2, QMLA_RMS_BF16, 512, 64, 64, 75, 2, true),
    // ... without an rms tail: 1152 bytes
    QMLA_WSB(2, QMLA_RMS_NONE, 512, 64, 64, 72, 2, false),
    // the plugin's fp8 rows at TP 1 (24 heads): rank 768 [latent | rope 232 | 24 codes] = 1024 bytes,
    // 2 tiles ahead (4 stages, 128 KB); rank 256: 512 bytes, 4 ahead
    QMLA_WSB(1, QMLA_RMS_LOG8, 768, 232, 256, 64, 2, false),
    QMLA_WSB(1, QMLA_RMS_E4M3, 768, 232, 256, 64, 2, false),
    QMLA_WSB(1, QMLA_RMS_BF16_BYTES, 768, 232, 256, 66, 2, false),
    QMLA_WSB(1, QMLA_RMS_LOG8, 256, 232, 256, 32, 4, false),
    QMLA_WSB(1, QMLA_RMS_E4M3, 256, 232, 256, 32, 4, false),
    QMLA_WSB(1, QMLA_RMS_BF16_BYTES, 256, 232, 256, 34, 4, false),
    // ... at TP 2 (12 heads): rope 116 in a 128-column window; rank 768 [latent | rope | 12 codes] =
    // 896 bytes, rank 256 384 bytes
    QMLA_WSB(1, QMLA_RMS_LOG8, 768, 116, 128, 56, 2, false),
    QMLA_WSB(1, QMLA_RMS_E4M3, 768, 116, 128, 56, 2, false),
    QMLA_WSB(1, QMLA_RMS_BF16_BYTES, 768, 116, 128, 57, 2, false),
    QMLA_WSB(1, QMLA_RMS_LOG8, 256, 116, 128, 24, 4, false),
    QMLA_WSB(1, QMLA_RMS_E4M3, 256, 116, 128, 24, 4, false),
    QMLA_WSB(1, QMLA_RMS_BF16_BYTES, 256, 116, 128, 25, 4, false),
    // verify rows (a request's heads over several workgroups reading the same token range): the
    // default cache policy keeps the rows in L2 for the range's other workgroups
    QMLA_WSB_SHARED(2, QMLA_RMS_BF16, 512, 64, 64, 75, 2, false),
    QMLA_WSB_SHARED(1, QMLA_RMS_LOG8, 768, 232, 256, 64, 2, false),
};

}  // namespace wsb

// A compiled instance for these rows (one latent group) whose query rows fit a workgroup (the
// warp-specialized head split), or -1.
int wsb_select(const qmla_decode_params* p) {
  if (p->groups != 1 || ws_head_split(p) == 0) return -1;
  const int eb = p->kv_dtype == QMLA_KV_FP8 ? 1 : 2;
  const bool cap = p->logit_cap > 0.f;
  const int64_t ts = p->token_stride * eb;
  const bool shared = ws_head_split(p) > 1;
  int pick = -1;
  for (int i = 0; i < (int)(sizeof(wsb::kInst) / sizeof(wsb::kInst[0])); ++i) {
    const wsb::Inst& in = wsb::kInst[i];
    if (in.eb != eb || in.rms != p->rms_mode || in.dc != p->d_c || in.rw != p->rope_w || in.cap != cap) continue;
    if ((int64_t)in.cpr * 16 > ts) continue;   // never read past a row
    if (p->rms_mode != QMLA_RMS_NONE) {
      const int rb = (p->rms_mode == QMLA_RMS_BF16 || p->rms_mode == QMLA_RMS_BF16_BYTES) ? 2 : 1;
      const int64_t roff = (int64_t)p->rms_offset * eb;
      if (roff + (int64_t)p->heads * rb > in.cpr * 16) continue;   // every head's rms is staged
      if (roff < (int64_t)(in.dc + in.rw) * eb) continue;          // the rms follows the rope
    }
    if (in.shared == shared) return i;   // the policy that fits the launch, else any
    if (pick < 0) pick = i;
  }
  return pick;
}

int wsb_launch(int inst, const qmla_decode_params* p, const KParams& k, int nwg, hipStream_t st) {
  KParams kk = k;
  kk.hsplit = ws_head_split(p);
  void* args[] = {&kk};
  dim3 grid = p->num_splits > 0 ? dim3(p->num_splits, k.n_req, kk.hsplit) : dim3(nwg * kk.hsplit, 1, 1);
  if (grid.x == 0 || grid.y == 0) return QMLA_OK;
  hipError_t e =
      hipLaunchKernel((const void*)wsb::kInst[inst].fn, grid, dim3(wsb::kInst[inst].nthr, 1, 1), args, 0, st);
  return e == hipSuccess ? QMLA_OK : QMLA_ERR_LAUNCH;
}

}  // namespace qmla
