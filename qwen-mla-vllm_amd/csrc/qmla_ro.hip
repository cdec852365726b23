// qmla_ro.hip -- gfx950 row-owner MLA decode for GLA-g2: two latent groups of 256 columns, rope 64,
// fp8 e4m3 rows with log8 rms codes, up to 48 query rows per group (12 heads x 4 verify tokens).
//
// A workgroup walks its token range (balanced plan or one fixed split) as one sequence of 32-token
// tiles over pieces, like the warp-specialized kernel (qmla_ws.hip), but the work inside a tile is
// split by query rows, not by role:
//   compute waves (0-5): wave (group, row block) owns 16 query rows of one latent group for every
//                        token of the tile. It scores them (S^T = K . Q^T on the fp8 MFMAs, the query
//                        as e4m3 hi + lo parts resident in VGPRs, the K bytes as stored), divides by
//                        the rms, keeps the rows' online softmax in its own registers and accumulates
//                        P . V over the group's 256 latent columns (fp16 MFMA; P stays in the score
//                        registers and V comes from LDS already as fp16 operands in the score
//                        registers' token order). No other wave takes part in a row, so a tile needs
//                        no exchange of maxima or P through LDS;
//   DMA waves (6-7):     wave h streams rows 16h..16h+15 of every tile global -> LDS with LDS-DMA,
//                        A tiles ahead, into a ring of A+1 stages, waiting only for its own loads;
//                        once its half of the next tile is in, it converts that half's V (both
//                        groups) to fp16 MFMA operands in a second, double-buffered area. The three
//                        compute waves of a group would each convert the same V; this way it is done
//                        once, on the SIMDs that hold one compute wave instead of two.
// The workgroup meets once per tile at one barrier (the ring stage of tile g is refilled after it).
// Rows are ordered head-major within a group (row = head * qrows + verify token).
//
// Staged rows keep each 16-byte chunk inside its region (four latent blocks of 8 chunks, the rope's
// 4, the rms codes' 2), rotated there by f(r) = ((r >> 3) + (r >> 4)) & 1. With 608-byte rows (152
// dwords, 24 banks apart) that keeps the K reads (16 consecutive rows) and the transposed V reads
// (8 consecutive rows) on distinct banks, and a lane's reads of every latent block share one base
// register: the block and chunk go into the offset fields. A stage is two halves of 16 rows, each
// padded to whole DMA instructions, so each DMA wave's loads hold exactly its half.
//
// Reference semantics: qwen_mla/ops/mla_decode_attention.py:297-586 (stage 1: fp8 dequant :451-463,
// rms divide :466-507, online softmax :553-560, partial store :562-586), with the GLA-g2 head-to-group
// mapping of qwen_mla/mla_impl.py:182-194 (group g's heads read only its latent columns).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qmla.h"
#include "qmla_common.h"
#include "qmla_device.h"
#include "qmla_window.h"

namespace qmla {
namespace ro {
using namespace ws;

constexpr float SHIFT = 15.0f;   // P = exp2(s - ref) <= 2^15 (fp16) before a row's reference moves
enum Role { COMPUTE, DMA };

// A tiles in flight ahead of the compute waves (ring of A + 1 stages); QUAD: 4 verify rows per head,
// whose lanes 4k..4k+3 share each rms code through a DPP broadcast.
template <int A_, bool QUAD_>
struct RO {
  static constexpr bool QUAD = QUAD_;
  static constexpr int DCG = 256, G = 2, DC = G * DCG;   // latent columns per group, of a row
  static constexpr int NB = DCG / 128;                   // 128-column blocks of the fp8 product
  static constexpr int A = A_, S = A_ + 1;
  static constexpr int CPR = 38, RB = 16 * CPR;   // 608-byte rows
  // a stage holds two halves of 16 rows, each padded to whole DMA instructions (640 chunks)
  static constexpr int HCH = 640, HALF = 16 * HCH, STAGE = 2 * HALF;
  static constexpr int NW = 8, NTHR = 64 * NW, NCW = 6, NDW = 2;
  static constexpr int NRB = 3;                          // row blocks per group (48 rows)
  static constexpr int NI = 2 * HCH / 64;                // DMA instructions per tile
  static constexpr int DPW = NI / NDW;                   // ... per DMA wave: its half's 16 rows
  static constexpr int NBQ = NB + 1;                     // ... and the rope as one more
  static constexpr int KPT = 2 * NBQ;                    // 16-byte K reads per lane and token block
  static constexpr int KQ = 4 * NBQ;                     // query loads (8 bf16) per lane
  static constexpr int CB = DCG / 16;                    // 16-column output blocks per wave
  static_assert(CPR * 16 >= DC + 64 + 24, "row slice: latent, rope, 24 log8 codes");
  static_assert(A >= 2 && A * DPW < 64, "lookahead / vmcnt range");
  static_assert(CPR == 38, "row regions: 4 latent blocks of 8 chunks, rope 4, rms 2");
};

template <class C>
struct Smem {
  char kv[C::S][C::STAGE];
  // V of a tile as fp16 MFMA B operands: [tile parity][group][16-column block][lane], 8 values each
  // (bytes 0-7 from the tile's first 16 rows, 8-15 from the second)
  alignas(16) char vh[2][C::G][C::CB][64][16];
  alignas(16) SegD seg[NSEG];
  alignas(16) int pid[PIDN];
  int win[4];
};

// Chunk rotation of staged row r (chunk_pos / pos_chunk of the shared row layout): odd rows shift
// their chunks by one inside each region. A ds_read_b128 is served 32 lanes at a time over 128
// banks here (measured: 16 rows of 608 bytes x two 16-byte chunks two apart run at 32 cycles per
// read and wave with four waves, contiguous lanes at 25), and with this rotation the compute
// waves' K reads (16 rows x the chunks of two lane groups per 32 lanes) fill the 128 banks once
__device__ __forceinline__ int rflip(int r) { return r & 1; }

// byte offset of staged row r in a stage (two halves of 16 rows)
template <class C>
__device__ __forceinline__ int rowoff(int r) {
  return (r >> 4) * C::HALF + (r & 15) * C::RB;
}

template <int OFF>
__device__ __forceinline__ void ldsw64_at(uint32_t a, const i32x2& v) {
  asm volatile("ds_write_b64 %0, %1 offset:%2" : : "v"(a), "v"(v), "n"(OFF));
}

// lane 4k + I's value, to the 4 lanes 4k .. 4k+3 (every lane is written: no old value)
template <int I>
__device__ __forceinline__ float quad_bcast(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), I | (I << 2) | (I << 4) | (I << 6), 0xF, 0xF, true));
}

template <class C, int ROLE>
__device__ __forceinline__ void role_main(const KParams& p, Smem<C>& sm, float kscale, bool fixed, int lo,
                                          int hi, int b0, int c0, int wr, int& bad) {
  constexpr int NTHR = C::NTHR;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln16 = lane & 15, lg = lane >> 4;
  const int qrows = p.qrows, hpg = p.hpg;
  const int nrows = qrows * hpg;   // rows per group
  const int P = p.page_size;

  // ---- compute wave: group grp, row block rbk; the lane's score row rg (head-major) ----
  const int grp = w / C::NRB, rbk = w % C::NRB;
  const int rg = 16 * rbk + ln16;
  const bool rok = ROLE == COMPUTE && rg < nrows;
  const int jq = rok ? rg % qrows : 0, hl = rok ? rg / qrows : 0;
  const int head = grp * hpg + hl;
  const int rms_b = p.rms_off_b + head;
  const bool live = ROLE == COMPUTE && 16 * rbk < nrows;   // the wave has rows
  const float c2b = p.sm_scale * kscale * kLog2e;

  i32x8 qh8[ROLE == COMPUTE ? C::NBQ : 1], ql8[ROLE == COMPUTE ? C::NB : 1];
  int qsc = 127;   // E8M0 scale of the row's query parts: 2^-e
  // rms multiplier |c2b| / rms = 2^(lc2 - code*6/255); the sign of c2b goes into the query
  const float lc2 = 3.0f + fast_log2(c2b != 0.f ? fabsf(c2b) : 1.0f);
  const float qsign = c2b > 0.f ? 1.0f : c2b < 0.f ? -1.0f : 0.0f;
  float mref = kNegInf, lpart = 0.f;
  f32x4 acc[ROLE == COMPUTE ? C::CB : 1];
#pragma unroll
  for (int cb = 0; cb < (ROLE == COMPUTE ? C::CB : 1); ++cb) acc[cb] = f32x4{0.f, 0.f, 0.f, 0.f};

  // the query of row rg of request req as fp8 MFMA operands in 128-column blocks (lane group lg
  // holding columns 128b + 32lg .. +32), as e4m3 hi + lo parts of q * 2^e (|q| * 2^e in (112, 448];
  // the MFMA's B scale 2^-e undoes the shift): the group's latent blocks (a hi and a lo MFMA each),
  // then the rope as one block whose lane groups 0, 1 hold the hi parts of rope columns 32lg .. +32
  // and lane groups 2, 3 the lo parts of the same columns (their K reads repeat lane groups 0, 1's),
  // so one MFMA takes both
  auto load_q = [&](int req) {
    const int row = req * qrows + jq;
    const __bf16* qnp = p.q_nope + (int64_t)row * p.qn_sr + (int64_t)head * p.qn_sh;
    const __bf16* qpp = p.q_pe + (int64_t)row * p.qp_sr + (int64_t)head * p.qp_sh;
    bf16x8 qn[C::KQ];
#pragma unroll
    for (int k = 0; k < C::KQ; ++k) {
      const bool rope = k >= 4 * C::NB;
      const int col = rope ? 32 * (lg & 1) + 8 * (k & 3) : 128 * (k >> 2) + 32 * lg + 8 * (k & 3);
      bf16x8 v = bf16x8{};
      if (rok) v = load_q8(rope ? qpp + col : qnp + col, p.q_vec);
      qn[k] = v;
    }
    float mx = 0.f;
#pragma unroll
    for (int k = 0; k < C::KQ; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf((float)qn[k][e]));
    mx = max_lg(mx);
    const float ex = mx > 0.f ? fminf(floorf(fast_log2(224.0f / mx)), 126.0f) : 0.0f;
    const float qs = fast_exp2(ex) * qsign;
    qsc = 127 - (int)ex;
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
    for (int b = 0; b < C::NB; ++b)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        qh8[b][e] = hq[8 * b + e];
        ql8[b][e] = lq[8 * b + e];
      }
#pragma unroll
    for (int e = 0; e < 8; ++e) qh8[C::NB][e] = lg < 2 ? hq[8 * C::NB + e] : lq[8 * C::NB + e];
  };

  // normalize and write the rows of request req (accumulator row 16rbk + 4lg + i on this lane)
  auto finalize = [&](int req, int fl) {
    const SegOut so = seg_out<C::DCG>(p, req, (fl & SEG_FINAL) != 0, wr);
    const float l = sum_lg(lpart);
    const float inv = inv_sum(kscale, l);   // fp8 values were accumulated unscaled
    const float invh = inv_sum(1.0f, l);    // ... and are stored so as fp16 partials
    const float lse_v = row_lse(mref, l);
    const int row0 = req * qrows;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float inv_i = __shfl(inv, 4 * lg + i, 64);   // row 4lg+i's values sit on lane 4lg+i
      const int ri = 16 * rbk + 4 * lg + i;
      if (ri >= nrows) continue;
      const int jr = ri % qrows, h = grp * hpg + ri / qrows;
      const int col = ln16;
      if (so.final_out) {
        const int64_t ob = (int64_t)(row0 + jr) * p.o_sr + (int64_t)h * p.o_sh + col;
#pragma unroll
        for (int cb = 0; cb < C::CB; ++cb) store_out(p.out, p.out_dt, ob + 16 * cb, acc[cb][i] * inv_i);
      } else if (so.plse && p.part_h) {
        _Float16* ob = reinterpret_cast<_Float16*>(so.po) + (int64_t)jr * so.po_sr + (int64_t)h * so.po_sh + col;
        const float invh_i = __shfl(invh, 4 * lg + i, 64);
#pragma unroll
        for (int cb = 0; cb < C::CB; ++cb) ob[16 * cb] = (_Float16)(acc[cb][i] * invh_i);
      } else {
        float* ob = so.po + (int64_t)jr * so.po_sr + (int64_t)h * so.po_sh + col;
#pragma unroll
        for (int cb = 0; cb < C::CB; ++cb) ob[16 * cb] = acc[cb][i] * inv_i;
      }
    }
    if (lg == 0 && rok) {
      if (so.final_out) {
        if (p.lse) store_out(p.lse, p.lse_dt, (int64_t)(row0 + jq) * p.lse_sr + head, lse_v);
      } else if (so.plse) {
        so.plse[(int64_t)jq * so.plse_sr + head] = lse_v;
      } else {
        so.po[(int64_t)jq * so.po_sr + (int64_t)head * so.po_sh + C::DCG] = lse_v;
      }
    }
  };

  // ---- DMA wave: instruction i = dw + 2j covers LDS chunks 64i .. 64i+63 of a stage (staged row
  //      q / CPR, position q % CPR, i.e. row chunk pos_chunk(position, flip of the row)) ----
  const int dw = w - C::NCW;
  uint32_t doff[ROLE == DMA ? C::DPW : 1];
  int drow[ROLE == DMA ? C::DPW : 1];
  if constexpr (ROLE == DMA) {
#pragma unroll
    for (int j = 0; j < C::DPW; ++j) {
      // chunk qq of half dw: row 16dw + qq / CPR, position qq % CPR; chunks past the 16 rows are
      // padding (an offset past every buffer: they read zeros, or are not issued)
      const int qq = 64 * j + lane;
      const bool pad = qq >= 16 * C::CPR;
      const int q = pad ? 0 : qq;
      const int rr = 16 * dw + q / C::CPR, pp = q % C::CPR;
      doff[j] = pad ? 0x80000000u : (uint32_t)(rr * C::RB + 16 * pos_chunk<C::CPR>(pp, rflip(rr)));
      drow[j] = pad ? -1 : rr;
    }
  }
  // the DMA wave's transposed reads of its half for the fp16 V: lane group L takes 16-column block
  // 2cp + (L & 1) of rows 16dw + 8(L >> 1) .. +7 (lane pair 2r', 2r'+1: row r'), whose bytes 0-3 are
  // column n's tokens for lane group 2(L >> 1) and bytes 4-7 for lane group 2(L >> 1) + 1
  uint32_t cva = 0, cvb = 0, cvw = 0;
  if constexpr (ROLE == DMA) {
    const int R = 16 * dw + 8 * (lg >> 1) + (ln16 >> 1), fr = rflip(R), k0 = lg & 1;
    cva = (uint32_t)(rowoff<C>(R) + 16 * (k0 + fr) + 8 * (ln16 & 1));
    cvb = (uint32_t)(rowoff<C>(R) + 16 * ((6 + k0 + fr) & 7) + 8 * (ln16 & 1));
    cvw = (uint32_t)(k0 * 1024 + (32 * (lg >> 1) + ln16) * 16 + 8 * dw);
  }
  const bool contig = p.token_stride_b == C::RB;

  // one piece descriptor (wave-uniform fields: scalar registers)
  auto read_seg = [&](int k) {
    // drained (a kernel argument the compiler reloads nearby may still be in flight)
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

  // window planning cursor (wave 0 only)
  int cb = fixed ? (int)blockIdx.y : b0, ctok = 0, cp = c0;

  for (;;) {
    if (w == 0) plan_window<kPlanSwitchRo>(p, sm, fixed, lo, hi, cb, ctok, cp);
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

    if constexpr (ROLE == DMA) {
      // ---- DMA cursor: piece ki, tile ti, page cursor (window page index ipg, token offset ioff) ----
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
      // issues tile g into ring stage g % S and advances the cursor
      auto issue = [&](int g) {
        const int tok0 = i_ta + ti * TILE;
        const int nvalid = i_te - tok0 < TILE ? i_te - tok0 : TILE;
        char* dst = sm.kv[g % C::S];
        if (contig && ioff + TILE <= P) {
          // the tile's rows are consecutive in one page; rows past the piece end read as zeros
          lds_wait_n<0>(pidv);
          const int pg = __builtin_amdgcn_readfirstlane(pidv);
          const char* base = p.kv + (int64_t)pg * p.page_stride_b + (int64_t)ioff * p.token_stride_b;
          const __amdgpu_buffer_rsrc_t rs = make_rsrc(base, (uint32_t)(nvalid * C::RB));
#pragma unroll
          for (int j = 0; j < C::DPW; ++j) dma16_buf(rs, doff[j], dst + (C::DPW * dw + j) * 1024);
        } else {
          // per-lane page lookup; rows past the piece end repeat its last row
#pragma unroll
          for (int j = 0; j < C::DPW; ++j) {
            const int i = C::DPW * dw + j;
            if (drow[j] >= 0) {
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
        wait_tiles<C::DPW, C::A - 1>(ahead);
      };
      // this wave's half of tile t (landed) as fp16 V operands of both groups into vh[t & 1]
      auto convert = [&](int t) {
        const uint32_t sb = lds_addr(sm.kv[t % C::S]);
        const uint32_t vo = lds_addr(&sm.vh[t & 1][0][0][0][0]) + cvw;
        i32x2 raw[2 * 8];
        static_for<0, 16>([&](auto kc) {
          constexpr int k = decltype(kc)::value, gg = k / 8, cp = k % 8, b = 2 * gg + cp / 4;
          if constexpr (cp % 4 < 3) raw[k] = ldstr8_at<128 * b + 32 * (cp % 4)>(sb + cva);
          else raw[k] = ldstr8_at<128 * b>(sb + cvb);
        });
        // read k has 15 - k reads and 2k writes issued after it when it is awaited (LDS operations
        // complete in order)
        static_for<0, 16>([&](auto kc) {
          constexpr int k = decltype(kc)::value, gg = k / 8, cp = k % 8;
          lds_wait_n<15>(raw[k]);
          const i32x4 v = __builtin_bit_cast(i32x4, fp8x8_to_f16(raw[k]));
          ldsw64_at<1024 * (C::CB * gg + 2 * cp)>(vo, i32x2{v[0], v[1]});
          ldsw64_at<1024 * (C::CB * gg + 2 * cp) + 256>(vo, i32x2{v[2], v[3]});
        });
      };
      enter_i();
      pidv = ldsr32(&sm.pid[ipg]);
      for (int t = 0; t < C::A && t < ntot; ++t) issue(t);
      wait_tile(0, (C::A < ntot ? C::A : ntot) - 1);
      convert(0);
      lds_barrier();
#pragma clang loop unroll(disable)
      for (int g = 0; g < ntot; ++g) {
        // stage (g + A) % S held tile g - 1, which every compute wave finished before the last barrier
        if (g + C::A < ntot) issue(g + C::A);
        if (g + 1 < ntot) {
          wait_tile(g + 1, g + C::A < ntot - 1 ? g + C::A : ntot - 1);
          convert(g + 1);
        }
        lds_barrier();
      }
      wait_vmcnt<0>();
    } else {
      lds_barrier();
      int ks = 0, ts = 0, s_ta = 0, s_nt = 0, s_fl = 0, s_req = 0, lim = 0, lim_min = 0;
      constexpr bool quad = C::QUAD;
      // ---- per-lane read offsets within a stage ----
      // K: token block tb, 16-byte half h of the lane group's 32 columns; latent block b adds 128b
      // bytes. The rope block: lane groups 2, 3 read lane groups 0, 1's rope chunks again (the
      // rms bytes past the rope could read as fp8 NaN)
      uint32_t koff[2][2], kofr[2][2];
#pragma unroll
      for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int krow = 16 * tb + ln16, fk = rflip(krow);
          koff[tb][h] = (uint32_t)(rowoff<C>(krow) + 16 * (grp * (C::DCG / 16) + ((2 * lg + h + fk) & 7)));
          kofr[tb][h] = (uint32_t)(rowoff<C>(krow) + 16 * (C::DC / 16 + ((2 * lg + h + fk) & 3)));
        }
      // rms codes: the lane's head in token row 16tb + 4lg + (the lane's quad slot, or i)
      constexpr int NCI = quad ? 1 : 4;
      uint32_t coff[2][NCI];
#pragma unroll
      for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int i = 0; i < NCI; ++i) {
          const int row = 16 * tb + 4 * lg + (quad ? (ln16 & 3) : i);
          coff[tb][i] = (uint32_t)(rowoff<C>(row) + 16 * chunk_pos<C::CPR>(rms_b >> 4, rflip(row)) + (rms_b & 15));
        }
#pragma clang loop unroll(disable)
      for (int g = 0; g < ntot; ++g) {
        if (ts == 0) {
          const SegD d = read_seg(ks);
          s_ta = d.ta;
          s_nt = d.nt;
          s_fl = d.fl;
          s_req = d.req;
          if (d.fl & SEG_FIRST) {
            mref = kNegInf;
            lpart = 0.f;
#pragma unroll
            for (int c = 0; c < C::CB; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (live) load_q(d.req);
          }
          const int lr = d.L - (qrows - 1 - jq);
          lim = rok ? (lr < d.te ? lr : d.te) : 0;
          // the first verify row has the smallest limit: tiles below it need no mask
          lim_min = d.L - (qrows - 1) < d.te ? d.L - (qrows - 1) : d.te;
        }
        if (live) {
          const uint32_t sb = lds_addr(sm.kv[g % C::S]);
          const int tok0 = s_ta + ts * TILE;
          // ---- LDS reads: rms codes, then the K rows of both token blocks (2 x 5) ----
          // 4 verify tokens: lanes 4k..4k+3 hold the 4 verify rows of one head, so lane j reads the
          // codes of tokens 4lg+j (block 0) and 16+4lg+j (block 1) and the quad shares them
          uint32_t code[2][NCI];
#pragma unroll
          for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int i = 0; i < NCI; ++i) code[tb][i] = ldsr8_at(sb + coff[tb][i]);
          // K: per token block the latent blocks' two halves, then the rope block's
          i32x4 kr[2][C::KPT];
#pragma unroll
          for (int tb = 0; tb < 2; ++tb) {
            const uint32_t a0 = sb + koff[tb][0], a1 = sb + koff[tb][1];
            static_for<0, C::NB>([&](auto bc) {
              constexpr int b = decltype(bc)::value;
              kr[tb][2 * b] = ldsr128_at<128 * b>(a0);
              kr[tb][2 * b + 1] = ldsr128_at<128 * b>(a1);
            });
            kr[tb][2 * C::NB] = ldsr128_at<0>(sb + kofr[tb][0]);
            kr[tb][2 * C::NB + 1] = ldsr128_at<0>(sb + kofr[tb][1]);
          }
          // ---- score multipliers c2b / rms (log8: 2^(3 + log2 c2b - c*6/255)) as the codes land ----
          float rsc[2][4];
          if constexpr (quad) {
            float r0[2];
            lds_wait_n<cmin15(2 * C::KPT + 1)>(code[0][0]);
            r0[0] = fast_exp2(fmaf((float)code[0][0], -6.0f / 255.0f, lc2));
            lds_wait_n<cmin15(2 * C::KPT)>(code[1][0]);
            r0[1] = fast_exp2(fmaf((float)code[1][0], -6.0f / 255.0f, lc2));
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
              rsc[tb][0] = quad_bcast<0>(r0[tb]);
              rsc[tb][1] = quad_bcast<1>(r0[tb]);
              rsc[tb][2] = quad_bcast<2>(r0[tb]);
              rsc[tb][3] = quad_bcast<3>(r0[tb]);
            }
          } else {
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                lds_wait_n<cmin15(2 * C::KPT)>(code[tb][i]);
                rsc[tb][i] = fast_exp2(fmaf((float)code[tb][i], -6.0f / 255.0f, lc2));
              }
          }
          // ---- S^T = K . Q^T: per token block one chain of 16x16x128 MFMAs (hi and lo parts of the
          //      latent blocks and the rope block, the row's 2^-e as the B scale); the two token
          //      blocks alternate, so a chain's consecutive MFMAs are never adjacent ----
          f32x4 sl[2];
#pragma unroll
          for (int tb = 0; tb < 2; ++tb) sl[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
          static_for<0, C::NBQ>([&](auto bc) {
            constexpr int b = decltype(bc)::value;
            i32x8 ka[2];
            static_for<0, 2>([&](auto tc) {
              constexpr int tb = decltype(tc)::value;
              constexpr int n_after = (1 - tb) * C::KPT + (C::KPT - 2 - 2 * b);   // reads issued after kr[tb][2b+1]
              lds_wait_n<cmin15(n_after)>(kr[tb][2 * b + 1]);
              lds_wait_n<cmin15(n_after + 1)>(kr[tb][2 * b]);
              ka[tb] = i32x8{kr[tb][2 * b][0], kr[tb][2 * b][1], kr[tb][2 * b][2], kr[tb][2 * b][3],
                             kr[tb][2 * b + 1][0], kr[tb][2 * b + 1][1], kr[tb][2 * b + 1][2], kr[tb][2 * b + 1][3]};
              sl[tb] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ka[tb], qh8[b], sl[tb], 0, 0, 0, 127, 0, qsc);
            });
            if constexpr (b < C::NB) {
              static_for<0, 2>([&](auto tc) {
                constexpr int tb = decltype(tc)::value;
                sl[tb] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ka[tb], ql8[b], sl[tb], 0, 0, 0, 127, 0, qsc);
              });
            }
          });
          // ---- V of the tile as fp16, converted by the DMA waves (the K reads have all landed) ----
          i32x4 vraw[C::CB];
          {
            const uint32_t a0 = lds_addr(&sm.vh[g & 1][grp][0][0][0]) + 16 * lane;
            static_for<0, C::CB>([&](auto cc) {
              constexpr int c = decltype(cc)::value;
              vraw[c] = ldsr128_at<1024 * c>(a0);
            });
          }
          // ---- rms divide and scale; mask only a tile that reaches a row's limit; tile max ----
          float v[2][4];
#pragma unroll
          for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int i = 0; i < 4; ++i) v[tb][i] = sl[tb][i] * rsc[tb][i];
          if (tok0 + TILE > lim_min) {
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
              for (int i = 0; i < 4; ++i) v[tb][i] = tok0 + 16 * tb + 4 * lg + i < lim ? v[tb][i] : kNegInf;
          }
          float tm = fmaxf(fmaxf(fmaxf(v[0][0], v[0][1]), fmaxf(v[0][2], v[0][3])),
                           fmaxf(fmaxf(v[1][0], v[1][1]), fmaxf(v[1][2], v[1][3])));
          tm = max_lg(tm);
          // ---- the row's reference moves when the tile max exceeds it by more than SHIFT ----
          const bool mv = tm > mref + SHIFT;
          if (__builtin_amdgcn_ballot_w64(mv)) {
            const float mn = mv ? tm : mref;
            const float al = mv ? (mref == kNegInf ? 0.f : fast_exp2(mref - mn)) : 1.0f;
            mref = mn;
            lpart *= al;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float a_i = __shfl(al, 4 * lg + i, 64);   // accumulator row 4lg+i
#pragma unroll
              for (int c = 0; c < C::CB; ++c) acc[c][i] *= a_i;
            }
          }
          const float mu = mref == kNegInf ? 0.f : mref;
          f16x8 pf;
          float ps = 0.f;
#pragma unroll
          for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float e = fast_exp2(v[tb][i] - mu);
              ps += e;
              pf[4 * tb + i] = (_Float16)e;
            }
          lpart += ps;
          // ---- O += P . V over the group's 256 columns ----
          static_for<0, C::CB>([&](auto cc) {
            constexpr int c = decltype(cc)::value;
            lds_wait_n<cmin15(C::CB - 1 - c)>(vraw[c]);
            acc[c] = mfma16(pf, __builtin_bit_cast(f16x8, vraw[c]), acc[c]);
          });
        }
        if (++ts == s_nt) {
          if (live && (s_fl & SEG_LAST)) finalize(s_req, s_fl);
          ts = 0;
          ++ks;
        }
        lds_barrier();
      }
    }
    if (!more) break;
  }
}

template <class C>
__global__ __launch_bounds__(C::NTHR, 1) void ro_kernel(const KParams p) {
  static_assert(sizeof(Smem<C>) <= 163840, "LDS budget of a workgroup");
  __shared__ __attribute__((aligned(16))) Smem<C> sm;
  const float kscale = p.k_scale ? *p.k_scale : 1.0f;
  const bool fixed = p.num_splits > 0;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wr = blockIdx.x;
  int lo = 0, hi = 0, b0 = 0, c0 = 0;
  if (!fixed) {
    if (wr == 0 && wv == 1) store_plan<kPlanSwitchRo>(p);   // for the balanced combine
    const BalRange r = balanced_range<kPlanSwitchRo>(p, wr);
    lo = r.lo;
    hi = r.hi;
    b0 = r.b0;
    c0 = r.c0;
    if (lo >= hi) return;
  }
  int bad = 0;
  if (wv < C::NCW) role_main<C, COMPUTE>(p, sm, kscale, fixed, lo, hi, b0, c0, wr, bad);
  else role_main<C, DMA>(p, sm, kscale, fixed, lo, hi, b0, c0, wr, bad);
  report_pages(p, bad);
}

typedef void (*RoFn)(const KParams);
// [0]: 4 verify rows per head, [1]: other verify counts
static const RoFn kRo[] = {&ro_kernel<RO<3, true>>, &ro_kernel<RO<3, false>>};

}  // namespace ro

// The row-owner kernel serves GLA-g2 on fp8 + log8 rows: two groups of 256 latent columns, rope 64,
// at most 48 rows per group, 608-byte staged rows holding every head's code, no logit cap.
int ro_select(const qmla_decode_params* p) {
  if (!rows16(p)) return -1;
  if (p->groups != 2 || p->kv_dtype != QMLA_KV_FP8 || p->rms_mode != QMLA_RMS_LOG8) return -1;
  if (p->d_c != 512 || p->rope_w != 64 || p->logit_cap > 0.f) return -1;
  if (p->qrows * (p->heads / 2) > 48) return -1;
  if (p->token_stride < 608 || (int64_t)p->rms_offset + p->heads > 608) return -1;
  return p->qrows == 4 ? 0 : 1;
}

int ro_launch(int inst, const qmla_decode_params* p, const KParams& k, int nwg, hipStream_t st) {
  KParams kk = k;
  kk.hsplit = 1;
  void* args[] = {&kk};
  dim3 grid = p->num_splits > 0 ? dim3(p->num_splits, k.n_req, 1) : dim3(nwg, 1, 1);
  if (grid.x == 0 || grid.y == 0) return QMLA_OK;
  hipError_t e = hipLaunchKernel((const void*)ro::kRo[inst], grid, dim3(512, 1, 1), args, 0, st);
  return e == hipSuccess ? QMLA_OK : QMLA_ERR_LAUNCH;
}

}  // namespace qmla
