// qmla_cs.hip -- gfx950 column-split MLA decode: the workgroup's waves split the LATENT COLUMNS.
//
// A workgroup owns a contiguous token range of one request and every query row of it, so each
// cached row is read from HBM once per call. Its waves form a grid
//     G latent groups  x  NCG column slices  x  NTG token groups
// Wave (g, c, tg) owns latent columns [c*DCW, (c+1)*DCW) of group g (and a slice of the rope
// columns) for BOTH the score product and P.V, and the tg-th T-token part of every workgroup tile.
// It stages only its slice of each of its rows in a private LDS ring and waits for its own DMA;
// one wave per token group also stages the rms tail for the others. Per tile:
//   QK       S^T = K . Q^T on MFMA over the wave's columns: partial scores of T tokens x 16*MB rows,
//            query fragments resident in VGPRs (a column slice of them: ~36-60 VGPRs, not 144+).
//   sum      the NCG partials of (g, tg) meet in LDS; every wave adds them in the same order, so the
//            NCG waves hold bit-identical scores and take identical softmax decisions.
//   softmax  rms divide (codes read with one transposed LDS read per 16 rows), scale, mask, lazily
//            moving reference max; P stays in registers: the MFMA score layout already is the
//            A-operand layout of P.V under the token order chosen for the score tiles.
//   PV       acc[16*MB x DCW] += P . V on MFMA, V^T fragments read with ds_read_b64_tr_b8/_b16.
// With NTG = 2 the two token groups keep separate (max, sum, acc) and merge in the epilogue.
// Eight waves (two per SIMD) hide each other's LDS/MFMA latency.
//
// Token order inside a 32-token score tile pair (NTB = 2): score tile 0 row m is token m, score
// tile 1 row m is token 16 + ((m + 8) mod 16). Lane (n, q) then holds tokens {4q..4q+3} and
// {24+4q..} / {16+4q-8..} -- the set whose V rows (read 8 per 16-lane block by tr_b8) and K rows
// (16 per half-wave) fall on distinct LDS banks for the odd-16-byte row strides used here.
//
// Reference semantics: qwen_mla/ops/mla_decode_attention.py:297-586 (stage 1, incl. the rms divide
// :466-507 and the verify limit), :1264-1359 (entry); wide latents replace the two-pass path
// :602-849 with the same single pass.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "qmla.h"
#include "qmla_common.h"
#include "qmla_device.h"

namespace qmla {
namespace cs {

typedef __attribute__((__vector_size__(4 * sizeof(short)))) short s16x4;
typedef __attribute__((__vector_size__(8 * sizeof(short)))) short s16x8;

constexpr int PIDN = 512;    // page ids staged per sub-range

// 32 x 32 x 16 bf16 product (A: lane l holds row l % 32, k 8 (l / 32) .. +8; B: column l % 32, the
// same k; D: lane l, register v holds row 8 (v / 4) + 4 (l / 32) + v % 4, column l % 32). Twice the
// flops of the 16x16x16 form per cycle on gfx950.
__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16k16(const s16x4& a, const s16x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// LDS reads issued as inline asm (through the builtins the compiler waits for every LDS-DMA in
// flight first); results are valid after lds_wait().
__device__ __forceinline__ i32x4 ldsr128(const char* p) {
  i32x4 r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(lds_addr(p)));
  return r;
}
// reads at a base register plus an immediate offset, and a wait for all but the N youngest LDS
// operations of the wave (LDS operations complete in order, so the older reads are in)
template <int OFF>
__device__ __forceinline__ i32x2 ldsr64_off(uint32_t a) {
  i32x2 r;
  asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(r) : "v"(a), "n"(OFF));
  return r;
}
template <int OFF>
__device__ __forceinline__ i32x4 ldsr128_off(uint32_t a) {
  i32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(a), "n"(OFF));
  return r;
}
template <int OFF>
__device__ __forceinline__ i32x2 ldstr16_off(uint32_t a) {
  i32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(a), "n"(OFF));
  return r;
}
template <int OFF>
__device__ __forceinline__ i32x2 ldstr8_off(uint32_t a) {
  i32x2 r;
  asm volatile("ds_read_b64_tr_b8 %0, %1 offset:%2" : "=v"(r) : "v"(a), "n"(OFF));
  return r;
}
template <int N, class T>
__device__ __forceinline__ void lds_wait_n(T& v) {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(v) : "n"(N));
}
// f(integral_constant<int, I>) for I = B .. E-1
template <int B, int E, class F>
__device__ __forceinline__ void sfor(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    sfor<B + 1, E>(f);
  }
}
__device__ __forceinline__ i32x2 ldsr64(const char* p) {
  i32x2 r;
  asm volatile("ds_read_b64 %0, %1" : "=v"(r) : "v"(lds_addr(p)));
  return r;
}
__device__ __forceinline__ int ldsr32(const char* p) {
  int r;
  asm volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(lds_addr(p)));
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

// Compile-time shape of one instance.
//   EB   cache element bytes (1 = fp8 e4m3fn, 2 = bf16);  RMS  QMLA_RMS_* tail format
//   DCG  latent columns per group, G latent groups;  NCG column slices per group
//   NTG  token groups;  NTB 16-token score tiles per token group and tile (T = 16*NTB tokens)
//   MB   16-row blocks per latent group (rows per group = qrows*heads/G <= 16*MB)
//   S    LDS ring stages;  CRM 16-byte chunks of the rms tail staged per token;  CAP tanh logit cap
//   RTR  rms codes read transposed (rows are the heads of one token: G = 1 and qrows = 1)
//   WP   rope columns staged per row: 64 (exactly the rope), or the padded window 128 / 256 of a
//        partial rope (116 / 232 wide), spread over all NCG waves; columns past rope_w are zeroed
//        in both operands (the row bytes there are rms codes, which may read as fp8 NaN)
//   DW   narrow rows: cached rows on 4-byte boundaries only, staged 4 bytes per lane (four DMA
//        instructions per 64 chunks, the same LDS image)
template <int EB_, int RMS_, int DCG_, int G_, int NCG_, int NTG_, int NTB_, int MB_, int S_, int CRM_,
          bool CAP_, bool RTR_, int WP_, bool DW_ = false>
struct CS {
  static constexpr int EB = EB_, RMS = RMS_, DCG = DCG_, G = G_, NCG = NCG_, NTG = NTG_, NTB = NTB_;
  static constexpr int MB = MB_, S = S_, CRM = CRM_, WP = WP_;
  static constexpr bool CAP = CAP_, RTR = RTR_, DW = DW_;
  static constexpr bool PR = WP != 64;                   // partial rope: mask columns >= rope_w
  static constexpr int NW = G * NCG * NTG, NTHR = 64 * NW;
  static constexpr int T = 16 * NTB, TT = NTG * T;
  static constexpr int DC = G * DCG;
  static constexpr int DCW = DCG / NCG;                  // latent columns per wave
  static constexpr int KS = DCW / 32;                    // 32-column k-steps
  static constexpr int CB = DCW / 16;                    // 16-column output blocks
  static constexpr int RW = PR ? WP / NCG : (NCG >= 4 ? 16 : 64 / NCG);   // rope columns per wave (WP 64, NCG 8: waves c < 4)
  static constexpr int CL = DCW * EB / 16;               // latent chunks of a row slice
  static constexpr int CR = RW * EB / 16;                // rope chunks
  static constexpr int CPW = (CL + CR) | 1;              // odd 16-byte count: conflict-free rows
  static constexpr int RS = 16 * CPW;                    // LDS row stride
  static constexpr int NCH = T * CPW;                    // chunks per tile per wave
  static constexpr int NI = (NCH + 63) / 64;             // DMA instructions per tile per wave
  static constexpr int SB = NCH * 16;                    // stage bytes per wave
  static constexpr int RB = (RMS == QMLA_RMS_NONE) ? 0 : ((RMS == QMLA_RMS_BF16 || RMS == QMLA_RMS_BF16_BYTES) ? 2 : 1);
  static constexpr int RRS = 16 * (CRM > 0 ? CRM : 1);   // staged rms row bytes
  static constexpr int NRI = CRM > 0 ? (T * CRM + 63) / 64 : 0;   // rms DMA instructions per tile
  // DMA instructions per tile as issued: 64 chunks each, or 16 with narrow rows
  static constexpr int NID = DW ? (NCH + 15) / 16 : NI;
  static constexpr int NRID = DW ? (T * CRM + 15) / 16 : NRI;
  static constexpr int ROWS = 16 * MB;
  static constexpr int XBW = NTB * MB;                   // partial-score f32x4 per lane
  // reduce-scatter of the partial scores over the 8 slices (one latent group and token group:
  // 16-token tiles and 32 rows, fp8 rows with 32-token tiles and 16 or 32 rows): wave c
  // sums and softmaxes its RPW rows only, RE scores per lane, and P reaches the other waves through
  // LDS; otherwise every wave sums all partials and repeats the whole softmax
  static constexpr int RPW = ROWS / 8;                   // rows per reducer wave
  static constexpr int RLR = 64 / T;                     // rows per wave instruction (T tokens each)
  static constexpr int RPS = 2 * T + (T == 16 ? 8 : 16); // P row stride (bytes) of the reduce-scatter
  // LDS of the ring, rms stages, partial scores and page ids, and what the reduce-scatter adds
  static constexpr int LDS0 = S * NW * SB + (S + 1) * NTG * T * RRS + NW * XBW * 64 * 16 + 4 * PIDN;
  static constexpr int LDSR = ROWS * RPS + 12 * ROWS + 32 + 48;
  static constexpr bool RSC = G == 1 && NCG == 8 && NTG == 1 && LDS0 + LDSR <= 163840 &&
                              ((NTB == 1 && MB == 2) || (EB == 1 && NTB == 2));
  static constexpr int RE = RSC ? RPW / RLR : 1;         // scores per lane
  // 16-token tiles of 32 rows: P.V on the 32x32x16 MFMA (32 rows x 32 columns per instruction)
  // instead of four 16x16x16 ones, which run at half the flops per cycle
  static constexpr bool W32 = RSC && NTB == 1 && MB == 2 && CB % 2 == 0 && NTG == 1;
  // The 32 columns of a 32x32 block are two 16-column blocks (a, a + d): lanes 0-31 of a
  // transposed V read cover 8 rows x 16 bytes (fp8) or 4 rows x 32 bytes (bf16: token rows 2r,
  // then 2r + 1) of each. The LDS serves 32 lanes at a time over 128 four-byte banks; with the odd
  // 16-byte row stride the rows of one block take half of the four-bank groups they can reach and
  // the block 128 bytes away (fp8 d = 8, bf16 d = 4) the other half, so the read has no conflicts.
  // A leftover pair takes d = 1 (two-way conflicts in that read).
  static constexpr int PD = EB == 1 ? 8 : 4;
  struct Pairs {
    int a[CB / 2 > 0 ? CB / 2 : 1], d[CB / 2 > 0 ? CB / 2 : 1];
    constexpr Pairs() : a(), d() {
      bool used[CB > 0 ? CB : 1] = {};
      int n = 0;
      for (int x = 0; x < CB; ++x) {
        if (used[x]) continue;
        int y = x + PD;
        if (y >= CB || used[y]) {
          y = x + 1;
          while (y < CB && used[y]) ++y;
        }
        used[x] = used[y] = true;
        a[n] = x;
        d[n] = y - x;
        ++n;
      }
    }
  };
  static constexpr Pairs PAIRS{};
  // fp8 rows: the per-lane DMA offsets of a tile (the same for every tile of a call) in an LDS
  // table, where it fits, instead of recomputing them at every issue
  static constexpr int NDV = NID + NRID;
  static constexpr bool DVT = EB == 1 && !DW && LDS0 + (RSC ? LDSR : 0) + NW * NDV * 256 + 64 <= 163840;
  static_assert(DCG % (32 * NCG) == 0, "whole 32-column k-steps per wave");
  static_assert(NTB == 1 || NTB == 2, "score tiles per token group");
  static_assert(EB == 2 || NTB == 2 || CB % 2 == 0, "fp8 values of 16-token tiles are read two column blocks at a time");
  static_assert(RW == 16 || RW == 32 || RW == 64, "rope slice");
  static_assert(!PR || (WP % NCG == 0 && (WP == 128 || WP == 256)), "padded rope window");
  static_assert((S - 1) * (NID + NRID) < 64, "vmcnt range");
  static_assert(!DW || !RTR, "narrow rows take per-row rms reads");
  static_assert(!RTR || CRM * 16 >= RB * ROWS, "transposed rms reads cover all row heads");
};

// reduce-scatter: P of the tile's 32 rows (bf16), the rows' rescale factors, per reducer wave
// whether its rows' reference moved, the rows' final max and sum
template <int ROWS, int RPS>
struct RsShared {
  alignas(16) char rp[ROWS * RPS];
  alignas(16) float ra[ROWS];
  alignas(16) int rf[8];
  alignas(16) float rfin[2][ROWS];
};
struct RsNone {};
template <int NW, int NDV>
struct DvTable {
  uint32_t o[NW][NDV][64];
};
struct DvNone {};

template <class C>
struct Smem {
  char ring[C::S][C::NW][C::SB];
  char rms[C::S + 1][C::NTG][C::T * C::RRS];   // S+1 deep: read after the exchange
  f32x4 xb[C::NW][C::XBW][64];                 // partial scores
  int pid[PIDN];
  [[no_unique_address]] std::conditional_t<C::RSC, RsShared<C::ROWS, C::RPS>, RsNone> rs;
  [[no_unique_address]] std::conditional_t<C::DVT, DvTable<C::NW, C::NDV>, DvNone> dv;
};


// score tile tb, tile row m -> token offset inside the token group's T tokens
__device__ __forceinline__ constexpr int tok_of(int tb, int m) { return tb == 0 ? m : 16 + ((m + 8) & 15); }
// k-slot 8q + r of the P.V product (NTB = 2) -> token offset: the lane's scores in order
__device__ __forceinline__ constexpr int vtok(int q, int r) { return r < 4 ? tok_of(0, 4 * q + r) : tok_of(1, 4 * q + r - 4); }

template <class C>
__device__ __forceinline__ void wait_tile(bool steady, bool rms_wave) {
  if (!steady) wait_vmcnt<0>();
  else if (rms_wave) wait_vmcnt<(C::S - 1) * (C::NID + C::NRID)>();
  else wait_vmcnt<(C::S - 1) * C::NID>();
}

// One contiguous token range [ta, te) of request `req` (length L), all query rows.
template <class C>
__device__ __forceinline__ void segment(const KParams& p, Smem<C>& sm, int req, int ta, int te, int L,
                                        const SegOut& so, float kscale, int& bad) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tg = w / (C::G * C::NCG);
  const int g = (w / C::NCG) % C::G;
  const int c = w % C::NCG;
  const bool rms_wave = (C::CRM > 0) && (w % (C::G * C::NCG)) == 0;   // (g 0, c 0) of each token group
  const bool has_rope = C::PR || C::NCG < 8 || c < 4;
  const int rope_col = (C::NCG >= 4 && !C::PR) ? 16 * (c & 3) : C::RW * c;
  // the rms tail is staged from the 16-byte boundary at or below its offset
  const int roff_al = p.rms_off_b & ~15, rdelta = p.rms_off_b & 15;
  const int ln16 = lane & 15, lg = lane >> 4;
  const int hpg = p.hpg;
  const int rows_pg = p.qrows * hpg;
  // rows (verify token x head of the group) [rbase, rbase + 16*MB) of the request: requests with
  // more rows than one workgroup holds are split over gridDim.z workgroups (each reads the rows)
  const int rbase = (int)blockIdx.z * C::ROWS;
  const int row0 = req * p.qrows;
  const int P = p.page_size;
  const int64_t TS = p.token_stride_b, PS = p.page_stride_b;
  // a folded request reads the block-table row of its last verify row, as its length does
  const int* btrow = p.bt + (int64_t)(row0 + p.qrows - 1) * p.bt_stride;
  const float csc = p.sm_scale * kLog2e * kscale;
  const float cap2 = p.logit_cap * kLog2e;

  // ---- query fragments (B operands) for this wave's columns; zero for padding rows ----
  bf16x8 qf[C::KS][C::MB];
  constexpr int RKS = C::RW == 64 ? 2 : 1;
  // rope: 16x16x32 steps. A 16-column slice is one step with the upper half zero (lanes lg 0-1
  // carry columns 8lg..8lg+7, lanes 2-3 zeros in both operands), so every product of the score
  // chain has the same MFMA shape: a 16x16x16 step accumulating onto a 16x16x32 result right
  // behind it reads the accumulator before it is complete
  bf16x8 qr8[RKS][C::MB];
  int lim[C::MB], hb[C::MB];
#pragma unroll
  for (int mb = 0; mb < C::MB; ++mb) {
    const int r = rbase + ln16 + 16 * mb;
    const bool ok = r < rows_pg;
    const int jq = ok ? r / hpg : 0, hh = ok ? r - jq * hpg : 0;
    const int head = g * hpg + hh;
    // verify row jq of the request sees its first L - (qrows-1-jq) tokens (mla_impl.py:628-662)
    const int lr = L - (p.qrows - 1 - jq);
    lim[mb] = ok ? (lr < te ? lr : te) : 0;
    hb[mb] = (ok ? head * C::RB : 0) + rdelta;
    const __bf16* qn = p.q_nope + (int64_t)(row0 + jq) * p.qn_sr + (int64_t)head * p.qn_sh + c * C::DCW + 8 * lg;
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
      bf16x8 v = load_q8(qn + 32 * ks, p.q_vec);
      if (!ok) v = bf16x8{};
      qf[ks][mb] = v;
    }
    const __bf16* qp = p.q_pe + (int64_t)(row0 + jq) * p.qp_sr + (int64_t)head * p.qp_sh + rope_col;
    const bool lane_rope = C::RW != 16 || lg < 2;
    if constexpr (C::PR) {
      // element loads of the real rope columns only; the window past rope_w is zero
#pragma unroll
      for (int k = 0; k < RKS; ++k) {
        bf16x8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int col = (C::RW == 16 ? 8 * (lg & 1) : 32 * k + 8 * lg) + e;
          v[e] = (ok && lane_rope && rope_col + col < p.rope_w) ? qp[col] : (__bf16)0.0f;
        }
        qr8[k][mb] = v;
      }
    } else {
#pragma unroll
      for (int k = 0; k < RKS; ++k) {
        bf16x8 v = load_q8(qp + (C::RW == 16 ? 8 * (lg & 1) : 32 * k + 8 * lg), p.q_vec);
        if (!ok || !has_rope || !lane_rope) v = bf16x8{};
        qr8[k][mb] = v;
      }
    }
  }
  // key masks of a padded rope window: word j of k-step k covers the lane's elements
  // [4j/EB, 4(j+1)/EB); elements at columns >= rope_w (rms codes, possibly fp8 NaN bytes) and the
  // zero half of a 16-column step are cleared. Without a window no mask is needed: the zero query
  // lanes meet rope bytes of the same row (a 16-column step's upper lanes read its lower half)
  constexpr bool KMASK = C::PR;
  uint32_t kmw[RKS][4];
#pragma unroll
  for (int k = 0; k < RKS; ++k) {
    const int col0 = rope_col + (C::RW == 16 ? 8 * (lg & 1) : 32 * k + 8 * lg);
    const bool lane_ok = has_rope && (C::RW != 16 || lg < 2);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t m = 0;
#pragma unroll
      for (int b = 0; b < 4 / C::EB; ++b) {
        const int e = j * (4 / C::EB) + b;
        if (lane_ok && (!C::PR || col0 + e < p.rope_w)) m |= (C::EB == 1 ? 0xFFu : 0xFFFFu) << (8 * C::EB * b);
      }
      kmw[k][j] = m;
    }
  }
  // smallest row limit: tiles below it need no masking
  const int limmin = L - (p.qrows - 1) < te ? L - (p.qrows - 1) : te;
  // reduce-scatter: score e of this lane is token tt of reducer row rrow[e] = RPW c + RLR e + lane / T;
  // the row's limit and rms byte offset, and its softmax state (the same in its T lanes; the sum is
  // per lane)
  const int tt = lane % C::T;
  int rrow[C::RE], rlim[C::RE], rhb[C::RE];
  float rmref[C::RE], rmthr[C::RE], rlp[C::RE];
#pragma unroll
  for (int e = 0; e < C::RE; ++e) {
    rrow[e] = C::RPW * c + C::RLR * e + lane / C::T;
    rlim[e] = 0;
    rhb[e] = 0;
    rmref[e] = kNegInf;
    rmthr[e] = kNegInf;
    rlp[e] = 0.f;
    if constexpr (C::RSC) {
      const int r = rbase + rrow[e];
      const bool ok = r < rows_pg;
      const int jq = ok ? r / hpg : 0, hh = ok ? r - jq * hpg : 0;
      const int lr = L - (p.qrows - 1 - jq);
      rlim[e] = ok ? (lr < te ? lr : te) : 0;
      rhb[e] = (ok ? (g * hpg + hh) * C::RB : 0) + rdelta;
    }
  }

  // ---- DMA source of chunk i of the wave's tile slice: row i / CPW, chunk i % CPW of
  //      [latent slice | rope slice | pad]; recomputed at every issue rather than held ----
  const int lat_off = (g * C::DCG + c * C::DCW) * C::EB;
  const int rope_off = C::DC * C::EB + rope_col * C::EB;
  // fp8 rows (i < 64 NI): the quotient by CPW from a 24-bit multiply, exact below 2^20 / CPW, and
  // selects instead of branches, so the issue costs a few full-rate VALU instructions per DMA
  // instruction (fp8 rank 1792, rope 232, B 128: 1325 -> 1280 us; the bf16 rank-1792 instances
  // measured 1% slower with it and keep the plain form)
  constexpr uint32_t CPW_M = ((1u << 20) + C::CPW - 1) / C::CPW;
  static_assert(64 * C::NI * C::CPW < (1 << 20) && 64 * C::NI < (1 << 10), "exact 24-bit quotient");
  auto src_chunk = [&](int i, int& row) {
    int t, ch, off;
    if constexpr (C::EB == 1) {
      t = (int)(__umul24((uint32_t)i, CPW_M) >> 20);
      ch = i - (int)__umul24((uint32_t)t, (uint32_t)C::CPW);
      off = ch < C::CL ? lat_off + 16 * ch : rope_off + 16 * (ch - C::CL);
      off = ch < C::CL + C::CR ? off : 0;
    } else {
      t = i / C::CPW;
      ch = i - t * C::CPW;
      if (ch < C::CL) off = lat_off + 16 * ch;
      else if (ch < C::CL + C::CR) off = rope_off + 16 * (ch - C::CL);
      else off = 0;
    }
    row = i < C::NCH ? t : 0;
    return off;
  };

  // mref: the softmax reference; mthr: mref + ref_shift of the running sum at its last evaluation
  // (the sum only grows while mref stays, so a tile max at or below mthr cannot move mref)
  float mref[C::MB], mthr[C::MB], lpart[C::MB];
  // accumulators: [row block][16-column block] of 16x16 tiles, or [32-column block] of 32x32 ones
  f32x4 acc[C::W32 ? 1 : C::MB][C::W32 ? 1 : C::CB];
  f32x16 acc32[C::W32 ? C::CB / 2 : 1];
#pragma unroll
  for (int mb = 0; mb < C::MB; ++mb) {
    mref[mb] = kNegInf;
    mthr[mb] = kNegInf;
    lpart[mb] = 0.f;
  }
  if constexpr (C::W32) {
#pragma unroll
    for (int j = 0; j < C::CB / 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc32[j][v] = 0.f;
  } else {
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
      for (int cb = 0; cb < C::CB; ++cb) acc[mb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  if constexpr (C::DVT) {
    // this wave's DMA offsets inside a contiguous tile (rows from the token group's first row)
    const uint32_t ts24 = (uint32_t)TS;   // < 2^24 (the host checks)
#pragma unroll
    for (int k = 0; k < C::NID; ++k) {
      int row;
      const int off = src_chunk(64 * k + lane, row);
      sm.dv.o[w][k][lane] = __umul24((uint32_t)(tg * C::T + row), ts24) + (uint32_t)off;
    }
    if (rms_wave) {
#pragma unroll
      for (int k = 0; k < C::NRID; ++k) {
        const int j = 64 * k + lane;
        const int row = j / (C::CRM > 0 ? C::CRM : 1);
        sm.dv.o[w][C::NID + k][lane] =
            __umul24((uint32_t)(tg * C::T + row), ts24) + (uint32_t)(roff_al + 16 * (j - row * C::CRM));
      }
    }
  }

  // sub-ranges of at most PIDN pages, in whole tiles
  int sub = (PIDN - 1) * P;
  sub = sub < C::TT ? C::TT : sub / C::TT * C::TT;
  const bool uni = (P % C::TT) == 0 && (ta % C::TT) == 0;   // every tile within one page
  for (int sa = ta; sa < te; sa += sub) {
    const int se = te - sa < sub ? te : sa + sub;
    const int pbase = sa / P;
    const int np = (se - 1) / P - pbase + 1;
    wait_vmcnt<0>();
    lds_barrier();   // every wave is done with the previous sub-range's page ids
    for (int i = tid; i < np; i += C::NTHR) sm.pid[i] = checked_page(p, btrow[pbase + i], bad);
    __syncthreads();
    const int nt = (se - sa + C::TT - 1) / C::TT;

    auto issue = [&](int t) {
      const int tok0 = sa + t * C::TT;
      const int nvalid = se - tok0 < C::TT ? se - tok0 : C::TT;
      char* dst = sm.ring[t % C::S][w];
      char* rdst = sm.rms[t % (C::S + 1)][tg];
      int ln = lane;
      asm volatile("" : "+v"(ln));   // keep the offsets from being hoisted out of the tile loop
      if (uni) {
        const int pg = __builtin_amdgcn_readfirstlane(sm.pid[tok0 / P - pbase]);
        const char* base = p.kv + (int64_t)pg * PS + (int64_t)(tok0 % P) * TS;
        // rows past the range end read as zeros (outside the resource)
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(base, (uint32_t)(nvalid * TS));
        const int tb0 = tg * C::T;
        const uint32_t ts24 = (uint32_t)TS;   // < 2^24 (the host checks)
        // chunk i of the stage lands at 16 i: instruction k carries chunks 64k.. (16 bytes a lane),
        // or 16k.. (narrow rows: lane ln the 4 bytes at 4 (ln & 3) of chunk 16k + ln / 4)
        constexpr int CPI = C::DW ? 16 : 64;
        const int cl = C::DW ? ln >> 2 : ln, bl = C::DW ? 4 * (ln & 3) : 0;
        if constexpr (C::DVT) {
          uint32_t vo[C::NDV];
#pragma unroll
          for (int k = 0; k < C::NDV; ++k) vo[k] = sm.dv.o[w][k][ln];
#pragma unroll
          for (int k = 0; k < C::NID; ++k)
            if (64 * k + 64 <= C::NCH || 64 * k + ln < C::NCH) dma16_buf<kCpolDefault>(rs, vo[k], dst + k * 1024);
          if (rms_wave) {
#pragma unroll
            for (int k = 0; k < C::NRID; ++k)
              if (64 * k + 64 <= C::T * C::CRM || 64 * k + ln < C::T * C::CRM)
                dma16_buf<kCpolDefault>(rs, vo[C::NID + k], rdst + k * 1024);
          }
        } else {
#pragma unroll
        for (int k = 0; k < C::NID; ++k) {
          int row;
          const int off = src_chunk(CPI * k + cl, row) + bl;
          if (CPI * k + CPI <= C::NCH || CPI * k + cl < C::NCH) {
            const uint32_t vo = C::EB == 1 ? __umul24((uint32_t)(tb0 + row), ts24) + (uint32_t)off
                                           : (uint32_t)((tb0 + row) * (int)TS + off);
            if constexpr (C::DW) dma4_buf(rs, vo, dst + k * 256);
            else dma16_buf<kCpolDefault>(rs, vo, dst + k * 1024);
          }
        }
        if (rms_wave) {
#pragma unroll
          for (int k = 0; k < C::NRID; ++k) {
            const int j = CPI * k + cl;
            const int row = j / (C::CRM > 0 ? C::CRM : 1);
            if (CPI * k + CPI <= C::T * C::CRM || j < C::T * C::CRM) {
              const uint32_t o = (C::EB == 1 ? __umul24((uint32_t)(tb0 + row), ts24) : (uint32_t)((tb0 + row) * (int)TS)) +
                                 (uint32_t)(roff_al + 16 * (j - row * C::CRM) + bl);
              if constexpr (C::DW) dma4_buf(rs, o, rdst + k * 256);
              else dma16_buf<kCpolDefault>(rs, o, rdst + k * 1024);
            }
          }
        }
        }
      } else {
        // pages change inside a tile: per-lane page lookup; rows past the end repeat the last row
        const int tb0 = tok0 + tg * C::T;
        const int nv = se - tb0;   // rows of this token group inside the range (may be <= 0)
        constexpr int CPI = C::DW ? 16 : 64;
        const int cl = C::DW ? ln >> 2 : ln, bl = C::DW ? 4 * (ln & 3) : 0;
#pragma unroll
        for (int k = 0; k < C::NID; ++k) {
          int row;
          const int off = src_chunk(CPI * k + cl, row) + bl;
          if (CPI * k + CPI <= C::NCH || CPI * k + cl < C::NCH) {
            const int rr = row < nv ? row : (nv > 0 ? nv - 1 : 0);
            const int tok = nv > 0 ? tb0 + rr : se - 1;
            const int q = tok / P;
            const int pg = sm.pid[q - pbase];
            const char* src = p.kv + (int64_t)pg * PS + (int64_t)(tok - q * P) * TS + off;
            if constexpr (C::DW) dma4(src, dst + k * 256);
            else dma16<kCpolDefault>(src, dst + k * 1024);
          }
        }
        if (rms_wave) {
#pragma unroll
          for (int k = 0; k < C::NRID; ++k) {
            const int j = CPI * k + cl;
            const int row = j / (C::CRM > 0 ? C::CRM : 1);
            const int ob = roff_al + 16 * (j - row * C::CRM) + bl;   // byte of the row
            // narrow rows: the staged tail may end past the row; those bytes are not read
            if ((CPI * k + CPI <= C::T * C::CRM || j < C::T * C::CRM) && (!C::DW || ob < (int)TS)) {
              const int rr = row < nv ? row : (nv > 0 ? nv - 1 : 0);
              const int tok = nv > 0 ? tb0 + rr : se - 1;
              const int q = tok / P;
              const int pg = sm.pid[q - pbase];
              const char* src = p.kv + (int64_t)pg * PS + (int64_t)(tok - q * P) * TS + ob;
              if constexpr (C::DW) dma4(src, rdst + k * 256);
              else dma16<kCpolDefault>(src, rdst + k * 1024);
            }
          }
        }
      }
    };

    for (int t = 0; t < C::S && t < nt; ++t) issue(t);

#pragma clang loop unroll(disable)
    for (int t = 0; t < nt; ++t) {
      wait_tile<C>(t + C::S - 1 < nt, rms_wave);
      const char* st = sm.ring[t % C::S][w];
      const int tok0 = sa + t * C::TT + tg * C::T;   // this token group's first token

      // ---- partial scores over this wave's columns ----
      f32x4 sp[C::NTB][C::MB];
#pragma unroll
      for (int tb = 0; tb < C::NTB; ++tb) {
#pragma unroll
        for (int mb = 0; mb < C::MB; ++mb) sp[tb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
        const char* kr = st + tok_of(tb, ln16) * C::RS;
        if constexpr (C::EB == 1) {
          // all K reads at once (base register + immediate offsets), each k-step as soon as its
          // read is in
          i32x2 kv[C::KS];
          const uint32_t kb = lds_addr(kr + 8 * lg);
          sfor<0, C::KS>([&](auto ks) { kv[ks] = ldsr64_off<32 * ks>(kb); });
          i32x2 rv[RKS];
#pragma unroll
          for (int k = 0; k < RKS; ++k)
            rv[k] = ldsr64(kr + 16 * C::CL + (C::RW == 16 ? 8 * (lg & 1) : 32 * k + 8 * lg));
          sfor<0, C::KS>([&](auto ks) {
            lds_wait_n<C::KS - 1 - ks + RKS>(kv[ks]);
            const bf16x8 kf = fp8x8_to_bf16(kv[ks]);
#pragma unroll
            for (int mb = 0; mb < C::MB; ++mb) sp[tb][mb] = mfma16(kf, qf[ks][mb], sp[tb][mb]);
          });
#pragma unroll
          for (int k = 0; k < RKS; ++k) {
            lds_wait(rv[k]);
            if constexpr (KMASK) {
              rv[k][0] &= (int)kmw[k][0];
              rv[k][1] &= (int)kmw[k][1];
            }
            const bf16x8 rf = fp8x8_to_bf16(rv[k]);
#pragma unroll
            for (int mb = 0; mb < C::MB; ++mb) sp[tb][mb] = mfma16(rf, qr8[k][mb], sp[tb][mb]);
          }
        } else {
          constexpr int KB = 4;   // k-steps per batch of LDS reads, each used as soon as it is in
          const uint32_t kb = lds_addr(kr + 16 * lg);
          sfor<0, (C::KS + KB - 1) / KB>([&](auto b) {
            constexpr int k0 = KB * b, nb = C::KS - k0 < KB ? C::KS - k0 : KB;
            i32x4 kv[KB];
            sfor<0, nb>([&](auto j) { kv[j] = ldsr128_off<64 * (k0 + j)>(kb); });
            sfor<0, nb>([&](auto j) {
              lds_wait_n<nb - 1 - j>(kv[j]);
              const bf16x8 kf = __builtin_bit_cast(bf16x8, kv[j]);
#pragma unroll
              for (int mb = 0; mb < C::MB; ++mb) sp[tb][mb] = mfma16(kf, qf[k0 + j][mb], sp[tb][mb]);
            });
          });
#pragma unroll
          for (int k = 0; k < RKS; ++k) {
            i32x4 rv = ldsr128(kr + 16 * C::CL + (C::RW == 16 ? 16 * (lg & 1) : 64 * k + 16 * lg));
            lds_wait(rv);
            if constexpr (KMASK) {
#pragma unroll
              for (int j = 0; j < 4; ++j) rv[j] &= (int)kmw[k][j];
            }
            const bf16x8 rf = __builtin_bit_cast(bf16x8, rv);
#pragma unroll
            for (int mb = 0; mb < C::MB; ++mb) sp[tb][mb] = mfma16(rf, qr8[k][mb], sp[tb][mb]);
          }
        }
      }

      bf16x8 pa8[C::MB];
      s16x4 pa4[C::MB];
      bf16x8 pa32;   // 32x32x16 A operand (W32)
      if constexpr (C::RSC) {
        // ---- reduce-scatter: each wave writes its partial scores as a [ROWS][T] fp32 tile (a row's
        //      4-token groups rotated by xrot(row), so the 16 rows of a write and the 64 scores of a
        //      read fall on distinct banks); wave c sums the 8 slices' partials of its rows ----
        float* xs = reinterpret_cast<float*>(&sm.xb[0][0][0]);
        constexpr int NG = C::T / 4;   // 4-token groups of a row
        auto xrot = [](int r) { return C::T == 16 ? (r & 15) >> 2 : (r >> 1) & 7; };
#pragma unroll
        for (int tb = 0; tb < C::NTB; ++tb)
#pragma unroll
          for (int mb = 0; mb < C::MB; ++mb) {
            const int row = 16 * mb + ln16;
            const int g0 = tok_of(tb, 4 * lg) >> 2;
            *reinterpret_cast<f32x4*>(xs + (w * C::ROWS + row) * C::T + 4 * ((g0 + xrot(row)) & (NG - 1))) = sp[tb][mb];
          }
        lds_barrier();
        int xr[C::RE][C::NCG];
#pragma unroll
        for (int e = 0; e < C::RE; ++e) {
          const int xpos = 4 * (((tt >> 2) + xrot(rrow[e])) & (NG - 1)) + (tt & 3);
#pragma unroll
          for (int v = 0; v < C::NCG; ++v)
            xr[e][v] = ldsr32(reinterpret_cast<const char*>(xs + (v * C::ROWS + rrow[e]) * C::T + xpos));
        }
        // rms divisors of (token tt, the rows' heads)
        uint32_t cd[C::RE];
        if constexpr (C::RMS != QMLA_RMS_NONE) {
          const char* rsb = sm.rms[t % (C::S + 1)][tg] + tt * C::RRS;
#pragma unroll
          for (int e = 0; e < C::RE; ++e) cd[e] = C::RB == 1 ? ldsr8(rsb + rhb[e]) : ldsr16(rsb + rhb[e]);
        }
#pragma unroll
        for (int e = 0; e < C::RE; ++e)
#pragma unroll
          for (int v = 0; v < C::NCG; ++v) lds_wait(xr[e][v]);
        if constexpr (C::RMS != QMLA_RMS_NONE) {
#pragma unroll
          for (int e = 0; e < C::RE; ++e) lds_wait(cd[e]);
        }
        bool moved = false;
        float alpha[C::RE];
#pragma unroll
        for (int e = 0; e < C::RE; ++e) {
          float sv = __int_as_float(xr[e][0]);
#pragma unroll
          for (int v = 1; v < C::NCG; ++v) sv += __int_as_float(xr[e][v]);
          float ri = 1.0f;
          if constexpr (C::RMS == QMLA_RMS_LOG8) {
            ri = fast_exp2(fmaf((float)cd[e], -6.0f / 255.0f, 3.0f));
          } else if constexpr (C::RMS == QMLA_RMS_E4M3) {
            const float rv = fp8_to_f32(cd[e]) * kscale;
            ri = rv > 0.f ? __builtin_amdgcn_rcpf(rv) : 1.0f;
          } else if constexpr (C::RMS == QMLA_RMS_BF16 || C::RMS == QMLA_RMS_BF16_BYTES) {
            const float rv = bf16_bits_to_f32(cd[e]);
            ri = rv > 0.f ? __builtin_amdgcn_rcpf(rv) : 1.0f;
          }
          float v = sv * ri * csc;
          if constexpr (C::CAP) {
            const float y = v / cap2;
            const float e2 = fast_exp2(2.0f * kLog2e * y);
            v = cap2 * (1.0f - 2.0f / (e2 + 1.0f));
          }
          if (tok0 + C::T > limmin && tok0 + tt >= rlim[e]) v = kNegInf;
          // row max over the row's T lanes
          float tm = max16(v);
          if constexpr (C::T == 32) tm = fmaxf(tm, __shfl_xor(tm, 16));
          // the row's reference moves as in the other layout (ref_shift of the row's sum, P <= 2^8)
          alpha[e] = 1.0f;
          if (__builtin_amdgcn_ballot_w64(tm > rmthr[e])) {
            float ls = sum16(rlp[e]);
            if constexpr (C::T == 32) ls += __shfl_xor(ls, 16);
            rmthr[e] = rmref[e] + ref_shift(ls, 8.0f);
            const bool mv = tm > rmthr[e];
            if (__builtin_amdgcn_ballot_w64(mv)) {
              const float mn = mv ? tm : rmref[e];
              alpha[e] = rmref[e] == kNegInf ? 0.f : fast_exp2(rmref[e] - mn);
              rlp[e] *= alpha[e];
              rmref[e] = mn;
              if (mv) rmthr[e] = mn;
              moved = true;
            }
          }
          const float pv = fast_exp2(v - (rmref[e] == kNegInf ? 0.f : rmref[e]));
          rlp[e] += pv;
          // bf16 rows: k-slot 8h + 4b + a of the 32x32 P.V operand is token 8h + 2a + b (16x16:
          // k-slot 4q + i is token 2i + 8 (q & 1) + (q >> 1)), the order of the V reads below
          const int ks = C::EB == 1 ? tt
                         : C::W32   ? ((tt & 8) | ((tt & 1) << 2) | ((tt >> 1) & 3))
                                    : (8 * (tt & 1) + 4 * ((tt >> 3) & 1) + ((tt >> 1) & 3));
          *reinterpret_cast<__bf16*>(sm.rs.rp + rrow[e] * C::RPS + 2 * ks) = (__bf16)pv;
        }
        if (moved && tt == 0) {
#pragma unroll
          for (int e = 0; e < C::RE; ++e) sm.rs.ra[rrow[e]] = alpha[e];
        }
        if (lane == 0) sm.rs.rf[c] = moved ? 1 : 0;
        lds_barrier();
        // ---- P of rows 16mb + ln16 as the A operand (16 tokens: 4lg .. 4lg+3; 32 tokens: the
        //      k-slot order vtok), and the rows of this lane's accumulators (16mb + 4lg + i),
        //      rescaled first where their reducer wave's reference moved ----
        i32x2 pr[C::MB][C::NTB];
        if constexpr (C::W32) {
          // P of row lane % 32, tokens 8 (lane / 32) .. +8: the 32x32x16 A operand
          const char* pp = sm.rs.rp + (lane & 31) * C::RPS + 16 * (lane >> 5);
          pr[0][0] = ldsr64(pp);
          pr[1][0] = ldsr64(pp + 8);
        } else {
#pragma unroll
          for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
            for (int tb = 0; tb < C::NTB; ++tb)
              pr[mb][tb] = ldsr64(sm.rs.rp + (16 * mb + ln16) * C::RPS + 2 * tok_of(tb, 4 * lg));
        }
        i32x4 f0 = ldsr128(reinterpret_cast<const char*>(&sm.rs.rf[0])), f1 = ldsr128(reinterpret_cast<const char*>(&sm.rs.rf[4]));
        lds_wait(f0, f1);
#pragma unroll
        for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
          for (int tb = 0; tb < C::NTB; ++tb) lds_wait(pr[mb][tb]);
        const int fa = f0[0] | f0[1] | f0[2] | f0[3] | f1[0] | f1[1] | f1[2] | f1[3];
        if (__builtin_amdgcn_readfirstlane(fa)) {
          const int fw[8] = {f0[0], f0[1], f0[2], f0[3], f1[0], f1[1], f1[2], f1[3]};
          if constexpr (C::W32) {
            // rows 8k + 4 (lane / 32) + i of register 4k + i; their reducer wave is 2k + lane / 32
            const int h32 = lane >> 5;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              i32x4 ar = ldsr128(reinterpret_cast<const char*>(&sm.rs.ra[8 * k + 4 * h32]));
              lds_wait(ar);
              const f32x4 al = __builtin_bit_cast(f32x4, ar);
              const int fl = (fw[2 * k + 1] & -h32) | (fw[2 * k] & (h32 - 1));   // no indexed private array
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const float a_i = fl ? al[i] : 1.0f;
#pragma unroll
                for (int j = 0; j < C::CB / 2; ++j) acc32[j][4 * k + i] *= a_i;
              }
            }
          } else {
#pragma unroll
            for (int mb = 0; mb < C::MB; ++mb) {
              i32x4 ar = ldsr128(reinterpret_cast<const char*>(&sm.rs.ra[16 * mb + 4 * lg]));
              lds_wait(ar);
              const f32x4 al = __builtin_bit_cast(f32x4, ar);
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                int fl = 0;   // the flag of row 16mb + 4lg + i's reducer wave
#pragma unroll
                for (int x = 0; x < 8; ++x) fl = (16 * mb + 4 * lg + i) / C::RPW == x ? fw[x] : fl;
                const float a_i = fl ? al[i] : 1.0f;
#pragma unroll
                for (int cb = 0; cb < C::CB; ++cb) acc[mb][cb][i] *= a_i;
              }
            }
          }
        }
        if constexpr (C::W32) pa32 = __builtin_bit_cast(bf16x8, i32x4{pr[0][0][0], pr[0][0][1], pr[1][0][0], pr[1][0][1]});
#pragma unroll
        for (int mb = 0; mb < C::MB; ++mb) {
          if constexpr (C::NTB == 1) {
            pa4[mb] = __builtin_bit_cast(s16x4, pr[mb][0]);
          } else {
            const i32x4 w4 = {pr[mb][0][0], pr[mb][0][1], pr[mb][C::NTB - 1][0], pr[mb][C::NTB - 1][1]};
            pa8[mb] = __builtin_bit_cast(bf16x8, w4);
          }
        }
      } else {
        // ---- sum the NCG partials of (g, tg) in slice order ----
  #pragma unroll
        for (int tb = 0; tb < C::NTB; ++tb)
  #pragma unroll
          for (int mb = 0; mb < C::MB; ++mb) sm.xb[w][tb * C::MB + mb][lane] = sp[tb][mb];
        lds_barrier();
        f32x4 s[C::NTB][C::MB];
        {
          const int w0 = w - c;   // slice 0 of this (g, tg)
  #pragma unroll
          for (int x = 0; x < C::XBW; ++x) {
            f32x4 a;
  #pragma unroll
            for (int v0 = 0; v0 < C::NCG; v0 += 4) {
              i32x4 xr[4];
  #pragma unroll
              for (int j = 0; j < 4; ++j)
                if (v0 + j < C::NCG) xr[j] = ldsr128(reinterpret_cast<const char*>(&sm.xb[w0 + v0 + j][x][lane]));
  #pragma unroll
              for (int j = 0; j < 4; ++j)
                if (v0 + j < C::NCG) {
                  lds_wait(xr[j]);
                  const f32x4 y = __builtin_bit_cast(f32x4, xr[j]);
                  a = (v0 + j == 0) ? y : a + y;
                }
            }
            s[x / C::MB][x % C::MB] = a;
          }
        }
        lds_barrier();   // the partial-score buffer is free again

        // ---- this tile's rms divisors. The rms ring is S+1 deep: the loader refills a stage for
        //      tile t+S only after the first barrier of tile t, by which time every wave has read the
        //      stages of tiles before t; tile t's own stage is not touched ----
        float rinv[C::NTB][C::MB][4];
        if constexpr (C::RMS == QMLA_RMS_NONE) {
  #pragma unroll
          for (int tb = 0; tb < C::NTB; ++tb)
  #pragma unroll
            for (int mb = 0; mb < C::MB; ++mb)
  #pragma unroll
              for (int e = 0; e < 4; ++e) rinv[tb][mb][e] = 1.0f;
        } else {
          const char* rs = sm.rms[t % (C::S + 1)][tg];
          uint32_t code[C::NTB][C::MB][4];
          if constexpr (C::RTR && C::RB == 1) {
            // one tr_b8 read per 16 rows: lane (n, q) gets head rbase+16mb+n of the 8 tokens vtok(q, 0..7)
            i32x2 raw[C::MB];
            const int rr = vtok(lg, ln16 >> 1);
  #pragma unroll
            for (int mb = 0; mb < C::MB; ++mb) raw[mb] = lds_read_tr8_async(rs + rr * C::RRS + rbase + 16 * mb + 8 * (ln16 & 1));
  #pragma unroll
            for (int mb = 0; mb < C::MB; ++mb) {
              lds_wait(raw[mb]);
  #pragma unroll
              for (int e = 0; e < 4; ++e) {
                code[0][mb][e] = ((uint32_t)raw[mb][0] >> (8 * e)) & 0xFF;
                if constexpr (C::NTB == 2) code[1][mb][e] = ((uint32_t)raw[mb][1] >> (8 * e)) & 0xFF;
              }
            }
          } else if constexpr (C::RTR && C::RB == 2) {
            // tr_b16: lanes 4r..4r+3 of a 16-lane block supply token row r; lane n gets head rbase+16mb+n
  #pragma unroll
            for (int tb = 0; tb < C::NTB; ++tb) {
              i32x2 raw[C::MB];
              const int rr = tok_of(tb, 4 * lg + (ln16 >> 2));
  #pragma unroll
              for (int mb = 0; mb < C::MB; ++mb)
                raw[mb] = lds_read_tr16_async(rs + rr * C::RRS + 2 * rbase + 32 * mb + 8 * (ln16 & 3));
  #pragma unroll
              for (int mb = 0; mb < C::MB; ++mb) {
                lds_wait(raw[mb]);
                code[tb][mb][0] = (uint32_t)raw[mb][0] & 0xFFFF;
                code[tb][mb][1] = (uint32_t)raw[mb][0] >> 16;
                code[tb][mb][2] = (uint32_t)raw[mb][1] & 0xFFFF;
                code[tb][mb][3] = (uint32_t)raw[mb][1] >> 16;
              }
            }
          } else {
            // general rows (verify tokens, latent groups): one read per score
  #pragma unroll
            for (int tb = 0; tb < C::NTB; ++tb)
  #pragma unroll
              for (int mb = 0; mb < C::MB; ++mb)
  #pragma unroll
                for (int e = 0; e < 4; ++e) {
                  const char* a = rs + tok_of(tb, 4 * lg + e) * C::RRS + hb[mb];
                  code[tb][mb][e] = C::RB == 1 ? ldsr8(a) : ldsr16(a);
                }
  #pragma unroll
            for (int tb = 0; tb < C::NTB; ++tb)
  #pragma unroll
              for (int mb = 0; mb < C::MB; ++mb)
  #pragma unroll
                for (int e = 0; e < 4; ++e) lds_wait(code[tb][mb][e]);
          }
  #pragma unroll
          for (int tb = 0; tb < C::NTB; ++tb)
  #pragma unroll
            for (int mb = 0; mb < C::MB; ++mb)
  #pragma unroll
              for (int e = 0; e < 4; ++e) {
                const uint32_t cd = code[tb][mb][e];
                float ri;
                if constexpr (C::RMS == QMLA_RMS_LOG8) {
                  // 1 / 2^(-3 + c*6/255) = 2^(3 - c*6/255)  (ops/mla_decode_attention.py:470-479)
                  ri = fast_exp2(fmaf((float)cd, -6.0f / 255.0f, 3.0f));
                } else if constexpr (C::RMS == QMLA_RMS_E4M3) {
                  const float rv = fp8_to_f32(cd) * kscale;
                  ri = rv > 0.f ? __builtin_amdgcn_rcpf(rv) : 1.0f;
                } else {
                  const float rv = bf16_bits_to_f32(cd);
                  ri = rv > 0.f ? __builtin_amdgcn_rcpf(rv) : 1.0f;
                }
                rinv[tb][mb][e] = ri;
              }
        }

        // ---- scale to log2 units, cap, mask; tile max per row ----
        const bool full = tok0 + C::T <= limmin;
        float tmax[C::MB];
  #pragma unroll
        for (int mb = 0; mb < C::MB; ++mb) {
          float m = kNegInf;
  #pragma unroll
          for (int tb = 0; tb < C::NTB; ++tb)
  #pragma unroll
            for (int e = 0; e < 4; ++e) {
              float v = s[tb][mb][e] * rinv[tb][mb][e] * csc;
              if constexpr (C::CAP) {
                // cap * tanh(x / cap) in log2 units: tanh(y) = 1 - 2 / (exp(2y) + 1)
                const float y = v / cap2;
                const float e2 = fast_exp2(2.0f * kLog2e * y);
                v = cap2 * (1.0f - 2.0f / (e2 + 1.0f));
              }
              if (!full && tok0 + tok_of(tb, 4 * lg + e) >= lim[mb]) v = kNegInf;
              s[tb][mb][e] = v;
              m = fmaxf(m, v);
            }
          tmax[mb] = max_lg(m);
        }
        // reference max: it moves when a tile max exceeds it by more than ref_shift(the row's running
        // sum), so a dominant token gets P = 1 exactly as under the reference's running max
        // (ops/mla_decode_attention.py:553-560) and rounding P to bf16 before P.V costs no more
        // than it does there; P <= 2^8
        bool cand = false;
  #pragma unroll
        for (int mb = 0; mb < C::MB; ++mb) cand |= tmax[mb] > mthr[mb];
        if (__builtin_amdgcn_ballot_w64(cand)) {
          bool need = false;
  #pragma unroll
          for (int mb = 0; mb < C::MB; ++mb) {
            mthr[mb] = mref[mb] + ref_shift(sum_lg(lpart[mb]), 8.0f);
            need |= tmax[mb] > mthr[mb];
          }
          if (__builtin_amdgcn_ballot_w64(need)) {
  #pragma unroll
            for (int mb = 0; mb < C::MB; ++mb) {
              const bool mv = tmax[mb] > mthr[mb];
              const float mn = mv ? tmax[mb] : mref[mb];
              const float alpha = mref[mb] == kNegInf ? 0.f : fast_exp2(mref[mb] - mn);
              lpart[mb] *= alpha;
              mref[mb] = mn;
              if (mv) mthr[mb] = mn;   // re-evaluated at the next tile max above the new reference
              // accumulator rows 4*lg + i live in lanes 4*lg + i of the score layout
              float al[4];
  #pragma unroll
              for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * lg + i);
  #pragma unroll
              for (int cb = 0; cb < C::CB; ++cb)
  #pragma unroll
                for (int i = 0; i < 4; ++i) acc[mb][cb][i] *= al[i];
            }
          }
        }

        // ---- P (bf16) in the A layout of P.V, row sums ----
  #pragma unroll
        for (int mb = 0; mb < C::MB; ++mb) {
          const float mu = mref[mb] == kNegInf ? 0.f : mref[mb];
  #pragma unroll
          for (int tb = 0; tb < C::NTB; ++tb)
  #pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float pv = fast_exp2(s[tb][mb][e] - mu);
              lpart[mb] += pv;
              if constexpr (C::NTB == 2) pa8[mb][4 * tb + e] = (__bf16)pv;
              else pa4[mb][e] = __builtin_bit_cast(short, (__bf16)pv);
            }
        }

      }

      // ---- P.V over this wave's columns ----
      if constexpr (C::EB == 1 && C::NTB == 2) {
        // tr_b8: lanes 2r, 2r+1 of block q supply token row vtok(q, r); lane n gets column n
        const char* vb = st + vtok(lg, ln16 >> 1) * C::RS + 8 * (ln16 & 1);
        constexpr int VB = 4;
#pragma unroll
        for (int c0 = 0; c0 < C::CB; c0 += VB) {
          i32x2 vr[VB];
#pragma unroll
          for (int j = 0; j < VB; ++j)
            if (c0 + j < C::CB) vr[j] = lds_read_tr8_async(vb + 16 * (c0 + j));
#pragma unroll
          for (int j = 0; j < VB; ++j)
            if (c0 + j < C::CB) {
              lds_wait(vr[j]);
              const bf16x8 vf = fp8x8_to_bf16(vr[j]);
#pragma unroll
              for (int mb = 0; mb < C::MB; ++mb) acc[mb][c0 + j] = mfma16(pa8[mb], vf, acc[mb][c0 + j]);
            }
        }
      } else if constexpr (C::EB == 1 && C::W32) {
        // 32x32x16: lane block b reads tokens 8 (b / 2) .. +8 of 16-column block a_j (b even) or
        // a_j + d_j (b odd) (tr_b8: lanes 2r, 2r+1 supply token row r), so lane l gets column
        // l % 32 of the pair for the k-slots 8 (l / 32) .. +8
        const int b16 = lane >> 4, li = lane & 15;
        const char* vrow = st + (8 * (b16 >> 1) + (li >> 1)) * C::RS + 8 * (li & 1);
        const uint32_t vbd = lds_addr(vrow + 16 * C::PD * (b16 & 1)), vb1 = lds_addr(vrow + 16 * (b16 & 1));
        constexpr int NJ = C::CB / 2;
        i32x2 vr[NJ];
        sfor<0, NJ>([&](auto j) {
          constexpr int a = C::PAIRS.a[j];
          vr[j] = ldstr8_off<16 * a>(C::PAIRS.d[j] == C::PD ? vbd : vb1);
        });
        sfor<0, NJ>([&](auto j) {
          lds_wait_n<NJ - 1 - j>(vr[j]);
          acc32[j] = mfma32(pa32, fp8x8_to_bf16(vr[j]), acc32[j]);
        });
      } else if constexpr (C::EB == 1) {
        // 16-token tiles: tr_b8 rows r = 0..3 of lane block q are tokens 4q .. 4q+3 of column block
        // 2j, rows 4..7 the same tokens of block 2j+1, so lane n gets both blocks' column n for the
        // k-slots 4q .. 4q+3 of two 16x16x16 products
        const int r8 = ln16 >> 1;
        const uint32_t vb = lds_addr(st + (4 * lg + (r8 & 3)) * C::RS + 16 * (r8 >> 2) + 8 * (ln16 & 1));
        constexpr int NP = C::CB / 2;
        i32x2 vr[NP];
        sfor<0, NP>([&](auto j) { vr[j] = ldstr8_off<32 * j>(vb); });
        sfor<0, NP>([&](auto j) {
          lds_wait_n<NP - 1 - j>(vr[j]);
          const s16x8 v8 = __builtin_bit_cast(s16x8, fp8x8_to_bf16(vr[j]));
          const s16x4 va = {v8[0], v8[1], v8[2], v8[3]}, vc = {v8[4], v8[5], v8[6], v8[7]};
#pragma unroll
          for (int mb = 0; mb < C::MB; ++mb) {
            acc[mb][2 * j] = mfma16k16(pa4[mb], va, acc[mb][2 * j]);
            acc[mb][2 * j + 1] = mfma16k16(pa4[mb], vc, acc[mb][2 * j + 1]);
          }
        });
      } else if constexpr (C::NTB == 2) {
        // tr_b16 twice: k-slots 8q..8q+3 (score tile 0) and 8q+4..8q+7 (score tile 1)
        const char* v0 = st + tok_of(0, 4 * lg + (ln16 >> 2)) * C::RS + 8 * (ln16 & 3);
        const char* v1 = st + tok_of(1, 4 * lg + (ln16 >> 2)) * C::RS + 8 * (ln16 & 3);
        constexpr int VB = 4;
#pragma unroll
        for (int c0 = 0; c0 < C::CB; c0 += VB) {
          i32x2 va[VB], vc[VB];
#pragma unroll
          for (int j = 0; j < VB; ++j)
            if (c0 + j < C::CB) {
              va[j] = lds_read_tr16_async(v0 + 32 * (c0 + j));
              vc[j] = lds_read_tr16_async(v1 + 32 * (c0 + j));
            }
#pragma unroll
          for (int j = 0; j < VB; ++j)
            if (c0 + j < C::CB) {
              lds_wait(va[j], vc[j]);
              const s16x4 a = __builtin_bit_cast(s16x4, va[j]), b = __builtin_bit_cast(s16x4, vc[j]);
              s16x8 ab;
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                ab[e] = a[e];
                ab[4 + e] = b[e];
              }
              const bf16x8 vf = __builtin_bit_cast(bf16x8, ab);
#pragma unroll
              for (int mb = 0; mb < C::MB; ++mb) acc[mb][c0 + j] = mfma16(pa8[mb], vf, acc[mb][c0 + j]);
            }
        }
      } else if constexpr (C::W32) {
        // 32x32x16: lane block b reads token rows 8 (b / 2) + 2r (then + 1) of 16-column block a_j
        // (b even) or a_j + d_j (b odd) (tr_b16: lanes 4r .. 4r+3 supply row r), so lane l gets
        // column l % 32 of the pair for the k-slots 8 (l / 32) .. +8 in the order P was written
        const int b16 = lane >> 4, li = lane & 15;
        const char* vrow = st + (8 * (b16 >> 1) + 2 * (li >> 2)) * C::RS + 8 * (li & 3);
        const uint32_t vbd = lds_addr(vrow + 32 * C::PD * (b16 & 1)), vb1 = lds_addr(vrow + 32 * (b16 & 1));
        constexpr int NJ = C::CB / 2, VB = 4;   // 32-column blocks per batch of reads
        sfor<0, (NJ + VB - 1) / VB>([&](auto bb) {
          constexpr int j0 = VB * bb, nb = NJ - j0 < VB ? NJ - j0 : VB;
          i32x2 va[VB], vc[VB];
          sfor<0, nb>([&](auto j) {
            constexpr int a = C::PAIRS.a[j0 + j];
            const uint32_t v = C::PAIRS.d[j0 + j] == C::PD ? vbd : vb1;
            va[j] = ldstr16_off<32 * a>(v);
            vc[j] = ldstr16_off<32 * a + C::RS>(v);
          });
          sfor<0, nb>([&](auto j) {
            lds_wait_n<2 * (nb - 1 - j)>(vc[j]);
            lds_wait_n<2 * (nb - 1 - j)>(va[j]);
            const bf16x8 vf = __builtin_bit_cast(bf16x8, i32x4{va[j][0], va[j][1], vc[j][0], vc[j][1]});
            acc32[j0 + j] = mfma32(pa32, vf, acc32[j0 + j]);
          });
        });
      } else {
        // lane block q reads tokens 4q .. 4q+3 (tr_b16: lanes 4r .. 4r+3 supply token row r); with
        // the reduce-scatter's P, tokens 2r + 8 (q & 1) + (q >> 1) instead: lanes 0-31 then cover
        // the 8 even rows (the odd ones in lanes 32-63), which with the odd 16-byte row stride
        // touch each LDS bank once instead of twice
        const int vrow = C::RSC ? 2 * (ln16 >> 2) + 8 * (lg & 1) + (lg >> 1) : 4 * lg + (ln16 >> 2);
        const uint32_t vb = lds_addr(st + vrow * C::RS + 8 * (ln16 & 3));
        constexpr int VB = 7;   // column blocks per batch of reads, each used as soon as it is in
        sfor<0, (C::CB + VB - 1) / VB>([&](auto b) {
          constexpr int c0 = VB * b, nb = C::CB - c0 < VB ? C::CB - c0 : VB;
          i32x2 vr[VB];
          sfor<0, nb>([&](auto j) { vr[j] = ldstr16_off<32 * (c0 + j)>(vb); });
          sfor<0, nb>([&](auto j) {
            lds_wait_n<nb - 1 - j>(vr[j]);
            const s16x4 vf = __builtin_bit_cast(s16x4, vr[j]);
#pragma unroll
            for (int mb = 0; mb < C::MB; ++mb) acc[mb][c0 + j] = mfma16k16(pa4[mb], vf, acc[mb][c0 + j]);
          });
        });
      }
      if (t + C::S < nt) issue(t + C::S);
    }
  }
  wait_vmcnt<0>();

  // ---- epilogue: per-row sums; merge the token groups; normalize and write ----
  float lrow[C::MB];
#pragma unroll
  for (int mb = 0; mb < C::MB; ++mb) lrow[mb] = sum_lg(lpart[mb]);
  // reduce-scatter: the reducer waves hand every row's max and sum to the waves holding its columns
  float rls[C::RE];
  if constexpr (C::RSC) {
#pragma unroll
    for (int e = 0; e < C::RE; ++e) {
      rls[e] = sum16(rlp[e]);
      if constexpr (C::T == 32) rls[e] += __shfl_xor(rls[e], 16);
      if (tt == 0) {
        sm.rs.rfin[0][rrow[e]] = rmref[e];
        sm.rs.rfin[1][rrow[e]] = rls[e];
      }
    }
    lds_barrier();
  }
  if constexpr (C::NTG == 2) {
    // token group 1 hands (max, sum, acc) to token group 0 through the (now idle) ring
    lds_barrier();
    float* xa = reinterpret_cast<float*>(&sm.ring[0][0][0]);
    const int slot = w % (C::G * C::NCG);
    float* mine = xa + (size_t)slot * (C::MB * C::CB * 4 + 2 * C::MB) * 64;
    if (tg == 1) {
#pragma unroll
      for (int mb = 0; mb < C::MB; ++mb) {
#pragma unroll
        for (int cb = 0; cb < C::CB; ++cb)
#pragma unroll
          for (int i = 0; i < 4; ++i) mine[((mb * C::CB + cb) * 4 + i) * 64 + lane] = acc[mb][cb][i];
        mine[(C::MB * C::CB * 4 + 2 * mb) * 64 + lane] = mref[mb];
        mine[(C::MB * C::CB * 4 + 2 * mb + 1) * 64 + lane] = lrow[mb];
      }
    }
    lds_barrier();
    if (tg == 1) return;
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb) {
      const float m1 = mine[(C::MB * C::CB * 4 + 2 * mb) * 64 + lane];
      const float l1 = mine[(C::MB * C::CB * 4 + 2 * mb + 1) * 64 + lane];
      const float mm = fmaxf(mref[mb], m1);
      const float a0 = mref[mb] == kNegInf ? 0.f : fast_exp2(mref[mb] - mm);
      const float a1 = m1 == kNegInf ? 0.f : fast_exp2(m1 - mm);
      lrow[mb] = lrow[mb] * a0 + l1 * a1;
      mref[mb] = mm;
      float b0[4], b1[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        b0[i] = __shfl(a0, 4 * lg + i);
        b1[i] = __shfl(a1, 4 * lg + i);
      }
#pragma unroll
      for (int cb = 0; cb < C::CB; ++cb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[mb][cb][i] = acc[mb][cb][i] * b0[i] + mine[((mb * C::CB + cb) * 4 + i) * 64 + lane] * b1[i];
    }
  }
  if constexpr (C::W32) {
    // 32x32 accumulators: register v of lane l holds row 8 (v / 4) + 4 (l / 32) + v % 4, column
    // l % 16 of 16-column block a_j (l % 32 < 16) or a_j + d_j
    const bool ph = !so.final_out && so.plse && p.part_h;
    // the lane index through an empty asm: the rows, heads and offsets below are then computed
    // here, at each range's end, instead of once before the range loop and kept (spilled) across it
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int hi = (ln >> 4) & 1;
    const int cold = c * C::DCW + (ln & 15) + 16 * C::PD * hi, col1 = c * C::DCW + (ln & 15) + 16 * hi;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int rl = 8 * (v >> 2) + 4 * (ln >> 5) + (v & 3);
      const float l_i = sm.rs.rfin[1][rl];
      const float ivv = ph ? inv_sum(1.0f, l_i) : inv_sum(kscale, l_i);
      const int r = rbase + rl;
      if (r >= rows_pg) continue;
      const int jq = r / hpg, hh = r - jq * hpg;
      const int head = g * hpg + hh;
      // element j of this lane's output row: column a_j * 16 + (d_j == PD ? cold : col1)
      auto put = [&](auto* o0, auto cvt) {
        sfor<0, C::CB / 2>([&](auto j) {
          constexpr int a = C::PAIRS.a[j];
          (C::PAIRS.d[j] == C::PD ? o0 + cold : o0 + col1)[16 * a] = cvt(acc32[j][v] * ivv);
        });
      };
      if (so.final_out) {
        const int64_t ob = (int64_t)(row0 + jq) * p.o_sr + (int64_t)head * p.o_sh;
        if (p.out_dt == QMLA_DT_BF16)
          put(reinterpret_cast<__bf16*>(p.out) + ob, [](float x) { return (__bf16)x; });
        else if (p.out_dt == QMLA_DT_F16)
          put(reinterpret_cast<_Float16*>(p.out) + ob, [](float x) { return (_Float16)x; });
        else
          put(reinterpret_cast<float*>(p.out) + ob, [](float x) { return x; });
      } else if (ph) {
        put(reinterpret_cast<_Float16*>(so.po) + (int64_t)jq * so.po_sr + (int64_t)head * so.po_sh,
            [](float x) { return (_Float16)x; });
      } else {
        put(so.po + (int64_t)jq * so.po_sr + (int64_t)head * so.po_sh, [](float x) { return x; });
      }
    }
  } else {
    // the lane's row group and column through an empty asm (as above)
    int lgx = lg, lnx = ln16;
    asm volatile("" : "+v"(lgx), "+v"(lnx));
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb) {
      const float l = lrow[mb];
      const float lse_v = row_lse(mref[mb], l);
      const float inv = inv_sum(kscale, l);   // fp8 values were accumulated unscaled
      const float invh = inv_sum(1.0f, l);    // ... and are stored so as fp16 partials
      const bool ph = !so.final_out && so.plse && p.part_h;
      float iv[4];
      if constexpr (C::RSC) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float l_i = sm.rs.rfin[1][16 * mb + 4 * lgx + i];
          iv[i] = ph ? inv_sum(1.0f, l_i) : inv_sum(kscale, l_i);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) iv[i] = __shfl(ph ? invh : inv, 4 * lgx + i);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = rbase + 16 * mb + 4 * lgx + i;
        if (r >= rows_pg) continue;
        const int jq = r / hpg, hh = r - jq * hpg;
        const int head = g * hpg + hh;
        const int col = c * C::DCW + lnx;
        if (so.final_out) {
          const int64_t ob = (int64_t)(row0 + jq) * p.o_sr + (int64_t)head * p.o_sh + col;
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
        } else if (ph) {
          _Float16* ob = reinterpret_cast<_Float16*>(so.po) + (int64_t)jq * so.po_sr + (int64_t)head * so.po_sh + col;
#pragma unroll
          for (int cb = 0; cb < C::CB; ++cb) ob[16 * cb] = (_Float16)(acc[mb][cb][i] * iv[i]);
        } else {
          float* ob = so.po + (int64_t)jq * so.po_sr + (int64_t)head * so.po_sh + col;
#pragma unroll
          for (int cb = 0; cb < C::CB; ++cb) ob[16 * cb] = acc[mb][cb][i] * iv[i];
        }
      }
      // lse from the score layout (row lnx + 16mb), one lane per row (reduce-scatter: below)
      const int r = rbase + lnx + 16 * mb;
      if (!C::RSC && c == 0 && lgx == 0 && r < rows_pg) {
        const int jq = r / hpg, hh = r - jq * hpg;
        const int head = g * hpg + hh;
        if (so.final_out) {
          if (p.lse) store_out(p.lse, p.lse_dt, (int64_t)(row0 + jq) * p.lse_sr + head, lse_v);
        } else if (so.plse) {
          so.plse[(int64_t)jq * so.plse_sr + head] = lse_v;
        } else {
          so.po[(int64_t)jq * so.po_sr + (int64_t)head * so.po_sh + C::DCG] = lse_v;
        }
      }
    }
  }
  if constexpr (C::RSC) {
    // the reducer lane of each row writes its lse
#pragma unroll
    for (int e = 0; e < C::RE; ++e) {
      const int r = rbase + rrow[e];
      if (tt == 0 && r < rows_pg) {
        const int jq = r / hpg, hh = r - jq * hpg;
        const int head = g * hpg + hh;
        const float lse_v = row_lse(rmref[e], rls[e]);
        if (so.final_out) {
          if (p.lse) store_out(p.lse, p.lse_dt, (int64_t)(row0 + jq) * p.lse_sr + head, lse_v);
        } else if (so.plse) {
          so.plse[(int64_t)jq * so.plse_sr + head] = lse_v;
        } else {
          so.po[(int64_t)jq * so.po_sr + (int64_t)head * so.po_sh + C::DCG] = lse_v;
        }
      }
    }
  }
}

template <class C>
__global__ __launch_bounds__(C::NTHR, 1) void cs_kernel(const KParams p) {
  static_assert(sizeof(Smem<C>) <= 163840, "LDS budget of a workgroup");
  static_assert(C::NTG == 1 || (C::NW / C::NTG) * (C::MB * C::CB * 4 + 2 * C::MB) * 64 * 4 <= C::S * C::NW * C::SB,
                "token-group merge fits in the ring");
  __shared__ __attribute__((aligned(16))) Smem<C> sm;
  // the per-layer scale dequantizes fp8 rows (and e4m3 rms codes); a bf16 cache ignores it, as
  // the reference does (mla_decode_attention.py:451-463)
  const float kscale = (C::EB == 1 && p.k_scale) ? *p.k_scale : 1.0f;
  if (p.num_splits == 0 && blockIdx.x == 0 && blockIdx.z == 0 && threadIdx.x < 64) store_plan<kPlanSwitchOther>(p);   // for the combine
  int bad = 0;
  for_each_segment<C::DCG, kPlanSwitchOther>(p, [&](int req, int a, int e, int L, const SegOut& so) {
    segment<C>(p, sm, req, a, e, L, so, kscale, bad);
    // the next range starts its sub-range set-up with a full barrier; nothing else to reset
  });
  report_pages(p, bad);
}

struct Inst {
  int eb, rms, dcg, g, mb, crm, wp, nthr;
  bool cap, rtr, dw;
  void (*fn)(const KParams);
};

#define QMLA_CSX(EB, RMS, DCG, G, NCG, NTG, NTB, MB, S, CRM, CAP, RTR, WP, DW)                                    \
  {EB, RMS, DCG, G, MB, CRM, WP, CS<EB, RMS, DCG, G, NCG, NTG, NTB, MB, S, CRM, CAP, RTR, WP, DW>::NTHR, CAP, RTR, DW, \
   &cs_kernel<CS<EB, RMS, DCG, G, NCG, NTG, NTB, MB, S, CRM, CAP, RTR, WP, DW>>}
#define QMLA_CS(EB, RMS, DCG, G, NCG, NTG, NTB, MB, S, CRM, CAP, RTR, WP) \
  QMLA_CSX(EB, RMS, DCG, G, NCG, NTG, NTB, MB, S, CRM, CAP, RTR, WP, false)

// One entry per compiled shape; rows [latent | rope | rms | pad].
static const Inst kInst[] = {
    // bf16 cache, d_c 1792 (the reference's two-pass widths): 8 column slices, 16-token tiles
    QMLA_CS(2, QMLA_RMS_BF16, 1792, 1, 8, 1, 1, 2, 2, 4, false, true, 64),
    // ... the same rows with verify tokens (rows are tokens x heads, so the rms codes are read per row;
    // 16 rows per workgroup: 32 spill 66 registers), e.g. 2 tokens x 24 heads over 3 workgroups
    QMLA_CS(2, QMLA_RMS_BF16, 1792, 1, 8, 1, 1, 1, 2, 3, false, false, 64),
    QMLA_CS(2, QMLA_RMS_NONE, 1792, 1, 8, 1, 1, 2, 2, 0, false, false, 64),
    // bf16 cache, rank 768 with a rope window of 256 (the plugin's 24-head rope 232 layout,
    // tests/test_fi_partial_rope.py:105-110, and full rope 256): 8 slices of 96 columns; the
    // per-group kernel's fragments for 24 heads exceed the register file
    QMLA_CS(2, QMLA_RMS_BF16, 768, 1, 8, 1, 1, 2, 4, 3, false, false, 256),
    QMLA_CS(2, QMLA_RMS_BF16, 768, 1, 8, 1, 1, 1, 4, 2, false, false, 256),   // 12 heads, rope 256
    // bf16 cache, rank 1792 with the plugin's partial-rope and full-rope-256 layouts
    // (tests/test_two_pass_1792.py:12-19 on the rows of tests/test_fi_partial_rope.py:27-31): rope 232
    // or 256 (window 256) and rope 116 (window 128, rms tail at 8 mod 16 bytes); two stages of 16
    // tokens. 24 heads in one workgroup per token range (32 rows: the reduce-scatter leaves the tile
    // loop free of spills), 12 heads in 16 rows
    QMLA_CS(2, QMLA_RMS_BF16, 1792, 1, 8, 1, 1, 2, 2, 3, false, false, 256),
    QMLA_CS(2, QMLA_RMS_BF16, 1792, 1, 8, 1, 1, 1, 2, 3, false, false, 256),
    QMLA_CS(2, QMLA_RMS_BF16, 1792, 1, 8, 1, 1, 1, 2, 2, false, false, 256),   // 12 heads: 32-byte tail
    QMLA_CS(2, QMLA_RMS_BF16, 1792, 1, 8, 1, 1, 1, 2, 2, false, false, 128),
    // the unpadded 12-head rows of the reference's numerics test (rank + 256 + 12 bf16 elements:
    // 2072 / 4120 bytes, on 8-byte boundaries, tests/test_decode_numerics.py:60-67): narrow rows
    QMLA_CSX(2, QMLA_RMS_BF16, 768, 1, 8, 1, 1, 1, 3, 2, false, false, 256, true),
    QMLA_CSX(2, QMLA_RMS_BF16, 1792, 1, 8, 1, 1, 1, 2, 2, false, false, 256, true),
    // fp8 cache, d_c 1792, rope 64, log8 codes: 32-token tiles, 16 rows per workgroup, more heads
    // split over gridDim.z (transposed rms reads: 2 chunks cover the heads of two row blocks):
    QMLA_CS(1, QMLA_RMS_LOG8, 1792, 1, 8, 1, 2, 1, 2, 2, false, true, 64),
    // the plugin's deployed fp8 layouts at rank 1792 (tests/test_fp8_kv.py:136-138): rope 116 with
    // 12 heads (window 128) and rope 232 with 24 heads (window 256); log8 / e4m3 / bf16-byte rms
    // tails at offsets that are not 16-byte aligned (general rms reads). 24 heads in one workgroup
    // per token range: 16-token tiles of 32 rows (the ring of 32-token tiles and their partial
    // scores exceed the LDS at 32 rows; the reduce-scatter keeps the tile loop free of spills);
    // 16 rows in 32-token tiles otherwise
    QMLA_CS(1, QMLA_RMS_LOG8, 1792, 1, 8, 1, 2, 1, 2, 1, false, false, 128),
    QMLA_CS(1, QMLA_RMS_E4M3, 1792, 1, 8, 1, 2, 1, 2, 1, false, false, 128),
    QMLA_CS(1, QMLA_RMS_BF16_BYTES, 1792, 1, 8, 1, 2, 1, 2, 2, false, false, 128),
    QMLA_CS(1, QMLA_RMS_LOG8, 1792, 1, 8, 1, 1, 2, 3, 2, false, false, 256),
    QMLA_CS(1, QMLA_RMS_E4M3, 1792, 1, 8, 1, 1, 2, 3, 2, false, false, 256),
    QMLA_CS(1, QMLA_RMS_BF16_BYTES, 1792, 1, 8, 1, 1, 2, 3, 4, false, false, 256),
    QMLA_CS(1, QMLA_RMS_LOG8, 1792, 1, 8, 1, 2, 1, 2, 2, false, false, 256),
    QMLA_CS(1, QMLA_RMS_E4M3, 1792, 1, 8, 1, 2, 1, 2, 2, false, false, 256),
    QMLA_CS(1, QMLA_RMS_BF16_BYTES, 1792, 1, 8, 1, 2, 1, 2, 4, false, false, 256),
};

// workgroups per request along z: its rows in blocks of 16*MB
static int row_splits(const Inst& in, const qmla_decode_params* p) {
  const int rows_pg = p->qrows * (p->heads / p->groups);
  return (rows_pg + 16 * in.mb - 1) / (16 * in.mb);
}

}  // namespace cs

// The instance that serves these params with the fewest workgroups per token range, then the
// fewest row blocks (no idle rows), or -1.
int cs_select(const qmla_decode_params* p) {
  const int eb = p->kv_dtype == QMLA_KV_FP8 ? 1 : 2;
  const int dcg = p->d_c / p->groups;
  const bool cap = p->logit_cap > 0.f;
  const int64_t ts = p->token_stride * eb;
  int best = -1, best_hs = 0;
  for (int i = 0; i < (int)(sizeof(cs::kInst) / sizeof(cs::kInst[0])); ++i) {
    const cs::Inst& in = cs::kInst[i];
    if (in.eb != eb || in.rms != p->rms_mode || in.dcg != dcg || in.g != p->groups || in.cap != cap) continue;
    if (in.dw == rows16(p)) continue;   // narrow-row instances serve exactly the rows off 16-byte boundaries
    const int hs = cs::row_splits(in, p);
    if (hs > 4) continue;   // at most 4 workgroups read each token range
    if (in.rtr && (p->qrows != 1 || p->groups != 1)) continue;
    // rope 64 exactly, or a partial rope inside the instance's padded window
    if (in.wp == 64 ? p->rope_w != 64 : (p->rope_w < 1 || p->rope_w > in.wp)) continue;
    if ((int64_t)p->d_c * eb + (int64_t)in.wp * eb > ts) continue;   // latent + rope window inside the row
    if (ts >= (1 << 24)) continue;                                     // 24-bit row offsets in the DMA issue
    if (in.crm > 0) {
      const int rb = (p->rms_mode == QMLA_RMS_BF16 || p->rms_mode == QMLA_RMS_BF16_BYTES) ? 2 : 1;
      const int64_t roff = (int64_t)p->rms_offset * eb;
      const int64_t delta = roff % 16;   // staged from the 16-byte boundary below the tail
      if (in.rtr && delta) continue;     // transposed reads need an aligned tail
      const int64_t need = in.rtr ? 16 * in.mb * hs * rb : delta + (int64_t)p->heads * rb;   // transposed reads cover 16*MB*hs heads
      if (need > 16 * in.crm || (!in.dw && roff - delta + 16 * in.crm > ts)) continue;
      if (in.dw && roff + (int64_t)p->rms_heads * rb > ts) continue;   // narrow rows load the row stride's bytes only
      if (!in.rtr && delta + (int64_t)p->rms_heads * rb > 16 * in.crm) continue;
    }
    if (best < 0 || hs < best_hs || (hs == best_hs && in.mb < cs::kInst[best].mb)) {
      best = i;
      best_hs = hs;
    }
  }
  return best;
}

int cs_row_splits(const qmla_decode_params* p) {
  const int i = cs_select(p);
  return i >= 0 ? cs::row_splits(cs::kInst[i], p) : 0;
}

int cs_launch(int inst, const qmla_decode_params* p, const KParams& k, int nwg, hipStream_t st) {
  KParams kk = k;
  void* args[] = {&kk};
  const int hs = cs::row_splits(cs::kInst[inst], p);
  dim3 grid = p->num_splits > 0 ? dim3(p->num_splits, k.n_req, hs) : dim3(nwg, 1, hs);
  if (grid.x == 0 || grid.y == 0) return QMLA_OK;
  hipError_t e = hipLaunchKernel((const void*)cs::kInst[inst].fn, grid, dim3(cs::kInst[inst].nthr, 1, 1), args, 0, st);
  return e == hipSuccess ? QMLA_OK : QMLA_ERR_LAUNCH;
}

}  // namespace qmla
