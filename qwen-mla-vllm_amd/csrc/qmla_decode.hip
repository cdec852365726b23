// qmla_decode.hip -- gfx950 (MI355X) absorbed-MLA decode over a paged latent KV cache.
//
// One workgroup = 4 waves (one per SIMD) owns a contiguous token range of one request and ALL of
// its query rows (every head, every spec-verify token, every latent group), so each cached row is
// read from HBM exactly once per call. Per 64-token tile:
//   * the paged rows [latent | rope | rms] stream global -> LDS with 16-byte LDS-DMA loads through
//     an S-stage ring (page ids are DMA'd 2(S-1) tiles ahead so no VGPR waits on the block table);
//   * QK^T on MFMA 16x16x32 bf16: query fragments stay in VGPRs for the whole segment, key
//     fragments come from LDS (fp8 e4m3 rows converted exactly to bf16 in registers, the per-layer
//     scale folded into the fp32 score);
//   * scores are divided by the per-(token, head) rms decoded from the row tail, scaled into the
//     log2 domain, masked (split end, spec-verify causal limit), and fed to an online softmax whose
//     row max / row sum are reduced across the 16 lanes of a row (DPP/permute) and across waves in
//     LDS;
//   * P (bf16) goes through LDS; P.V runs on MFMA with the value fragments read transposed straight
//     from the staged rows by ds_read_b64_tr_b8 / _b16 (no separate V copy), each wave owning a
//     column slice of the latent output.
// Split-K partials use the reference attn_logits layout [rows, heads, S, Dv+1] (fixed mode) or a
// balanced plan where every workgroup gets the same number of tiles (balanced mode), and an
// LSE-weighted combine kernel merges them.
//
// Reference semantics: qwen_mla/ops/mla_decode_attention.py:297-586 (stage 1), :1064-1137 (stage 2),
// :1264-1359 (entry, verify folding); qwen_mla/mla_impl.py:125-145 (rms tail formats).

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <mutex>

#include "qmla.h"
#include "qmla_common.h"
#include "qmla_device.h"

namespace qmla {


// Compile-time shape of one kernel instance.
//   EB   cache element bytes (1 = fp8 e4m3fn, 2 = bf16)
//   RMS  QMLA_RMS_* tail format
//   DCG  latent columns per group, G groups (d_c = G*DCG)
//   WP   rope columns padded to a multiple of 64 (scores read [latent | rope_w], rest masked)
//   MB   16-row MFMA blocks per group (rows per group = qrows * heads/G <= 16*MB)
//   S    LDS ring stages, CPR 16-byte chunks staged per row (LDS row = 16*CPR bytes)
//   TILE tokens per pipeline step (32 or 64), WGPC workgroups resident per compute unit
//   DW   narrow rows: cached rows on 4-byte boundaries only, staged 4 bytes per lane (four DMA
//        instructions per 64 chunks, the same LDS image; two stages, so every wait is for all)
//
// Work split inside a workgroup (4 waves, WPG = 4/G per latent group):
//   scores  the group's (16-token block, 16-row block) items are dealt to its waves so that a
//           wave owns a fixed set of MBW row blocks (MSPLIT = MB/MBW wave sets) and TBW token
//           blocks; its query fragments (B operand) stay in VGPRs for the whole segment.
//   P.V     each wave owns NCOL latent output columns for all rows of its group.
template <int EB_, int RMS_, int DCG_, int WP_, int MB_, int G_, int S_, int CPR_, bool CAP_, int TILE_, int WGPC_,
          int NW_, bool DW_ = false>
struct Cfg {
  static constexpr int EB = EB_, RMS = RMS_, DCG = DCG_, WP = WP_, MB = MB_, G = G_, S = S_;
  static constexpr int NW = NW_, NTHR = 64 * NW_;   // waves per workgroup
  static constexpr int CPR = CPR_;
  static constexpr bool CAP = CAP_, DW = DW_;
  static constexpr int TILE = TILE_, WGPC = WGPC_;
  static constexpr int DC = G * DCG;
  static constexpr int RB = 16 * CPR;              // LDS row stride (bytes)
  static constexpr int STAGE = TILE * RB;          // bytes per stage
  static constexpr int NTB = TILE / 16;            // 16-token blocks per tile
  static constexpr int WPG = NW / G;               // waves per group
  // Row blocks are split across waves only when the token blocks alone cannot occupy every wave
  // (two-per-CU 32-token tiles); otherwise each wave scores all row blocks of its own token blocks,
  // so every staged key row is read from LDS and converted exactly once.
  static constexpr int MSPLIT = (NTB % WPG == 0) ? 1 : ((WPG % MB == 0) ? MB : 1);
  static constexpr int MBW = MB / MSPLIT;          // row blocks per wave (scores)
  static constexpr int WPM = WPG / MSPLIT;         // waves sharing a row-block set
  static constexpr int TBW = NTB / WPM;            // token blocks per wave (scores)
  static constexpr int KQ = (DCG + WP) / 32;       // k-steps of the score product
  static constexpr int KP = KQ / 2;                // k-step pairs (64 columns each)
  static constexpr int NCOL = DCG / WPG;           // output columns per wave
  static constexpr int CB = NCOL / 16;             // 16-column output blocks per wave
  static constexpr int ROWS = 16 * MB;
  static constexpr int PSTRIDE = TILE * 2 + 16;    // bf16 P row stride in LDS (bytes, padded)
  static constexpr int NI = (TILE * CPR + 63) / 64;          // DMA instructions per tile
  static constexpr int NDMA = (NI + NW - 1) / NW;            // ... per wave (at most)
  static_assert(WP % 64 == 0 && DCG % 64 == 0, "64-column pairs");
  static_assert(NW % G == 0 && DCG % (16 * WPG) == 0, "column split");
  static_assert(NTB % WPM == 0 && TBW >= 1, "token-block split");
  static_assert(TILE % 32 == 0 && PLAN_TILE % TILE == 0, "tile");
  static_assert(S >= 2 && CPR >= 16, "ring");
  static_assert(!DW || (S == 2 && 4 * NDMA + 1 < 64), "narrow rows: one tile in flight, within the vmcnt range");
};

// Staged rows are rotated by 16-byte chunks: chunk c of LDS row r sits at position
// (c + (r & 15)) mod CPR. The 608/1200-byte row stride alone puts rows r and r+4 on the same LDS
// banks; with the rotation the 16 rows a K-fragment or V^T read touches start 16*7*r bytes apart
// (mod 256), which is conflict-free.
template <int CPR>
__device__ __forceinline__ int rot_pos(int c, int r) {
  int p = c + (r & 15);
  return p >= CPR ? p - CPR : p;
}
// byte offset of byte b (within the staged row) of LDS row r
template <int CPR>
__device__ __forceinline__ int lds_byte(int r, int b) {
  return r * (16 * CPR) + 16 * rot_pos<CPR>(b >> 4, r) + (b & 15);
}

// DMA instructions wave `wave` issues per tile (instructions i = wave, wave+4, ... < NI)
template <class C>
__device__ __forceinline__ constexpr int dma_per_wave(int wave) {
  return (C::NI - wave + C::NW - 1) / C::NW;
}
// Steady-state wait for tile t: after data(t) each wave has issued S-2 more tile groups (its
// data DMAs, plus one page-id DMA for wave 0), so "vmcnt <= that count" means data(t) and
// everything before it landed.
template <class C>
__device__ __forceinline__ void wait_steady(int wave) {
  // waves issue either ceil(NI/NW) or floor(NI/NW) data DMAs per tile (wave 0 also the page ids)
  if (wave == 0) wait_vmcnt<(C::S - 2) * (dma_per_wave<C>(0) + 1)>();
  else if (dma_per_wave<C>(wave) == dma_per_wave<C>(1)) wait_vmcnt<(C::S - 2) * dma_per_wave<C>(1)>();
  else wait_vmcnt<(C::S - 2) * dma_per_wave<C>(C::NW - 1)>();
}

template <class C>
struct Smem {
  char kv[C::S][C::STAGE];
  int pid[2 * C::S][C::TILE];
  char p[C::G][C::ROWS][C::PSTRIDE];
  float red[2][C::NW][C::ROWS];   // per-wave row max / row sum of the current tile
  float alpha[C::G][C::ROWS];     // accumulator rescale of the current tile (when any row moved)
  float fin[2][C::G][C::ROWS];    // final reference max / sum per row (epilogue)
  int flag[C::NW];
};

// Everything a segment needs to know about where its results go.
// One contiguous token range [tok_a, tok_e) of request `req` (length L), all query rows.
//
// Score layout (S^T = K . Q^T on MFMA): lane (n = row column ln16, lg) of row block mb holds the
// scores of tokens tb*16 + 4*lg + i (i = 0..3) for query row mb*16 + ln16, so the per-row
// softmax reductions over a 16-token block are 3 in-lane ops plus 2 cross-lane steps. The value
// accumulator (O = P . V) keeps the D layout: lane (col ln16, lg) holds rows mb*16 + 4*lg + i.
template <class C>
__device__ __forceinline__ void process_segment(const KParams& p, Smem<C>& sm, int req, int tok_a, int tok_e,
                                                int L, const SegOut& so, float kscale, int& bad) {
  constexpr int TILE = C::TILE;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform -> SGPR
  const int g = wave / C::WPG, wl = wave % C::WPG;
  const int mgrp = wl / C::WPM, wt = wl % C::WPM;   // row-block set and token-block phase (scores)
  const int ln16 = lane & 15, lg = lane >> 4;
  const int qrows = p.qrows, hpg = p.hpg;
  const int nrows = qrows * hpg;  // valid rows per group (verify token x head, token-major)
  // rows [rbase, rbase + ROWS) of the group are this workgroup's: a request with more rows than one
  // workgroup holds splits them over gridDim.z workgroups that read the same token range
  const int rbase = (int)blockIdx.z * C::ROWS;
  const int row0 = req * qrows;   // first flattened query row of this request
  const int* bt = p.bt + (int64_t)(row0 + qrows - 1) * p.bt_stride;
  const int ntiles = (tok_e - tok_a + TILE - 1) / TILE;
  const int P = p.page_size;
  constexpr int RMS_EB = (C::RMS == QMLA_RMS_BF16 || C::RMS == QMLA_RMS_BF16_BYTES) ? 2 : 1;

  // ---- this lane's score rows: (mgrp*MBW + mbl)*16 + ln16 of group g ----
  int rms_b[C::MBW];    // byte offset of the row's rms inside a staged cache row
  int lim_off[C::MBW];  // qrows-1-jq: verify token jq sees the first L-(qrows-1-jq) tokens
#pragma unroll
  for (int mbl = 0; mbl < C::MBW; ++mbl) {
    const int r = rbase + (mgrp * C::MBW + mbl) * 16 + ln16;
    const int rr = r < nrows ? r : nrows - 1;
    const int jq = rr / hpg, h = rr - jq * hpg;
    rms_b[mbl] = p.rms_off_b + (g * hpg + h) * RMS_EB;
    lim_off[mbl] = qrows - 1 - jq;
  }

  // ---- page-id and data DMA issue ----
  // LDS chunk q = 64*i + lane of a stage holds row q / CPR, position q % CPR, i.e. global chunk
  // (position - (row & 15)) mod CPR; its byte offset inside a contiguous tile is fixed per
  // (instruction, lane), so it is computed once here.
  uint32_t doff[C::NDMA];
#pragma unroll
  for (int j = 0; j < C::NDMA; ++j) {
    int q = (wave + C::NW * j) * 64 + lane;
    q = q < TILE * C::CPR ? q : TILE * C::CPR - 1;
    const int r = q / C::CPR, pp = q - r * C::CPR;
    int c = pp - (r & 15);
    c = c < 0 ? c + C::CPR : c;
    doff[j] = (uint32_t)(r * C::RB + 16 * c);
  }
  const bool lane_live_last = (C::NI * 64 == TILE * C::CPR) ||
                              ((wave + C::NW * (C::NDMA - 1)) * 64 + lane < TILE * C::CPR);
  auto issue_pid = [&](int t) {
    int tok = tok_a + t * TILE + lane;
    tok = tok < tok_e ? tok : tok_e - 1;
    if (lane < TILE) dma4(bt + tok / P, reinterpret_cast<char*>(sm.pid[t % (2 * C::S)]));
  };
  auto issue_data = [&](int t) {
    const int tok0 = tok_a + t * TILE;
    const int* pidt = sm.pid[t % (2 * C::S)];
    char* dst = sm.kv[t % C::S];
    if (!C::DW && tok0 / P == (tok0 + TILE - 1) / P && p.token_stride_b == C::RB) {
      // the TILE rows are consecutive in one page: one contiguous block, addressed through a
      // buffer resource so the per-tile cost is scalar (rows past tok_e stay inside the page)
      const int page = checked_page(p, __builtin_amdgcn_readfirstlane(pidt[0]), bad);
      const char* base = p.kv + (int64_t)page * p.page_stride_b + (int64_t)(tok0 % P) * p.token_stride_b;
      const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(base, (uint32_t)(TILE * C::RB));
#pragma unroll
      for (int j = 0; j < C::NDMA; ++j) {
        const int i = wave + C::NW * j;
        if (i < C::NI && (j < C::NDMA - 1 || lane_live_last)) dma16_buf(rsrc, doff[j], dst + i * 1024);
      }
      return;
    }
    int tok = tok0 + (lane < TILE ? lane : TILE - 1);
    tok = tok < tok_e ? tok : tok_e - 1;
    const int64_t off = (int64_t)checked_page(p, pidt[lane < TILE ? lane : TILE - 1], bad) * p.page_stride_b +
                        (int64_t)(tok % P) * p.token_stride_b;
    const int off_lo = (int)(uint32_t)off, off_hi = (int)(uint32_t)((uint64_t)off >> 32);
    if constexpr (C::DW) {
      // instruction i's 64 chunks as four 16-chunk quarters: lane l of quarter s carries the 4 bytes
      // at 4 (l & 3) of LDS chunk 64 i + 16 s + l / 4; bytes past the row (the next row's) are skipped
#pragma unroll
      for (int j = 0; j < C::NDMA; ++j) {
        const int i = wave + C::NW * j;
        if (i < C::NI) {
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            int q = 64 * i + 16 * s + (lane >> 2);
            const bool live = q < TILE * C::CPR;
            q = live ? q : TILE * C::CPR - 1;
            const int r = q / C::CPR, pp = q - r * C::CPR;
            int c = pp - (r & 15);
            c = c < 0 ? c + C::CPR : c;
            const int ib = 16 * c + 4 * (lane & 3);
            const uint32_t lo = (uint32_t)__shfl(off_lo, r), hi = (uint32_t)__shfl(off_hi, r);
            const int64_t roff = (int64_t)(((uint64_t)hi << 32) | lo);
            if (live && ib < p.token_stride_b) dma4(p.kv + roff + ib, dst + i * 1024 + 256 * s);
          }
        }
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < C::NDMA; ++j) {
      const int i = wave + C::NW * j;
      if (i < C::NI) {
        const int tk = (int)(doff[j] / (uint32_t)C::RB), cb = (int)(doff[j] - (uint32_t)tk * C::RB);
        const uint32_t lo = (uint32_t)__shfl(off_lo, tk), hi = (uint32_t)__shfl(off_hi, tk);
        const int64_t roff = (int64_t)(((uint64_t)hi << 32) | lo);
        if (j < C::NDMA - 1 || lane_live_last) dma16(p.kv + roff + cb, dst + i * 1024);
      }
    }
  };

  // ---- query fragments (B operand of S^T): pair jj, lane group lg holds q columns
  //      64*jj + 16*lg .. +16 of query row (mgrp*MBW + mbl)*16 + ln16; zero outside [latent | rope_w) ----
  bf16x8 qf[C::MBW][C::KQ];
#pragma unroll
  for (int mbl = 0; mbl < C::MBW; ++mbl) {
    const int r = rbase + (mgrp * C::MBW + mbl) * 16 + ln16;
    const bool rv = r < nrows;
    const int rr = rv ? r : 0;
    const int jq = rr / hpg, h = rr - jq * hpg;
    const int64_t qrow = row0 + jq, head = g * hpg + h;
    const __bf16* qn = p.q_nope + qrow * p.qn_sr + head * p.qn_sh;
    const __bf16* qp = p.q_pe + qrow * p.qp_sr + head * p.qp_sh;
#pragma unroll
    for (int jj = 0; jj < C::KP; ++jj) {
      const int kcol = 64 * jj + 16 * lg;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        bf16x8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (__bf16)0.0f;
        if (rv) {
          const int col = kcol + 8 * half;
          if (col < C::DCG) {
            v = load_q8(qn + col, p.q_vec);
          } else {
            const int pc = col - C::DCG;
            if (pc + 8 <= p.rope_w) {
              v = load_q8(qp + pc, p.q_vec);
            } else if (pc < p.rope_w) {
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                const int c = pc + e < p.rope_w ? pc + e : p.rope_w - 1;
                const __bf16 x = qp[c];
                v[e] = pc + e < p.rope_w ? x : (__bf16)0.0f;
              }
            }
          }
        }
        qf[mbl][2 * jj + half] = v;
      }
    }
  }

  f32x4 acc[C::MB][C::CB];
#pragma unroll
  for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
    for (int cb = 0; cb < C::CB; ++cb) acc[mb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float mref[C::MBW], l_run[C::MBW];  // per score row (log2-domain reference max, running sum)
#pragma unroll
  for (int mbl = 0; mbl < C::MBW; ++mbl) {
    mref[mbl] = kNegInf;
    l_run[mbl] = 0.f;
  }

  const float c2 = p.sm_scale * kscale * kLog2e;   // raw q.k -> log2-domain score (before /rms)
  const float capc = p.logit_cap;
  const int latent_cols_end = C::DCG + p.rope_w;  // valid score columns (group-local k space)

  // ---- prologue: page ids for tiles 0 .. S-2, wait; then S-1 pseudo-iterations issuing
  //      pid(t + S-1) and data(t) exactly like the steady-state loop below ----
  if (wave == 0) {
#pragma unroll
    for (int t = 0; t < C::S - 1; ++t) issue_pid(t);
  }
  wait_vmcnt<0>();
  lds_barrier();
#pragma unroll
  for (int t = 0; t < C::S - 1; ++t) {
    if (wave == 0) issue_pid(t + C::S - 1);
    if (t < ntiles) issue_data(t);
  }

  for (int t = 0; t < ntiles; ++t) {
    // wait for this wave's DMA of tile t (and everything issued before it), then publish
    if (t + C::S - 2 < ntiles) wait_steady<C>(wave);
    else wait_vmcnt<0>();
    lds_barrier();  // (A) tile t visible; every wave is done with tile t-1
    if (wave == 0) issue_pid(t + 2 * C::S - 2);
    if (t + C::S - 1 < ntiles) issue_data(t + C::S - 1);

    const char* kvs = sm.kv[t % C::S];
    const int tok0 = tok_a + t * TILE;

    // ---- scores S^T = K . Q^T for this wave's (token block, row block) items: every 64-column
    //      pair of the block's rows is read up front, and each row block accumulates on two
    //      independent MFMA chains (even / odd pairs) ----
    f32x4 sacc[C::MBW][C::TBW];
#pragma unroll
    for (int tbi = 0; tbi < C::TBW; ++tbi) {
      const int tb = wt + tbi * C::WPM;
      const int krow = tb * 16 + ln16;
      const char* rowp = kvs + krow * C::RB;
      i32x4 kr0[C::KP], kr1[C::KP];
#pragma unroll
      for (int jj = 0; jj < C::KP; ++jj) {
        const int kcol = 64 * jj + 16 * lg;
        const int cbyte = (kcol < C::DCG ? g * C::DCG + kcol : C::DC + kcol - C::DCG) * C::EB;
        kr0[jj] = lds_read_b128(rowp + 16 * rot_pos<C::CPR>(cbyte >> 4, krow));
        if constexpr (C::EB == 2) kr1[jj] = lds_read_b128(rowp + 16 * rot_pos<C::CPR>((cbyte >> 4) + 1, krow));
      }
      f32x4 s2[C::MBW][2];
#pragma unroll
      for (int mbl = 0; mbl < C::MBW; ++mbl) s2[mbl][0] = s2[mbl][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int jj = 0; jj < C::KP; ++jj) {
        const int kcol = 64 * jj + 16 * lg;
        bf16x8 ka, kb;
        if constexpr (C::EB == 1) {
          fp8x16_to_bf16(kr0[jj], ka, kb);
        } else {
          ka = __builtin_bit_cast(bf16x8, kr0[jj]);
          kb = __builtin_bit_cast(bf16x8, kr1[jj]);
        }
        if (jj * 64 + 64 > C::DCG + (C::WP - 64) && kcol + 16 > latent_cols_end) {
          // columns past the rope width (padding up to a 64-column pair): zero them so
          // whatever bytes follow the rope (rms codes, padding) cannot leak NaN into scores
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            if (kcol + e >= latent_cols_end) ka[e] = (__bf16)0.0f;
            if (kcol + 8 + e >= latent_cols_end) kb[e] = (__bf16)0.0f;
          }
        }
#pragma unroll
        for (int mbl = 0; mbl < C::MBW; ++mbl) {
          s2[mbl][jj & 1] = mfma16(ka, qf[mbl][2 * jj], s2[mbl][jj & 1]);
          s2[mbl][jj & 1] = mfma16(kb, qf[mbl][2 * jj + 1], s2[mbl][jj & 1]);
        }
      }
#pragma unroll
      for (int mbl = 0; mbl < C::MBW; ++mbl) sacc[mbl][tbi] = s2[mbl][0] + s2[mbl][1];
    }

    // ---- rms divisors of this lane's (token, row) scores, read before the V^T reads go out ----
    float rinv_t[C::TBW][4][C::MBW];
#pragma unroll
    for (int tbi = 0; tbi < C::TBW; ++tbi) {
      const int tb = wt + tbi * C::WPM;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tt = tb * 16 + 4 * lg + i;
#pragma unroll
        for (int mbl = 0; mbl < C::MBW; ++mbl) {
          float rinv = 1.0f;
          if constexpr (C::RMS != QMLA_RMS_NONE) {
            const char* rp = kvs + lds_byte<C::CPR>(tt, rms_b[mbl]);
            if constexpr (C::RMS == QMLA_RMS_LOG8) {
              const float code = (float)(uint32_t)(uint8_t)rp[0];
              rinv = fast_exp2(3.0f - code * (6.0f / 255.0f));
            } else if constexpr (C::RMS == QMLA_RMS_BF16 || C::RMS == QMLA_RMS_BF16_BYTES) {
              const float r = bf16_bits_to_f32(*reinterpret_cast<const uint16_t*>(rp));
              rinv = r > 0.f ? __builtin_amdgcn_rcpf(r) : 1.0f;
            } else if constexpr (C::RMS == QMLA_RMS_E4M3) {
              const float r = fp8_to_f32((uint8_t)rp[0]) * kscale;
              rinv = r > 0.f ? __builtin_amdgcn_rcpf(r) : 1.0f;
            }
          }
          rinv_t[tbi][i][mbl] = rinv;
        }
      }
    }

    // ---- value fragments for P.V, read transposed from the staged rows; they complete while
    //      the softmax below runs ----
    i32x2 vraw[TILE / 32][C::CB][C::EB];
#pragma unroll
    for (int kk = 0; kk < TILE / 32; ++kk)
#pragma unroll
      for (int cb = 0; cb < C::CB; ++cb) {
        const int col0 = g * C::DCG + wl * C::NCOL + cb * 16;
        if constexpr (C::EB == 1) {
          const int vr = kk * 32 + 8 * lg + (ln16 >> 1);
          vraw[kk][cb][0] = lds_read_tr8_async(kvs + lds_byte<C::CPR>(vr, col0 + 8 * (ln16 & 1)));
        } else {
          const int vr = kk * 32 + 8 * lg + (ln16 >> 2);
          const int vb = (col0 + 4 * (ln16 & 3)) * 2;
          vraw[kk][cb][0] = lds_read_tr16_async(kvs + lds_byte<C::CPR>(vr, vb));
          vraw[kk][cb][C::EB - 1] = lds_read_tr16_async(kvs + lds_byte<C::CPR>(vr + 4, vb));
        }
      }

    // ---- divide by rms, scale to log2 units, mask; tile max per score row ----
    float lmax[C::MBW];
#pragma unroll
    for (int mbl = 0; mbl < C::MBW; ++mbl) lmax[mbl] = kNegInf;
#pragma unroll
    for (int tbi = 0; tbi < C::TBW; ++tbi) {
      const int tb = wt + tbi * C::WPM;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tok = tok0 + tb * 16 + 4 * lg + i;
#pragma unroll
        for (int mbl = 0; mbl < C::MBW; ++mbl) {
          const float rinv = rinv_t[tbi][i][mbl];
          float v;
          if constexpr (C::CAP) {
            const float sn = sacc[mbl][tbi][i] * (c2 * kLn2) * rinv;   // natural-unit score
            const float x = sn / capc;
            const float th = 1.0f - 2.0f / (fast_exp2(2.0f * kLog2e * x) + 1.0f);
            v = capc * th * kLog2e;
          } else {
            v = sacc[mbl][tbi][i] * c2 * rinv;
          }
          int lim = tok_e;
          if (qrows > 1) { const int lv = L - lim_off[mbl]; lim = lv < lim ? lv : lim; }
          v = tok < lim ? v : kNegInf;
          sacc[mbl][tbi][i] = v;
          lmax[mbl] = fmaxf(lmax[mbl], v);
        }
      }
    }
#pragma unroll
    for (int mbl = 0; mbl < C::MBW; ++mbl) lmax[mbl] = max_lg(lmax[mbl]);

    // ---- optimistic softmax: P = exp2(s - mref) with the reference max of earlier tiles. A row
    //      whose tile max exceeds it by more than ref_shift(its running sum) (or that had no max
    //      yet) raises the flag; then every wave rebuilds its P block against the rows' new maxima
    //      (a second exchange) and the accumulator is rescaled. A dominant token thus gets P = 1
    //      exactly, as the running max of the reference's online softmax gives it
    //      (ops/mla_decode_attention.py:553-560), and the bf16 rounding of P before P.V costs no
    //      more than it does there. ----
    float psum[C::MBW];
    auto write_p = [&]() {
#pragma unroll
      for (int mbl = 0; mbl < C::MBW; ++mbl) psum[mbl] = 0.f;
#pragma unroll
      for (int tbi = 0; tbi < C::TBW; ++tbi) {
        const int tb = wt + tbi * C::WPM;
#pragma unroll
        for (int mbl = 0; mbl < C::MBW; ++mbl) {
          const float sh = mref[mbl] == kNegInf ? 0.f : mref[mbl];
          bf16x4 pk;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float e = fast_exp2(sacc[mbl][tbi][i] - sh);
            psum[mbl] += e;
            pk[i] = (__bf16)e;
          }
          *reinterpret_cast<bf16x4*>(&sm.p[g][(mgrp * C::MBW + mbl) * 16 + ln16][(tb * 16 + 4 * lg) * 2]) = pk;
        }
      }
#pragma unroll
      for (int mbl = 0; mbl < C::MBW; ++mbl) psum[mbl] = sum_lg(psum[mbl]);
    };
    bool need = false;
#pragma unroll
    for (int mbl = 0; mbl < C::MBW; ++mbl) need |= lmax[mbl] > mref[mbl] + ref_shift(l_run[mbl], 8.0f);
    const bool need_w = __builtin_amdgcn_ballot_w64(need) != 0;
    if (!need_w) write_p();
    if (lg == 0) {
#pragma unroll
      for (int mbl = 0; mbl < C::MBW; ++mbl) {
        sm.red[0][wave][(mgrp * C::MBW + mbl) * 16 + ln16] = lmax[mbl];
        if (!need_w) sm.red[1][wave][(mgrp * C::MBW + mbl) * 16 + ln16] = psum[mbl];
      }
    }
    if (lane == 0) sm.flag[wave] = need_w ? 1 : 0;
    lds_barrier();  // (B)
    int anyf = 0;
#pragma unroll
    for (int w = 0; w < C::NW; ++w) anyf |= sm.flag[w];
    const bool any = anyf != 0;
    float alpha[C::MBW];
    if (any) {
#pragma unroll
      for (int mbl = 0; mbl < C::MBW; ++mbl) {
        const int r = (mgrp * C::MBW + mbl) * 16 + ln16;
        float gm = mref[mbl];
#pragma unroll
        for (int w = 0; w < C::WPM; ++w) gm = fmaxf(gm, sm.red[0][g * C::WPG + mgrp * C::WPM + w][r]);
        alpha[mbl] = mref[mbl] == kNegInf ? 0.f : fast_exp2(mref[mbl] - gm);
        mref[mbl] = gm;
        if (wt == 0 && lg == 0) sm.alpha[g][r] = alpha[mbl];
      }
      write_p();
      if (lg == 0) {
#pragma unroll
        for (int mbl = 0; mbl < C::MBW; ++mbl) sm.red[1][wave][(mgrp * C::MBW + mbl) * 16 + ln16] = psum[mbl];
      }
      lds_barrier();  // (B')
    } else {
#pragma unroll
      for (int mbl = 0; mbl < C::MBW; ++mbl) alpha[mbl] = 1.0f;
    }
#pragma unroll
    for (int mbl = 0; mbl < C::MBW; ++mbl) {
      float ts = 0.f;
#pragma unroll
      for (int w = 0; w < C::WPM; ++w) ts += sm.red[1][g * C::WPG + mgrp * C::WPM + w][(mgrp * C::MBW + mbl) * 16 + ln16];
      l_run[mbl] = l_run[mbl] * alpha[mbl] + ts;
    }
    if (any) {
      // rescale every accumulator row of the group (row owners published alpha before B')
#pragma unroll
      for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float a = sm.alpha[g][mb * 16 + 4 * lg + i];
#pragma unroll
          for (int cb = 0; cb < C::CB; ++cb) acc[mb][cb][i] *= a;
        }
    }

    // ---- P.V: wave owns columns [g*DCG + wl*NCOL, +NCOL) for all rows of its group ----
#pragma unroll
    for (int kk = 0; kk < TILE / 32; ++kk) {
      bf16x8 pf[C::MB];
#pragma unroll
      for (int mb = 0; mb < C::MB; ++mb)
        pf[mb] = *reinterpret_cast<const bf16x8*>(&sm.p[g][mb * 16 + ln16][(kk * 32 + 8 * lg) * 2]);
#pragma unroll
      for (int cb = 0; cb < C::CB; ++cb) {
        i32x2 c0 = vraw[kk][cb][0], c1 = vraw[kk][cb][C::EB - 1];
        if constexpr (C::EB == 1) lds_wait(c0);
        else lds_wait(c0, c1);
        bf16x8 vf;
        if constexpr (C::EB == 1) {
          vf = fp8x8_to_bf16(c0);
        } else {
          const i16x4 v0 = __builtin_bit_cast(i16x4, c0), v1 = __builtin_bit_cast(i16x4, c1);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            vf[e] = __builtin_bit_cast(__bf16, (short)v0[e]);
            vf[4 + e] = __builtin_bit_cast(__bf16, (short)v1[e]);
          }
        }
#pragma unroll
        for (int mb = 0; mb < C::MB; ++mb) acc[mb][cb] = mfma16(pf[mb], vf, acc[mb][cb]);
      }
    }
  }
  wait_vmcnt<0>();  // trailing page-id loads must land before the LDS ring is reused

  // ---- epilogue: the row owners publish (reference max, sum); every wave normalizes its
  //      columns and writes the output (final or partial) and natural-log lse ----
  if (wt == 0 && lg == 0) {
#pragma unroll
    for (int mbl = 0; mbl < C::MBW; ++mbl) {
      sm.fin[0][g][(mgrp * C::MBW + mbl) * 16 + ln16] = mref[mbl];
      sm.fin[1][g][(mgrp * C::MBW + mbl) * 16 + ln16] = l_run[mbl];
    }
  }
  lds_barrier();
#pragma unroll
  for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = mb * 16 + 4 * lg + i;   // row of the workgroup; rbase + r of the group
      if (rbase + r >= nrows) continue;
      const float m = sm.fin[0][g][r];
      const float l = sm.fin[1][g][r];
      const int jq = (rbase + r) / hpg, h = rbase + r - jq * hpg;
      const int head = g * hpg + h;
      const float inv = inv_sum(kscale, l);   // fp8 values were accumulated unscaled
      const float invh = inv_sum(1.0f, l);    // ... and are stored so as fp16 partials
      const float lse_v = row_lse(m, l);
      if (so.final_out) {
        const int64_t ob = (int64_t)(row0 + jq) * p.o_sr + (int64_t)head * p.o_sh + wl * C::NCOL + ln16;
#pragma unroll
        for (int cb = 0; cb < C::CB; ++cb) store_out(p.out, p.out_dt, ob + cb * 16, acc[mb][cb][i] * inv);
        if (wl == 0 && ln16 == 0 && p.lse)
          store_out(p.lse, p.lse_dt, (int64_t)(row0 + jq) * p.lse_sr + head, lse_v);
      } else if (so.plse && p.part_h) {
        _Float16* ob = reinterpret_cast<_Float16*>(so.po) + (int64_t)jq * so.po_sr + (int64_t)head * so.po_sh + wl * C::NCOL + ln16;
#pragma unroll
        for (int cb = 0; cb < C::CB; ++cb) ob[cb * 16] = (_Float16)(acc[mb][cb][i] * invh);
        if (wl == 0 && ln16 == 0) so.plse[(int64_t)jq * so.plse_sr + head] = lse_v;
      } else {
        float* ob = so.po + (int64_t)jq * so.po_sr + (int64_t)head * so.po_sh + wl * C::NCOL + ln16;
#pragma unroll
        for (int cb = 0; cb < C::CB; ++cb) ob[cb * 16] = acc[mb][cb][i] * inv;
        if (wl == 0 && ln16 == 0) {
          if (so.plse) so.plse[(int64_t)jq * so.plse_sr + head] = lse_v;
          else so.po[(int64_t)jq * so.po_sr + (int64_t)head * so.po_sh + C::DCG] = lse_v;
        }
      }
    }
  lds_barrier();  // LDS ring and P buffers free for the next segment
}

template <class C>
__global__ __launch_bounds__(C::NTHR, C::WGPC) void partial_kernel(const KParams p) {
  __shared__ __attribute__((aligned(16))) Smem<C> sm;
  // the per-layer scale dequantizes fp8 rows (and e4m3 rms codes); a bf16 cache ignores it, as
  // the reference does (mla_decode_attention.py:451-463)
  const float kscale = (C::EB == 1 && p.k_scale) ? *p.k_scale : 1.0f;
  if (p.num_splits == 0 && blockIdx.x == 0 && blockIdx.z == 0 && threadIdx.x < 64) store_plan<kPlanSwitchOther>(p);   // for the combine
  int bad = 0;
  for_each_segment<C::DCG, kPlanSwitchOther>(p, [&](int req, int a, int e, int L, const SegOut& so) {
    process_segment<C>(p, sm, req, a, e, L, so, kscale, bad);
  });
  report_pages(p, bad);
}

// Balanced plan: tiles per request, prefix sums, per-workgroup chunk. One workgroup.
__global__ __launch_bounds__(1024) void plan_kernel(const int* seq_lens, int n_req, int qrows, int nwg,
                                                    int plan_sw, int* plan) {
  __shared__ int wsum[16];
  __shared__ int carry;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  if (tid == 0) carry = 0;
  __syncthreads();
  for (int base = 0; base < n_req; base += 1024) {
    const int b = base + tid;
    int n = 0;
    if (b < n_req) {
      int L = seq_lens[(int64_t)b * qrows + qrows - 1];
      n = L > 0 ? (L + PLAN_TILE - 1) / PLAN_TILE + plan_sw : 0;
    }
    // inclusive wave scan
    int x = n;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o);
      if (lane >= o) x += y;
    }
    if (lane == 63) wsum[wv] = x;
    __syncthreads();
    int before = carry;
    for (int k = 0; k < wv; ++k) before += wsum[k];
    if (b < n_req) plan[2 + b] = before + x - n;  // exclusive prefix
    __syncthreads();
    if (tid == 0) {
      int t = carry;
      for (int k = 0; k < 16; ++k) t += wsum[k];
      carry = t;
      for (int k = 0; k < 16; ++k) wsum[k] = 0;
    }
    __syncthreads();
  }
  if (tid == 0) {
    const int total = carry;
    plan[2 + n_req] = total;
    plan[1] = total;
    plan[0] = total > 0 ? (total + nwg - 1) / nwg : 1;
  }
}

// LSE-weighted combine, fixed-split mode (mla_decode_attention.py:1064-1137): one 256-thread
// workgroup per (row, head). Split bounds are recomputed exactly as in the partial pass; the live
// splits are a prefix [0, nl) (a split is empty only when it starts at or past L). Their weights
// exp(lse_s - M) / sum are formed once in LDS, then every thread streams its output columns over
// the live splits, four splits per batch of loads. Empty splits are never read.
constexpr int CF_MAXS = 1024;   // split count limit of the fixed-mode combine
__global__ __launch_bounds__(256) void combine_kernel(const KParams p, int dv) {
  const int head = blockIdx.x, row = blockIdx.y;   // row = flattened query row
  const int tid = threadIdx.x;
  const int req = row / p.qrows;
  const int L = req_len(p, req);
  __shared__ float s_w[CF_MAXS];
  __shared__ float s_red[2][4];
  int per = (L + p.num_splits - 1) / p.num_splits;
  if (p.split_align > 0) per = (per + p.split_align - 1) / p.split_align * p.split_align;
  const int nl = per > 0 ? ((L + per - 1) / per < p.num_splits ? (L + per - 1) / per : p.num_splits) : 0;
  const int64_t obase = (int64_t)row * p.o_sr + (int64_t)head * p.o_sh;
  if (nl == 0) {   // empty row: zero output, -inf lse
    for (int c = tid; c < dv; c += 256) store_out(p.out, p.out_dt, obase + c, 0.f);
    if (tid == 0 && p.lse) store_out(p.lse, p.lse_dt, (int64_t)row * p.lse_sr + head, kNegInf);
    return;
  }
  const float* base = p.ws + (int64_t)row * p.ws_sr + (int64_t)head * p.ws_sh;
  // split LSEs -> max -> weights
  float mloc = kNegInf;
  for (int s = tid; s < nl; s += 256) {
    const float v = base[(int64_t)s * p.ws_ss + dv];
    s_w[s] = v;
    mloc = fmaxf(mloc, v);
  }
  for (int o = 32; o > 0; o >>= 1) mloc = fmaxf(mloc, __shfl_xor(mloc, o));
  if ((tid & 63) == 0) s_red[0][tid >> 6] = mloc;
  __syncthreads();
  const float m = fmaxf(fmaxf(s_red[0][0], s_red[0][1]), fmaxf(s_red[0][2], s_red[0][3]));
  float sloc = 0.f;
  for (int s = tid; s < nl; s += 256) {
    // a split without tokens (lse -inf) weighs 0; a NaN lse stays NaN (fmaxf above skipped it)
    const float e = is_neg_inf(s_w[s]) ? 0.f : __expf(s_w[s] - m);
    s_w[s] = e;
    sloc += e;
  }
  for (int o = 32; o > 0; o >>= 1) sloc += __shfl_xor(sloc, o);
  if ((tid & 63) == 0) s_red[1][tid >> 6] = sloc;
  __syncthreads();
  const float l = (s_red[1][0] + s_red[1][1]) + (s_red[1][2] + s_red[1][3]);
  const float inv = inv_sum(1.0f, l);
  if (tid == 0 && p.lse) store_out(p.lse, p.lse_dt, (int64_t)row * p.lse_sr + head, empty_sum(l) ? kNegInf : m + __logf(l));
  for (int c = tid; c < dv; c += 256) {
    float acc = 0.f;
    int s = 0;
    for (; s + 4 <= nl; s += 4) {
      float x[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) x[k] = base[(int64_t)(s + k) * p.ws_ss + c];
#pragma unroll
      for (int k = 0; k < 4; ++k) acc += s_w[s + k] * x[k];
    }
    for (; s < nl; ++s) acc += s_w[s] * base[(int64_t)s * p.ws_ss + c];
    store_out(p.out, p.out_dt, obase + c, acc * inv);
  }
}

// LSE-weighted combine, balanced mode: one 256-thread workgroup per (query row, block of CH_HB
// heads). Request b's partials sit in slots w + b for the workgroups w0..w1 that touched it; a
// request covered by one workgroup was finished by the partial pass and is skipped here. Every
// thread owns two adjacent output columns of the CH_HB heads and combines the segments CH_NS at a
// time with a running maximum: the segment LSEs (the same for all threads) and the partial outputs
// of a batch are loaded together, so a batch costs one memory round trip and no barrier. Two heads
// per workgroup: at 128 x 24 rows the merge took 11.0 us against 11.9 (4 heads) and 15.1 (8 heads).
constexpr int CH_HB = 2;
constexpr int CH_NS = 4;   // segments per batch of loads
// the columns of one (row, head block): H = fp16 partials without the fp8 scale, osc applies it;
// NC adjacent columns per thread (2, or 8 for the wide latent rows, whose partials are then read
// 16 or 32 bytes a load instead of 4 or 8, in one pass over the columns instead of four), NS
// segments per batch of loads
template <bool H, int NC, int HB, int NS = CH_NS>
__device__ __forceinline__ void combine_cols(const KParams& p, int dv, int row, int jq, int req, int h0, int nh,
                                             int w0, int nseg) {
  const int tid = threadIdx.x;
  const int64_t nrow = (int64_t)p.qrows * p.heads;
  const int rl0 = jq * p.heads + h0;
  const float osc = H && p.k_scale ? *p.k_scale : 1.0f;
  for (int cb = NC * tid; cb < dv; cb += NC * 256) {
    float m[HB], l[HB], a[HB][NC];
#pragma unroll
    for (int h = 0; h < HB; ++h) {
      m[h] = kNegInf, l[h] = 0.f;
#pragma unroll
      for (int c = 0; c < NC; ++c) a[h][c] = 0.f;
    }
    for (int s0 = 0; s0 < nseg; s0 += NS) {
      float ls[NS][HB];
      float v[NS][HB][NC];
#pragma unroll
      for (int k = 0; k < NS; ++k) {
        const int sg = s0 + k < nseg ? s0 + k : nseg - 1;   // past the end: a valid slot, weight 0
        const int64_t slot = (int64_t)w0 + sg + req;
        const float* pl = p.part_lse + slot * nrow + rl0;
#pragma unroll
        for (int h = 0; h < HB; ++h) {
          const int hh = h < nh ? h : 0;
          ls[k][h] = s0 + k < nseg ? pl[hh] : kNegInf;
          const int64_t e = (slot * nrow + rl0 + hh) * (int64_t)dv + cb;   // the slot's element
          if constexpr (H) {
            // fp16 partials: the slot's rows at the start of its (fp32-sized) area
            const _Float16* src = reinterpret_cast<const _Float16*>(p.part_o + slot * nrow * (int64_t)dv) +
                                  (e - slot * nrow * (int64_t)dv);
            if constexpr (NC == 2) {
              const f16x2 t = *reinterpret_cast<const f16x2*>(src);
              v[k][h][0] = (float)t[0];
              v[k][h][1] = (float)t[1];
            } else {
              const f16x8 t = *reinterpret_cast<const f16x8*>(src);
#pragma unroll
              for (int c = 0; c < 8; ++c) v[k][h][c] = (float)t[c];
            }
          } else {
            if constexpr (NC == 2) {
              const float2 t = *reinterpret_cast<const float2*>(p.part_o + e);
              v[k][h][0] = t.x;
              v[k][h][1] = t.y;
            } else {
              const f32x4 t0 = *reinterpret_cast<const f32x4*>(p.part_o + e);
              const f32x4 t1 = *reinterpret_cast<const f32x4*>(p.part_o + e + 4);
#pragma unroll
              for (int c = 0; c < 4; ++c) {
                v[k][h][c] = t0[c];
                v[k][h][4 + c] = t1[c];
              }
            }
          }
        }
      }
#pragma unroll
      for (int h = 0; h < HB; ++h) {
        // segments without tokens (lse -inf) weigh 0 and a batch of them only is skipped; a NaN lse
        // (fmaxf skips it) weighs NaN, so a row whose inputs hold a NaN merges to NaN
        float mm = m[h];
        bool live = false;
#pragma unroll
        for (int k = 0; k < NS; ++k) {
          mm = fmaxf(mm, ls[k][h]);
          live |= !is_neg_inf(ls[k][h]);
        }
        if (!live) continue;
        const float sc = m[h] == kNegInf ? 0.f : __expf(m[h] - mm);
        l[h] *= sc;
#pragma unroll
        for (int c = 0; c < NC; ++c) a[h][c] *= sc;
#pragma unroll
        for (int k = 0; k < NS; ++k) {
          const float wgt = is_neg_inf(ls[k][h]) ? 0.f : __expf(ls[k][h] - mm);
          l[h] += wgt;
#pragma unroll
          for (int c = 0; c < NC; ++c) a[h][c] += wgt * v[k][h][c];
        }
        m[h] = mm;
      }
    }
#pragma unroll
    for (int h = 0; h < HB; ++h) {
      if (h >= nh) continue;
      const float inv = inv_sum(osc, l[h]);
      const int64_t ob = (int64_t)row * p.o_sr + (int64_t)(h0 + h) * p.o_sh + cb;
#pragma unroll
      for (int c = 0; c < NC; ++c)
        if (cb + c < dv) store_out(p.out, p.out_dt, ob + c, a[h][c] * inv);
      if (cb == 0 && p.lse) store_out(p.lse, p.lse_dt, (int64_t)row * p.lse_sr + h0 + h, empty_sum(l[h]) ? kNegInf : m[h] + __logf(l[h]));
    }
  }
}

// HB heads per workgroup: CH_HB, or 1 on the wide latent rows (d_c 1792 rank 1792, combine stage
// bf16 / fp8 rows: 18.9 / 18.6 us with 2 heads, 17.4 / 16.9 with 1, 21.5 / 22.4 with 4)
template <int HB>
__global__ __launch_bounds__(256) void combine_bal_kernel(const KParams p, int dv) {
  const int hblk = blockIdx.x, row = blockIdx.y;
  const int tid = threadIdx.x;
  const int req = row / p.qrows, jq = row - req * p.qrows;
  const int h0 = hblk * HB;
  const int nh = p.heads - h0 < HB ? p.heads - h0 : HB;
  const int chunk = p.plan[0];
  const int c0 = p.plan[2 + req], c1 = p.plan[3 + req];
  if (c1 <= c0) {  // empty request: zero output, -inf lse
    for (int h = 0; h < nh; ++h)
      for (int c = tid; c < dv; c += 256)
        store_out(p.out, p.out_dt, (int64_t)row * p.o_sr + (int64_t)(h0 + h) * p.o_sh + c, 0.f);
    if (tid < nh && p.lse) store_out(p.lse, p.lse_dt, (int64_t)row * p.lse_sr + h0 + tid, kNegInf);
    return;
  }
  // the first workgroup with tokens of the request holds its first token's tile (c0 + plan_sw)
  const int w0 = (c0 + p.plan_sw) / chunk, w1 = (c1 - 1) / chunk;
  if (w0 == w1) return;
  const int nseg = w1 - w0 + 1;
  // the wide latent rows: 8 columns a thread (partials 16-byte aligned: dv % 8). Measured at d_c
  // 1792 (combine stage, bf16 / fp8 rows): 25.4 / 23.8 us with 2 columns, 18.8 / 18.9 with 8; 8
  // segments a batch instead of 4: 19.0 / 22.3
  const bool w8 = dv > 1024 && dv % 8 == 0;
  if (p.part_h) {
    if (w8) combine_cols<true, 8, HB>(p, dv, row, jq, req, h0, nh, w0, nseg);
    else combine_cols<true, 2, HB>(p, dv, row, jq, req, h0, nh, w0, nseg);
  } else {
    if (w8) combine_cols<false, 8, HB>(p, dv, row, jq, req, h0, nh, w0, nseg);
    else combine_cols<false, 2, HB>(p, dv, row, jq, req, h0, nh, w0, nseg);
  }
}

}  // namespace qmla

// ================================================================================================
// host side: validation, instance selection, launches, C ABI
// ================================================================================================
namespace qmla {

typedef void (*PartialFn)(const KParams);

struct Inst {
  int eb, rms, dcg, wp, mb, g, s, cpr;
  bool cap;
  int tile, wgpc, nthr;
  PartialFn fn;
  bool dw;
};

#define QMLA_INST(EB, RMS, DCG, WP, MB, G, S, CPR, CAP, TILE, WGPC, NW)                    \
  {EB, RMS, DCG, WP, MB, G, S, CPR, CAP, TILE, WGPC, 64 * NW,                                \
   &partial_kernel<Cfg<EB, RMS, DCG, WP, MB, G, S, CPR, CAP, TILE, WGPC, NW>>, false}
#define QMLA_INST_DW(EB, RMS, DCG, WP, MB, G, S, CPR, CAP, TILE, WGPC, NW) \
  {EB, RMS, DCG, WP, MB, G, S, CPR, CAP, TILE, WGPC, 64 * NW,             \
   &partial_kernel<Cfg<EB, RMS, DCG, WP, MB, G, S, CPR, CAP, TILE, WGPC, NW, true>>, true}

// One entry per compiled shape. Rows are [latent | rope | rms | pad]; CPR*16 bytes are staged.
static const Inst kInst[] = {
    // fp8 e4m3 cache + log8 rms codes, d_c 512, rope 64, up to 32 rows (24 heads): 608 B staged
    QMLA_INST(1, QMLA_RMS_LOG8, 512, 64, 2, 1, 3, 38, false, 64, 1, 8),
    QMLA_INST(1, QMLA_RMS_LOG8, 512, 64, 2, 1, 3, 38, false, 64, 1, 4),
    QMLA_INST(1, QMLA_RMS_LOG8, 512, 64, 2, 1, 3, 38, true, 64, 1, 4),
    QMLA_INST(1, QMLA_RMS_BF16_BYTES, 512, 64, 2, 1, 3, 39, false, 64, 1, 4),
    QMLA_INST(1, QMLA_RMS_E4M3, 512, 64, 2, 1, 3, 38, false, 64, 1, 4),
    // bf16 cache, d_c 512, rope 64, 24 heads (rms 24 bf16): 1200 B staged
    QMLA_INST(2, QMLA_RMS_BF16, 512, 64, 2, 1, 2, 75, false, 64, 1, 4),
    QMLA_INST(2, QMLA_RMS_BF16, 512, 64, 2, 1, 2, 75, true, 64, 1, 4),
    QMLA_INST(2, QMLA_RMS_NONE, 512, 64, 2, 1, 2, 72, false, 64, 1, 4),
    // GLA-g2 (two latent groups of 256, 12 heads each, up to 4 verify tokens: 48 rows per group) on
    // the cache formats the warp-specialized kernel does not take: fp8 rows with e4m3 or bf16-byte
    // rms, bf16 rows with bf16 rms (the reference decodes them as its rank-local TP = 2 shape)
    QMLA_INST(1, QMLA_RMS_E4M3, 256, 64, 3, 2, 3, 38, false, 64, 1, 4),
    QMLA_INST(1, QMLA_RMS_BF16_BYTES, 256, 64, 3, 2, 3, 39, false, 64, 1, 4),
    QMLA_INST(2, QMLA_RMS_BF16, 256, 64, 3, 2, 3, 75, false, 32, 1, 4),
    // the plugin's deployed fp8 layouts (tests/test_fp8_kv.py): partial rope of 4 groups x 58 = 232
    // with 24 heads (one GPU) or 2 x 58 = 116 with 12 heads (rank-local at TP 2), latent ranks 256
    // and 768; rows [latent | rope | rms (1 byte, or 2 for raw bf16) | pad to 16 bytes]
    QMLA_INST(1, QMLA_RMS_LOG8, 256, 256, 2, 1, 3, 32, false, 64, 1, 4),
    QMLA_INST(1, QMLA_RMS_E4M3, 256, 256, 2, 1, 3, 32, false, 64, 1, 4),
    QMLA_INST(1, QMLA_RMS_BF16_BYTES, 256, 256, 2, 1, 3, 34, false, 64, 1, 4),
    QMLA_INST(1, QMLA_RMS_LOG8, 768, 256, 2, 1, 3, 64, false, 32, 1, 4),
    QMLA_INST(1, QMLA_RMS_E4M3, 768, 256, 2, 1, 3, 64, false, 32, 1, 4),
    QMLA_INST(1, QMLA_RMS_BF16_BYTES, 768, 256, 2, 1, 3, 66, false, 32, 1, 4),
    QMLA_INST(1, QMLA_RMS_LOG8, 256, 128, 1, 1, 3, 24, false, 64, 1, 4),
    QMLA_INST(1, QMLA_RMS_E4M3, 256, 128, 1, 1, 3, 24, false, 64, 1, 4),
    QMLA_INST(1, QMLA_RMS_BF16_BYTES, 256, 128, 1, 1, 3, 25, false, 64, 1, 4),
    QMLA_INST(1, QMLA_RMS_LOG8, 768, 128, 1, 1, 2, 56, false, 64, 1, 4),
    QMLA_INST(1, QMLA_RMS_E4M3, 768, 128, 1, 1, 2, 56, false, 64, 1, 4),
    QMLA_INST(1, QMLA_RMS_BF16_BYTES, 768, 128, 1, 1, 2, 57, false, 64, 1, 4),
    // the same layouts on bf16 caches (tests/test_fi_partial_rope.py): one bf16 rms per head
    QMLA_INST(2, QMLA_RMS_BF16, 256, 256, 2, 1, 3, 64, false, 32, 1, 4),
    QMLA_INST(2, QMLA_RMS_BF16, 256, 128, 1, 1, 2, 48, false, 64, 1, 4),
    // full rope 256 (the reference test's tp1full / tp2full layouts, :105): rms tails end at bytes
    // 1072 (24 heads) and 1048 (12 heads), past the 1024 bytes of latent + rope
    QMLA_INST(2, QMLA_RMS_BF16, 256, 256, 2, 1, 3, 67, false, 32, 1, 4),
    QMLA_INST(2, QMLA_RMS_BF16, 256, 256, 1, 1, 2, 66, false, 64, 1, 4),
    QMLA_INST(2, QMLA_RMS_BF16, 768, 128, 2, 1, 2, 112, false, 32, 1, 4),
    // the unpadded 12-head rows of the reference's numerics test at rank 256 (rank + 256 + 12 bf16
    // elements: 1048 bytes, on 8-byte boundaries, tests/test_decode_numerics.py:60-67): narrow rows
    QMLA_INST_DW(2, QMLA_RMS_BF16, 256, 256, 2, 1, 2, 66, false, 32, 1, 4),
};

static int g_cu_count[64];

static int cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (g_cu_count[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    g_cu_count[dev] = n;
  }
  return g_cu_count[dev];
}

static int elem_bytes(int kv_dtype) { return kv_dtype == QMLA_KV_FP8 ? 1 : 2; }

static int rms_elem_bytes(const qmla_decode_params* p) {
  switch (p->rms_mode) {
    case QMLA_RMS_BF16: return 2;
    case QMLA_RMS_BF16_BYTES: return 2;
    case QMLA_RMS_LOG8: return 1;
    case QMLA_RMS_E4M3: return 1;
    default: return 0;
  }
}

static int wp_of(int rope_w) { return (rope_w + 63) / 64 * 64; }

// staged bytes per row: scores read [0, (d_c + WP)*EB) (the padded pair is masked but still read),
// plus the rms tail
static int64_t needed_row_bytes(const qmla_decode_params* p) {
  const int eb = elem_bytes(p->kv_dtype);
  int64_t need = (int64_t)(p->d_c + wp_of(p->rope_w)) * eb;
  if (p->rms_mode != QMLA_RMS_NONE) {
    const int64_t rms_end = (int64_t)p->rms_offset * eb + (int64_t)p->rms_heads * rms_elem_bytes(p);
    if (rms_end > need) need = rms_end;
  }
  return need;
}

static bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

// Checks of a parameter block; `ptrs` = false checks the shapes and modes only (no pointers, no
// address alignment), for questions asked before the tensors exist.
static int validate(const qmla_decode_params* p, bool ptrs = true) {
  if (!p) return QMLA_ERR_NULL;
  if (ptrs && (!p->q_nope || !p->kv_cache || !p->block_table || !p->seq_lens || !p->out)) return QMLA_ERR_NULL;
  if (ptrs && p->rope_w > 0 && !p->q_pe) return QMLA_ERR_NULL;
  if (p->kv_dtype != QMLA_KV_BF16 && p->kv_dtype != QMLA_KV_FP8) return QMLA_ERR_MODE;
  if (p->out_dtype < 0 || p->out_dtype > 2 || (p->lse && (p->lse_dtype < 0 || p->lse_dtype > 2)))
    return QMLA_ERR_MODE;
  if (p->kv_dtype == QMLA_KV_BF16) {
    if (p->rms_mode != QMLA_RMS_NONE && p->rms_mode != QMLA_RMS_BF16) return QMLA_ERR_MODE;
  } else {
    if (p->rms_mode != QMLA_RMS_NONE && p->rms_mode != QMLA_RMS_LOG8 &&
        p->rms_mode != QMLA_RMS_BF16_BYTES && p->rms_mode != QMLA_RMS_E4M3)
      return QMLA_ERR_MODE;
  }
  if ((p->rms_mode == QMLA_RMS_NONE) != (p->rms_offset < 0)) return QMLA_ERR_MODE;
  if (p->rows < 0 || p->heads <= 0 || p->qrows <= 0 || p->groups <= 0 || p->d_c <= 0 || p->rope_w < 0 ||
      p->page_size <= 0)
    return QMLA_ERR_SHAPE;
  if (p->rows % p->qrows) return QMLA_ERR_SHAPE;
  if (p->heads % p->groups || p->d_c % p->groups) return QMLA_ERR_SHAPE;
  if (p->rms_mode != QMLA_RMS_NONE && (p->rms_heads < p->heads / p->groups * p->groups || p->rms_heads <= 0))
    return QMLA_ERR_SHAPE;
  if (p->num_splits < 0 || p->num_splits > CF_MAXS || p->split_align < 0 || p->num_pages < 0) return QMLA_ERR_SHAPE;
  const int eb = elem_bytes(p->kv_dtype);
  // 4-byte boundaries here; rows off 16-byte boundaries are served by the narrow-row instances only
  if ((ptrs && (uintptr_t)p->kv_cache % 4) || (p->page_stride * eb) % 4 || (p->token_stride * eb) % 4)
    return QMLA_ERR_ALIGN;
  if (needed_row_bytes(p) > p->token_stride * eb && p->page_size > 1) return QMLA_ERR_SHAPE;
  // queries: element alignment (16-byte aligned rows take the vector loads)
  if (ptrs && ((uintptr_t)p->q_nope % 2 || (p->rope_w > 0 && (uintptr_t)p->q_pe % 2))) return QMLA_ERR_ALIGN;
  return QMLA_OK;
}

// No compiled kernel for these params: rows off 16-byte boundaries that no narrow-row instance
// serves report the alignment, everything else the missing kernel.
static int no_kernel(const qmla_decode_params* p) { return rows16(p) ? QMLA_ERR_NOKERNEL : QMLA_ERR_ALIGN; }

// Workgroups per token range of a per-group instance: a request's rows per group (verify tokens x
// heads) in blocks of 16*MB, at most kMaxRowSplit of them (each reads the range's cached rows; the
// balanced mode places them on one XCD, whose L2 then serves all but the first read).
constexpr int kMaxRowSplit = 4;
static int row_splits(const Inst& in, const qmla_decode_params* p) {
  const int rows_pg = p->qrows * (p->heads / p->groups);
  return (rows_pg + 16 * in.mb - 1) / (16 * in.mb);
}

// The instance with the fewest workgroups per token range, then the fewest row blocks (no idle
// rows), then the fewest staged bytes.
static const Inst* find_inst(const qmla_decode_params* p) {
  const int eb = elem_bytes(p->kv_dtype);
  const int dcg = p->d_c / p->groups;
  const int64_t need = needed_row_bytes(p);
  const bool cap = p->logit_cap > 0.f;
  const Inst* best = nullptr;
  int best_hs = 0;
  for (const Inst& in : kInst) {
    if (in.eb != eb || in.rms != p->rms_mode || in.dcg != dcg || in.g != p->groups || in.cap != cap) continue;
    if (in.wp != wp_of(p->rope_w)) continue;
    if (in.dw == rows16(p)) continue;   // narrow-row instances serve exactly the rows off 16-byte boundaries
    const int hs = row_splits(in, p);
    if (hs > kMaxRowSplit) continue;
    if ((int64_t)in.cpr * 16 < need) continue;
    if (!in.dw && (int64_t)in.cpr * 16 > p->token_stride * eb) continue;   // never read past the row
    if (in.dw && need > p->token_stride * eb) continue;   // narrow rows load the row stride's bytes only
    if (!best || hs < best_hs || (hs == best_hs && (in.mb < best->mb || (in.mb == best->mb && in.cpr < best->cpr)))) {
      best = &in;
      best_hs = hs;
    }
  }
  return best;
}

// Token ranges of the balanced mode (workgroups, except that the warp-specialized kernel's head split
// runs hsplit workgroups per range): one workgroup per compute unit; with a head split a multiple of
// 8 ranges, so each range's workgroups share an XCD.
static int balanced_nwg(const qmla_decode_params* p) {
  if (p->num_workgroups > 0) return p->num_workgroups;
  // workgroups sharing each token range: the warp-specialized kernel's head split, the column-split
  // and per-group kernels' row splits
  int hs = 1, wgpc = 1;
  if (ws_select(p) >= 0) {
    hs = ws_head_split(p);
  } else if (cs_select(p) >= 0) {
    hs = cs_row_splits(p);
  } else if (const Inst* in = find_inst(p)) {
    hs = row_splits(*in, p);
    wgpc = in->wgpc;
  }
  if (hs > 1) {   // every workgroup resident at once, a range's workgroups on one XCD
    const int r = cu_count() * wgpc / (8 * hs) * 8;
    return r > 8 ? r : 8;
  }
  return cu_count() * wgpc;
}

struct BalancedLayout {
  size_t plan_off, lse_off, o_off, total;
};

static BalancedLayout balanced_layout(const qmla_decode_params* p) {
  const int64_t n_req = p->rows / p->qrows;
  const int64_t nwg = balanced_nwg(p);
  const int64_t nrow = (int64_t)p->qrows * p->heads;
  const int64_t dv = p->d_c / p->groups;
  const int64_t slots = nwg + n_req;
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  BalancedLayout b;
  b.plan_off = 0;
  b.lse_off = up((size_t)(3 + n_req) * 4);
  b.o_off = b.lse_off + up((size_t)(slots * nrow) * 4);
  b.total = b.o_off + up((size_t)(slots * nrow * dv) * 4);
  return b;
}

// Plan tiles (of PLAN_TILE tokens) the balanced plan charges per request switch, per kernel family:
// what a workgroup spends on a piece besides its tokens (the query load and conversion at its first
// tile, the output write at its last), measured as the time of that many tiles. Fixed splits: 0.
static int plan_switch(const qmla_decode_params* p) {
  if (p->num_splits != 0) return 0;
  if (ro_select(p) >= 0) return kPlanSwitchRo;
  if (ws_select(p) >= 0) return kPlanSwitchWs;
  return kPlanSwitchOther;
}

static KParams make_kparams(const qmla_decode_params* p) {
  KParams k;
  const int eb = elem_bytes(p->kv_dtype);
  k.q_vec = aligned16(p->q_nope) && (p->q_nope_stride_row * 2) % 16 == 0 && (p->q_nope_stride_head * 2) % 16 == 0 &&
            (p->rope_w == 0 || (aligned16(p->q_pe) && (p->q_pe_stride_row * 2) % 16 == 0 &&
                                (p->q_pe_stride_head * 2) % 16 == 0));
  k.q_nope = reinterpret_cast<const __bf16*>(p->q_nope);
  k.qn_sr = p->q_nope_stride_row;
  k.qn_sh = p->q_nope_stride_head;
  k.q_pe = reinterpret_cast<const __bf16*>(p->q_pe ? p->q_pe : p->q_nope);
  k.qp_sr = p->q_pe_stride_row;
  k.qp_sh = p->q_pe_stride_head;
  k.kv = reinterpret_cast<const char*>(p->kv_cache);
  k.page_stride_b = p->page_stride * eb;
  k.token_stride_b = p->token_stride * eb;
  k.page_size = p->page_size;
  k.rope_w = p->rope_w;
  k.rms_off_b = p->rms_offset >= 0 ? p->rms_offset * eb : 0;
  k.k_scale = p->k_scale;
  k.sm_scale = p->sm_scale;
  k.logit_cap = p->logit_cap;
  k.bt = p->block_table;
  k.bt_stride = p->bt_stride;
  k.seq_lens = p->seq_lens;
  k.n_req = p->rows / p->qrows;
  k.qrows = p->qrows;
  k.hpg = p->heads / p->groups;
  k.heads = p->heads;
  k.out = p->out;
  k.o_sr = p->out_stride_row;
  k.o_sh = p->out_stride_head;
  k.out_dt = p->out_dtype;
  k.lse = p->lse;
  k.lse_sr = p->lse_stride_row;
  k.lse_dt = p->lse_dtype;
  k.num_splits = p->num_splits;
  k.split_align = p->split_align;
  k.ws = p->workspace;
  k.ws_sr = p->ws_stride_row;
  k.ws_sh = p->ws_stride_head;
  k.ws_ss = p->ws_stride_split;
  // without a page count only negative entries are caught
  k.page_bound = p->num_pages > 0 ? (uint32_t)p->num_pages : 0x80000000u;
  k.status = p->status;
  k.nwg = 0;
  k.plan_sw = plan_switch(p);
  k.part_h = p->kv_dtype == QMLA_KV_FP8 ? 1 : 0;
  k.plan = nullptr;
  k.part_o = nullptr;
  k.part_lse = nullptr;
  if (p->num_splits == 0 && p->workspace) {
    const BalancedLayout bl = balanced_layout(p);
    char* base = reinterpret_cast<char*>(p->workspace);
    k.nwg = balanced_nwg(p);
    k.plan = reinterpret_cast<int*>(base + bl.plan_off);
    k.part_lse = reinterpret_cast<float*>(base + bl.lse_off);
    k.part_o = reinterpret_cast<float*>(base + bl.o_off);
  }
  return k;
}

static int launch(const void* fn, dim3 grid, dim3 block, void** args, hipStream_t st) {
  if (grid.x == 0 || grid.y == 0 || grid.z == 0) return QMLA_OK;
  hipError_t e = hipLaunchKernel(fn, grid, block, args, 0, st);
  return e == hipSuccess ? QMLA_OK : QMLA_ERR_LAUNCH;
}

static int run_partial(const qmla_decode_params* p, const Inst* in, KParams& k, hipStream_t st) {
  void* args[] = {&k};
  // a range's row splits are consecutive in z: workgroup (x, 0, z) is dispatched as x + z * nwg, so
  // with nwg a multiple of 8 the splits of range x share XCD x % 8
  const int hs = row_splits(*in, p);
  if (p->num_splits > 0)
    return launch((const void*)in->fn, dim3(p->num_splits, k.n_req, hs), dim3(in->nthr, 1, 1), args, st);
  return launch((const void*)in->fn, dim3(k.nwg, 1, hs), dim3(in->nthr, 1, 1), args, st);
}

// One split: the decode kernels write final rows for the token ranges they own, and a request of
// length 0 owns none. Its rows get what every combine writes for them: zero output, -inf lse.
// Block (head, row); requests with tokens return at once.
__global__ __launch_bounds__(64) void empty_rows_kernel(const KParams p, int dv) {
  const int head = blockIdx.x, row = blockIdx.y;
  if (req_len(p, row / p.qrows) > 0) return;
  const int64_t obase = (int64_t)row * p.o_sr + (int64_t)head * p.o_sh;
  for (int c = threadIdx.x; c < dv; c += 64) store_out(p.out, p.out_dt, obase + c, 0.f);
  if (threadIdx.x == 0 && p.lse) store_out(p.lse, p.lse_dt, (int64_t)row * p.lse_sr + head, kNegInf);
}

static int run_empty_rows(const qmla_decode_params* p, KParams& k, hipStream_t st) {
  int dv = p->d_c / p->groups;
  void* args[] = {&k, &dv};
  return launch((const void*)&empty_rows_kernel, dim3(p->heads, p->rows, 1), dim3(64, 1, 1), args, st);
}

static int run_combine(const qmla_decode_params* p, KParams& k, hipStream_t st) {
  int dv = p->d_c / p->groups;
  void* args[] = {&k, &dv};
  if (p->num_splits == 0 && (dv & 1)) return QMLA_ERR_SHAPE;   // the balanced combine reads column pairs
  if (p->num_splits == 0)
    return dv > 1024 ? launch((const void*)&combine_bal_kernel<1>, dim3(p->heads, p->rows, 1), dim3(256, 1, 1), args, st)
                     : launch((const void*)&combine_bal_kernel<CH_HB>, dim3((p->heads + CH_HB - 1) / CH_HB, p->rows, 1),
                              dim3(256, 1, 1), args, st);
  return launch((const void*)&combine_kernel, dim3(p->heads, p->rows, 1), dim3(256, 1, 1), args, st);
}

static int run_plan(const qmla_decode_params* p, KParams& k, hipStream_t st) {
  const int* sl = p->seq_lens;
  int n_req = k.n_req, qrows = k.qrows, nwg = k.nwg, sw = k.plan_sw;
  int* plan = k.plan;
  void* args[] = {&sl, &n_req, &qrows, &nwg, &sw, &plan};
  return launch((const void*)&plan_kernel, dim3(1, 1, 1), dim3(1024, 1, 1), args, st);
}

}  // namespace qmla

using namespace qmla;

extern "C" {

int qmla_version(void) { return QMLA_ABI_VERSION; }

const char* qmla_build_info(void) {
  return "qmla gfx950: warp-specialized FP8 decode (fp8 MFMA scores, query as e4m3 hi+lo), wide-row "
         "warp-specialized decode (bf16 rows, the deployed fp8 rank-768/256 rows), row-owner GLA-g2 decode, "
         "segment decode (bf16 MFMA QK/PV) for the other layouts, column-split single-pass wide latent "
         "(d_c 1792); LDS-DMA paged rows, tr8/tr16 value reads, fixed and balanced split-K + LSE combine; "
         "cache-row writer";
}

size_t qmla_workspace_bytes(const qmla_decode_params* p) {
  if (!p || p->rows <= 0 || p->qrows <= 0 || p->groups <= 0) return 0;
  const int64_t dv = p->d_c / p->groups;
  if (p->num_splits > 0) {
    if (p->num_splits == 1) return 0;
    return (size_t)p->rows * p->heads * p->num_splits * (dv + 1) * 4;
  }
  return balanced_layout(p).total;
}

static int check_balanced_ws(const qmla_decode_params* p) {
  if (!p->workspace) return QMLA_ERR_WORKSPACE;
  if (p->workspace_bytes < qmla_workspace_bytes(p)) return QMLA_ERR_WORKSPACE;
  if (!aligned16(p->workspace)) return QMLA_ERR_ALIGN;
  return QMLA_OK;
}

// Fixed splits: attn_logits [rows, heads, S, dv + 1] fp32 at the caller's strides. The buffer must
// hold the dense layout's bytes and the largest partial offset, (rows-1)*sr + (heads-1)*sh +
// (S-1)*ss + dv, with positive strides; one split needs no workspace.
static int check_fixed_ws(const qmla_decode_params* p) {
  if (p->num_splits <= 1) return QMLA_OK;
  if (!p->workspace) return QMLA_ERR_WORKSPACE;
  if (p->workspace_bytes < qmla_workspace_bytes(p)) return QMLA_ERR_WORKSPACE;
  if (p->ws_stride_row <= 0 || p->ws_stride_head <= 0 || p->ws_stride_split <= 0) return QMLA_ERR_WORKSPACE;
  if ((uintptr_t)p->workspace % 4) return QMLA_ERR_ALIGN;
  const int64_t dv = p->d_c / p->groups;
  const int64_t last = (int64_t)(p->rows - 1) * p->ws_stride_row + (int64_t)(p->heads - 1) * p->ws_stride_head +
                       (int64_t)(p->num_splits - 1) * p->ws_stride_split + dv;
  if (p->rows > 0 && (last + 1) * 4 > (int64_t)p->workspace_bytes) return QMLA_ERR_WORKSPACE;
  return QMLA_OK;
}

int qmla_decode_supported(const qmla_decode_params* p) {
  const int rc = validate(p, false);
  if (rc) return rc;
  if (p->d_c / p->groups > 2048) return QMLA_ERR_SHAPE;
  return (ws_select(p) >= 0 || cs_select(p) >= 0 || find_inst(p)) ? QMLA_OK : no_kernel(p);
}

int qmla_plan_switch_tiles(const qmla_decode_params* p) {
  const int rc = validate(p);
  return rc ? rc : qmla::plan_switch(p);
}

int qmla_plan(const qmla_decode_params* p, void* stream) {
  int rc = validate(p);
  if (rc) return rc;
  if (p->num_splits != 0) return QMLA_ERR_MODE;
  rc = check_balanced_ws(p);
  if (rc) return rc;
  KParams k = make_kparams(p);
  return run_plan(p, k, (hipStream_t)stream);
}

int qmla_decode_partial(const qmla_decode_params* p, void* stream) {
  int rc = validate(p);
  if (rc) return rc;
  if (p->d_c / p->groups > 2048) return QMLA_ERR_SHAPE;
  const int si = ws_select(p);
  const int wi = si >= 0 ? -1 : cs_select(p);
  const Inst* in = (si >= 0 || wi >= 0) ? nullptr : find_inst(p);
  if (!in && wi < 0 && si < 0) return no_kernel(p);
  rc = p->num_splits == 0 ? check_balanced_ws(p) : check_fixed_ws(p);
  if (rc) return rc;
  KParams k = make_kparams(p);
  hipStream_t st = (hipStream_t)stream;
  rc = si >= 0 ? ws_launch(si, p, k, k.nwg, st) : in ? run_partial(p, in, k, st) : cs_launch(wi, p, k, k.nwg, st);
  // one split writes the final rows here (the combine has nothing to do)
  if (rc || p->num_splits != 1) return rc;
  return run_empty_rows(p, k, st);
}

int qmla_combine(const qmla_decode_params* p, void* stream) {
  int rc = validate(p);
  if (rc) return rc;
  // the same refusal as the decode pass for rows no kernel can stage
  if (!rows16(p) && ws_select(p) < 0 && cs_select(p) < 0 && !find_inst(p)) return QMLA_ERR_ALIGN;
  if (p->num_splits == 1) return QMLA_OK;
  if (p->d_c / p->groups > 2048) return QMLA_ERR_SHAPE;
  rc = p->num_splits == 0 ? check_balanced_ws(p) : check_fixed_ws(p);
  if (rc) return rc;
  KParams k = make_kparams(p);
  return run_combine(p, k, (hipStream_t)stream);
}

// ---- the decode without a caller workspace ------------------------------------------------------
// Library-owned scratch for qmla_decode_static: one array per GPU (each device the library runs on
// holds its own copy until the process ends). Host code never uses the array's name as an address:
// its device address is fetched once per device with hipGetSymbolAddress and kept below.
static __device__ __align__(256) char scratch[QMLA_STATIC_SCRATCH_BYTES];
static void* g_scratch_ptr[64];
static std::mutex g_scratch_mu;

// Device address of this device's scratch (the current device), or nullptr on failure.
static void* scratch_ptr() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

int qmla_decode_static(const qmla_decode_params* p, void* stream) {
  int rc = validate(p);
  if (rc) return rc;
  qmla_decode_params q = *p;
  const int64_t dv = p->d_c / p->groups;
  if (q.num_splits > 1) {
    // the reference-layout partials, dense [rows, heads, S, dv + 1], in the scratch
    q.ws_stride_split = dv + 1;
    q.ws_stride_head = (int64_t)q.num_splits * (dv + 1);
    q.ws_stride_row = (int64_t)q.heads * q.ws_stride_head;
  }
  const size_t need = qmla_workspace_bytes(&q);
  if (need > (size_t)QMLA_STATIC_SCRATCH_BYTES) return QMLA_ERR_WORKSPACE;
  if (need > 0) {
    void* ptr = scratch_ptr();
    if (!ptr) return QMLA_ERR_LAUNCH;
    q.workspace = reinterpret_cast<float*>(ptr);
    q.workspace_bytes = (size_t)QMLA_STATIC_SCRATCH_BYTES;
  } else {
    q.workspace = nullptr;
    q.workspace_bytes = 0;
  }
  return qmla_decode(&q, stream);
}

int qmla_decode(const qmla_decode_params* p, void* stream) {
  int rc = validate(p);
  if (rc) return rc;
  if (p->d_c / p->groups > 2048) return QMLA_ERR_SHAPE;
  const int si = ws_select(p);
  const int wi = si >= 0 ? -1 : cs_select(p);
  const Inst* in = (si >= 0 || wi >= 0) ? nullptr : find_inst(p);
  if (!in && wi < 0 && si < 0) return no_kernel(p);
  hipStream_t st = (hipStream_t)stream;
  if (p->num_splits > 0) {
    rc = check_fixed_ws(p);
    if (rc) return rc;
    KParams k = make_kparams(p);
    rc = si >= 0 ? ws_launch(si, p, k, 0, st) : in ? run_partial(p, in, k, st) : cs_launch(wi, p, k, 0, st);
    if (rc) return rc;
    return p->num_splits == 1 ? run_empty_rows(p, k, st) : run_combine(p, k, st);
  }
  rc = check_balanced_ws(p);
  if (rc) return rc;
  KParams k = make_kparams(p);
  // the decode kernels derive the balanced plan themselves (and store it for the combine)
  rc = si >= 0 ? ws_launch(si, p, k, k.nwg, st) : in ? run_partial(p, in, k, st) : cs_launch(wi, p, k, k.nwg, st);
  if (rc) return rc;
  return run_combine(p, k, st);
}

}  // extern "C"
