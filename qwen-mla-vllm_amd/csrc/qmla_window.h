// Shared by the warp-specialized (qmla_ws.hip) and row-owner (qmla_ro.hip) decode kernels: the walk
// of a workgroup's token range as one sequence of 32-token tiles over pieces (one per request),
// planned in windows of up to NSEG pieces and PIDN page ids; counted LDS reads; the rotated row
// layout of staged tiles.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "qmla.h"
#include "qmla_common.h"
#include "qmla_device.h"

namespace qmla {
namespace ws {

constexpr int TILE = 32;          // tokens per tile
constexpr int NSEG = 64;          // pieces per window (one per lane of the wave that plans it)
constexpr int PIDN = 1024;        // page ids per window
enum { SEG_FIRST = 1, SEG_LAST = 2, SEG_FINAL = 4 };

__device__ __forceinline__ i32x4 ldsr128(const void* p) {
  i32x4 r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(lds_addr(static_cast<const char*>(p))));
  return r;
}
__device__ __forceinline__ i32x2 ldsr64(const void* p) {
  i32x2 r;
  asm volatile("ds_read_b64 %0, %1" : "=v"(r) : "v"(lds_addr(static_cast<const char*>(p))));
  return r;
}
__device__ __forceinline__ int ldsr32(const void* p) {
  int r;
  asm volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(lds_addr(static_cast<const char*>(p))));
  return r;
}
__device__ __forceinline__ float ldsr32f(const void* p) {
  float r;
  asm volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(lds_addr(static_cast<const char*>(p))));
  return r;
}
__device__ __forceinline__ uint32_t ldsr8(const void* p) {
  uint32_t r;
  asm volatile("ds_read_u8 %0, %1" : "=v"(r) : "v"(lds_addr(static_cast<const char*>(p))));
  return r;
}
// Reads that may follow a scalar load the compiler placed (kernel arguments it reloads under
// register pressure): one statement that drains the counter first and waits for its own reads, so
// no counted wait is involved and nothing can be scheduled in between. The destinations are
// early-clobber: a read's result may land while a later read of the statement still waits to issue,
// so no destination may share a register with an address.
__device__ __forceinline__ void ldsr32f3_drained(const void* a, const void* b, const void* c, float& x, float& y,
                                                 float& z) {
  asm volatile(
      "s_waitcnt lgkmcnt(0)\n\tds_read_b32 %0, %3\n\tds_read_b32 %1, %4\n\tds_read_b32 %2, %5\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(x), "=&v"(y), "=&v"(z)
      : "v"(lds_addr(static_cast<const char*>(a))), "v"(lds_addr(static_cast<const char*>(b))),
        "v"(lds_addr(static_cast<const char*>(c))));
}
__device__ __forceinline__ void ldsr128x2_drained(const void* a, const void* b, i32x4& x, i32x4& y) {
  asm volatile("s_waitcnt lgkmcnt(0)\n\tds_read_b128 %0, %2\n\tds_read_b128 %1, %3\n\ts_waitcnt lgkmcnt(0)"
               : "=&v"(x), "=&v"(y)
               : "v"(lds_addr(static_cast<const char*>(a))), "v"(lds_addr(static_cast<const char*>(b))));
}
__device__ __forceinline__ uint32_t ldsr16(const void* p) {
  uint32_t r;
  asm volatile("ds_read_u16 %0, %1" : "=v"(r) : "v"(lds_addr(static_cast<const char*>(p))));
  return r;
}

// Wait until at most N of this wave's LDS operations are outstanding; LDS operations complete in
// issue order, so with N = the number issued after the one producing v, v is ready (more younger
// operations than counted only make the wait longer). The register tie orders v's uses after it.
// No scalar memory load is ever outstanding inside the tile loop, so the count is LDS-only.
template <int N, class T>
__device__ __forceinline__ void lds_wait_n(T& v) {
  static_assert(N >= 0 && N <= 15, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(v) : "n"(N));
}
constexpr int cmin15(int n) { return n < 15 ? n : 15; }

template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

__device__ __forceinline__ int lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
}

// one piece of the workgroup's range: tokens [ta, te) of request req (length L); nt tiles; its pages
// start at window page index pf
struct SegD {
  int req, ta, te, L;
  int nt, pf, fl, pad;
};

// Staged row layout of fp8 MLA rows (4 latent blocks of 8 16-byte chunks, the rope's 4 chunks, then
// the rms codes' CPR - 36): each chunk stays in its region, rotated there by the row's flip f(r).
// A ds_read_b128 is served 32 lanes at a time over 128 banks (measured: 16 rows of 608 bytes x two
// chunks two apart run at 32 cycles per read and wave with four waves, contiguous lanes at 25). So
// 608-byte rows (CPR 38, 152 dwords: rows 24 banks apart mod 128) flip by (r & 1) ^ ((r >> 4) & 1):
// the K reads of 16 consecutive rows by two lane groups (chunks 2lg + h) and the transposed V reads
// of rows 8lg .. 8lg+7 (32 or 64 lanes a pass) then fill the banks once; 592-byte rows (CPR 37)
// take no flip. Reads of one latent block then share a base register per lane and pattern, the
// block and chunk going into the instructions' offset fields.
template <int CPR>
__device__ __forceinline__ int lflip(int r) {
  return CPR == 38 ? (r & 1) ^ ((r >> 4) & 1) : 0;
}
template <int CPR>
__device__ __forceinline__ int region_base(int c) {
  return c < 32 ? (c & ~7) : c < 36 ? 32 : 36;
}
template <int CPR>
__device__ __forceinline__ int region_mask(int c) {
  return c < 32 ? 7 : c < 36 ? 3 : (CPR - 36 >= 2 ? 1 : 0);
}
// position of chunk c in a row with flip f, and the inverse
template <int CPR>
__device__ __forceinline__ int chunk_pos(int c, int f) {
  const int b = region_base<CPR>(c);
  return b + ((c - b + f) & region_mask<CPR>(c));
}
template <int CPR>
__device__ __forceinline__ int pos_chunk(int q, int f) {
  const int b = region_base<CPR>(q);
  return b + ((q - b - f) & region_mask<CPR>(q));
}
// byte b of staged row r
template <int CPR>
__device__ __forceinline__ int lbyte(int r, int b) {
  return r * (16 * CPR) + 16 * chunk_pos<CPR>(b >> 4, lflip<CPR>(r)) + (b & 15);
}

// LDS reads at a base address plus an immediate offset (the loop keeps one base register per lane
// and read pattern, not one address per read)
template <int OFF>
__device__ __forceinline__ i32x4 ldsr128_at(uint32_t a) {
  i32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(a), "n"(OFF));
  return r;
}
template <int OFF>
__device__ __forceinline__ i32x2 ldstr8_at(uint32_t a) {
  i32x2 r;
  asm volatile("ds_read_b64_tr_b8 %0, %1 offset:%2" : "=v"(r) : "v"(a), "n"(OFF));
  return r;
}
template <int OFF>
__device__ __forceinline__ i32x2 ldstr16_at(uint32_t a) {
  i32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(a), "n"(OFF));
  return r;
}
template <int OFF>
__device__ __forceinline__ uint32_t ldsr16_at(uint32_t a) {
  uint32_t r;
  asm volatile("ds_read_u16 %0, %1 offset:%2" : "=v"(r) : "v"(a), "n"(OFF));
  return r;
}
template <int OFF>
__device__ __forceinline__ uint32_t ldsr8_off(uint32_t a) {
  uint32_t r;
  asm volatile("ds_read_u8 %0, %1 offset:%2" : "=v"(r) : "v"(a), "n"(OFF));
  return r;
}
__device__ __forceinline__ uint32_t ldsr8_at(uint32_t a) {
  uint32_t r;
  asm volatile("ds_read_u8 %0, %1" : "=v"(r) : "v"(a));
  return r;
}


// vmcnt <= ahead * D (ahead tiles of D loads each issued after the awaited one), ahead <= K
template <int D, int K>
__device__ __forceinline__ void wait_tiles(int ahead) {
  if constexpr (K <= 0 || D == 0) {
    wait_vmcnt<0>();
  } else {
    if (ahead >= K) wait_vmcnt<K * D>();
    else wait_tiles<D, K - 1>(ahead);
  }
}

// Wave 0: the next window of pieces, from request cb at token ctok on, into sm.seg / sm.win.
// Lane l looks at request cb + l; pieces are taken in request order while their pages fit PN (the
// first piece that does not fit is cut at a page boundary). Balanced mode: cp is the plan prefix
// C_cb of the cursor's request, and the lanes' C_b follow from a scan of their tile counts.
template <int SW, int PN = PIDN, class SM>
__device__ void plan_window(const KParams& p, SM& sm, bool fixed, int lo, int hi, int& cb, int& ctok,
                            int& cp) {
  const int lane = threadIdx.x & 63;
  const int P = p.page_size;
  int nseg = 0, ntot = 0, npg = 0;
  bool more = true;
  while (more && nseg == 0) {
    const int b = cb + lane;
    int a = 0, e = 0, L = 0, fl = 0;
    // plan tiles [c0, c1) of request b (balanced mode)
    const int tb = (!fixed && b < p.n_req) ? plan_tiles<SW>(p, b) : 0;
    const int tincl = wave_incl_sum(tb);
    const int c0 = cp + tincl - tb, c1 = cp + tincl;
    bool beyond;
    if (fixed) {
      beyond = lane != 0;
      if (!beyond) {
        L = req_len(p, b);
        const int per = split_len(p, L);
        const int a0 = per * (int)blockIdx.x;
        e = a0 + per < L ? a0 + per : L;
        a = a0 > ctok ? a0 : ctok;
        fl = (a == a0 ? SEG_FIRST : 0) | SEG_LAST | (p.num_splits == 1 ? SEG_FINAL : 0);
      }
    } else {
      beyond = b >= p.n_req;
      if (!beyond) {
        beyond = c0 >= hi;
        if (!beyond && c1 > lo) {
          L = req_len(p, b);
          const PieceTok pt = piece_tokens<SW>(L, c0, c1, lo, hi);
          const int a0 = pt.a;
          e = pt.e;
          a = lane == 0 && ctok > a0 ? ctok : a0;
          fl = (a == a0 ? SEG_FIRST : 0) | SEG_LAST | (pt.whole ? SEG_FINAL : 0);
        }
      }
    }
    const bool live = !beyond && a < e;
    const int pages = live ? (e - 1) / P - a / P + 1 : 0;
    const int cum = wave_incl_sum(pages);
    const int excl = cum - pages;
    const bool take = live && excl < PN;
    int et = e;
    if (take && cum > PN) {
      const int cut = (a / P + (PN - excl)) * P;   // page-aligned, > a
      et = cut < e ? cut : e;
    }
    if (et < e) fl &= ~SEG_LAST;
    const int nt = take ? (et - a + TILE - 1) / TILE : 0;
    const int npt = take ? (et - 1) / P - a / P + 1 : 0;
    const uint64_t tm = __builtin_amdgcn_ballot_w64(take);
    const int tcum = wave_incl_sum(nt);
    const int pcum = wave_incl_sum(npt);
    if (take) {
      SegD d;
      d.req = b;
      d.ta = a;
      d.te = et;
      d.L = L;
      d.nt = nt;
      d.pf = pcum - npt;
      d.fl = fl;
      d.pad = 0;
      sm.seg[lanes_below(tm)] = d;
    }
    nseg = __builtin_popcountll(tm);
    ntot = __shfl(tcum, 63, 64);
    npg = __shfl(pcum, 63, 64);
    // cursor: the first live request not finished here; else the range is done if a request at or
    // past its end was seen; else the next 64 requests
    const uint64_t um = __builtin_amdgcn_ballot_w64(live && (!take || et < e));
    const uint64_t bm = __builtin_amdgcn_ballot_w64(beyond);
    if (um) {
      const int x = __builtin_ctzll(um);
      const int etx = __shfl(et, x, 64);
      const bool tookx = (tm >> x) & 1;
      cb += x;
      cp = __shfl(c0, x, 64);
      ctok = tookx ? etx : 0;
    } else if (bm) {
      more = false;
    } else {
      cb += 64;
      cp = __shfl(c1, 63, 64);
      ctok = 0;
    }
  }
  if (lane == 0) {
    sm.win[0] = nseg;
    sm.win[1] = ntot;
    sm.win[2] = npg;
    sm.win[3] = more ? 1 : 0;
  }
}

}  // namespace ws
}  // namespace qmla
