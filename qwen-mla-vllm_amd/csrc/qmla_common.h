// Shared by the decode translation units of libqmla.so: the kernel parameter block, the output
// descriptor of one token range, and the split of a launch into token ranges (fixed splits or the
// balanced plan).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qmla.h"
#include "qmla_device.h"

namespace qmla {

constexpr int PLAN_TILE = 64;  // balancing granularity of the balanced plan (tokens)
// plan tiles the balanced plan charges per request switch (see plan_tiles), per kernel family: the
// warp-specialized and row-owner decode (measured: a piece's query load and output write cost about
// two plan tiles of work), the per-group and column-split kernels (none)
constexpr int kPlanSwitchWs = 2, kPlanSwitchRo = 2, kPlanSwitchOther = 0;

struct KParams {
  const __bf16* q_nope;
  int64_t qn_sr, qn_sh;
  const __bf16* q_pe;
  int64_t qp_sr, qp_sh;
  const char* kv;
  int64_t page_stride_b, token_stride_b;  // bytes
  int page_size;
  int rope_w;
  int rms_off_b;  // byte offset of the rms tail inside a row
  const float* k_scale;
  float sm_scale, logit_cap;
  const int* bt;
  int64_t bt_stride;
  const int* seq_lens;
  int n_req;      // requests = rows / qrows
  int qrows, hpg; // verify tokens per request, heads per latent group
  int heads;      // heads per row (= groups * hpg)
  void* out;
  int64_t o_sr, o_sh;
  int out_dt;
  void* lse;
  int64_t lse_sr;
  int lse_dt;
  int num_splits, split_align;
  float* ws;
  int64_t ws_sr, ws_sh, ws_ss;
  // balanced mode
  int nwg;
  int* plan;        // [0] = chunk (tiles per workgroup), [1] = total tiles, [2 + b] = prefix C_b
  float* part_o;    // [(nwg + n_req), qrows*heads, Dv]
  float* part_lse;  // [(nwg + n_req), qrows*heads]
  int q_vec;        // query rows and strides 16-byte aligned: 16-byte query loads (else element loads)
  int hsplit;       // warp-specialized kernel: workgroups sharing a request's token range, each with
                    // heads/hsplit of its heads (balanced mode: nwg ranges x hsplit workgroups)
  uint32_t page_bound;  // block-table entries must lie in [0, page_bound)
  int* status;          // QMLA_ERR_PAGE is stored here when one does not (may be null)
  int plan_sw;          // plan tiles charged for a request switch (see plan_tiles): read by the
                        // combine and the plan kernel; the decode kernels have their family's as a
                        // constant
  int part_h;           // balanced partial outputs in fp16 and without the fp8 scale (fp8 caches:
                        // |value| <= 448), which the combine applies; else fp32
};

// A block-table entry checked against the page bound: an entry outside [0, page_bound) reads page 0
// (in bounds) and raises `bad`, which the kernel reports once its memory traffic has drained.
__device__ __forceinline__ int checked_page(const KParams& p, int id, int& bad) {
  const bool ok = (uint32_t)id < p.page_bound;
  bad |= ok ? 0 : 1;
  return ok ? id : 0;
}
__device__ __forceinline__ void report_pages(const KParams& p, int bad) {
  if (bad && p.status) *p.status = QMLA_ERR_PAGE;
}

// 8 consecutive query elements: one 16-byte load when the caller's query rows are 16-byte aligned,
// else eight element loads (queries are read once per request or segment, so this costs nothing
// that shows). `vec` is the same for every lane.
__device__ __forceinline__ bf16x8 load_q8(const __bf16* ptr, bool vec) {
  if (vec) return *reinterpret_cast<const bf16x8*>(ptr);
  bf16x8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = ptr[e];
  return v;
}

__device__ __forceinline__ void store_out(void* base, int dt, int64_t idx, float v) {
  if (dt == QMLA_DT_BF16) reinterpret_cast<__bf16*>(base)[idx] = (__bf16)v;
  else if (dt == QMLA_DT_F16) reinterpret_cast<_Float16*>(base)[idx] = (_Float16)v;
  else reinterpret_cast<float*>(base)[idx] = v;
}

// Where the result of one token range goes.
struct SegOut {
  bool final_out;       // write normalized output + lse directly
  float* po;            // partial output base of this request (query-row 0 of it)
  int64_t po_sr, po_sh; // float strides for (verify token of the request, head)
  float* plse;          // balanced-mode lse base (nullptr: lse stored after the Dv columns)
  int64_t plse_sr;
};

// request length: the last flattened row of the request carries it (mla_impl.py:628-662)
__device__ __forceinline__ int req_len(const KParams& p, int req) {
  int L = p.seq_lens[(int64_t)req * p.qrows + p.qrows - 1];
  return L > 0 ? L : 0;
}

// ---- the balanced plan, computed by the decode kernels themselves ---------------------------------
// Request b owns plan tiles [C_b, C_b + T_b) of the concatenated requests, with T_b = ceil(L_b /
// PLAN_TILE) + plan_sw for a non-empty request (0 for an empty one) and C_b the exclusive prefix of
// the T's; workgroup w of nwg owns plan tiles [w*chunk, min((w+1)*chunk, total)) with chunk =
// ceil(total / nwg). A request's first plan_sw tiles hold no tokens: they charge the fixed work of
// a piece (the query load, the output write) to the workgroup that starts the request, so a
// workgroup holding two pieces gets fewer tokens than one holding one; the following tiles hold
// PLAN_TILE tokens each. Every workgroup derives
// its own range from seq_lens at its start (no planning launch: a launch of its own costs more
// than the scan, and inside a HIP graph far more), and workgroup 0 also stores the plan for the
// balanced combine.

__device__ __forceinline__ int wave_incl_sum(int x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  return x;
}

template <int SW>
__device__ __forceinline__ int plan_tiles(const KParams& p, int b) {
  const int L = req_len(p, b);
  return L > 0 ? (L + PLAN_TILE - 1) / PLAN_TILE + SW : 0;
}

// The tokens [a, e) of a request of length L with plan tiles [c0, c1) that plan tiles [lo, hi) hold
// (e <= a: none), and whether they are all of its tokens.
struct PieceTok {
  int a, e;
  bool whole;
};
template <int SW>
__device__ __forceinline__ PieceTok piece_tokens(int L, int c0, int c1, int lo, int hi) {
  const int v_lo = (lo > c0 ? lo : c0) - c0 - SW, v_hi = (hi < c1 ? hi : c1) - c0 - SW;
  const int t_lo = v_lo > 0 ? v_lo : 0, t_hi = v_hi > 0 ? v_hi : 0;
  PieceTok r;
  r.a = t_lo * PLAN_TILE;
  r.e = t_hi * PLAN_TILE < L ? t_hi * PLAN_TILE : L;
  r.whole = t_lo == 0 && t_hi == c1 - c0 - SW;
  return r;
}

struct BalRange {
  int lo, hi;      // plan tiles of this workgroup
  int chunk, total;
  int b0, c0;      // the last request with C_b <= lo, and its C_b
};

// One wave computes workgroup w's range (wave-uniform results; any wave may call it).
template <int SW>
__device__ inline BalRange balanced_range(const KParams& p, int w) {
  const int lane = threadIdx.x & 63;
  BalRange r;
  int total = 0;
  for (int base = 0; base < p.n_req; base += 64) {
    const int b = base + lane;
    total += __shfl(wave_incl_sum(b < p.n_req ? plan_tiles<SW>(p, b) : 0), 63, 64);
  }
  // wave-uniform values: scalar registers (shuffle results are vector registers to the compiler)
  total = __builtin_amdgcn_readfirstlane(total);
  r.total = total;
  r.chunk = total > 0 ? (total + p.nwg - 1) / p.nwg : 1;
  r.lo = w * r.chunk;
  r.hi = r.lo + r.chunk < total ? r.lo + r.chunk : total;
  r.b0 = 0;
  r.c0 = 0;
  if (r.lo >= r.hi) return r;
  int run = 0;
  for (int base = 0; base < p.n_req && run <= r.lo; base += 64) {
    const int b = base + lane;
    const int t = b < p.n_req ? plan_tiles<SW>(p, b) : 0;
    const int incl = wave_incl_sum(t);
    const int c = run + incl - t;
    const uint64_t m = __builtin_amdgcn_ballot_w64(b < p.n_req && c <= r.lo);
    if (m) {
      const int x = 63 - __builtin_clzll(m);
      r.b0 = base + x;
      r.c0 = __shfl(c, x, 64);
    }
    run += __shfl(incl, 63, 64);
  }
  r.b0 = __builtin_amdgcn_readfirstlane(r.b0);
  r.c0 = __builtin_amdgcn_readfirstlane(r.c0);
  return r;
}

// One wave of one workgroup stores the plan the balanced combine reads: [0] chunk, [1] total,
// [2 + b] = C_b for b <= n_req.
template <int SW>
__device__ inline void store_plan(const KParams& p) {
  const int lane = threadIdx.x & 63;
  int run = 0;
  for (int base = 0; base <= p.n_req; base += 64) {
    const int b = base + lane;
    const int t = b < p.n_req ? plan_tiles<SW>(p, b) : 0;
    const int incl = wave_incl_sum(t);
    if (b <= p.n_req) p.plan[2 + b] = run + incl - t;
    run += __shfl(incl, 63, 64);
  }
  if (lane == 0) {
    p.plan[0] = run > 0 ? (run + p.nwg - 1) / p.nwg : 1;
    p.plan[1] = run;
  }
}

// Tokens per split in the fixed-split mode: ceil(ceil(L/S)/align)*align (mla_decode_attention.py:389-396).
__device__ __forceinline__ int split_len(const KParams& p, int L) {
  int per = (L + p.num_splits - 1) / p.num_splits;
  if (p.split_align > 0) per = (per + p.split_align - 1) / p.split_align * p.split_align;
  return per;
}

// Output of request b's token range in this workgroup: fixed splits write the reference's
// attn_logits row of split blockIdx.x; the balanced mode writes slot blockIdx.x + b of the partial
// buffers; final_out (the workgroup covers the whole request) writes the normalized output directly.
template <int DV>
__device__ __forceinline__ SegOut seg_out(const KParams& p, int b, bool final_out, int w = -1) {
  if (w < 0) w = blockIdx.x;   // the workgroup's split (fixed) or range (balanced)
  SegOut so;
  so.final_out = final_out;
  if (p.num_splits > 0) {
    so.po = p.ws + (int64_t)b * p.qrows * p.ws_sr + (int64_t)w * p.ws_ss;
    so.po_sr = p.ws_sr;
    so.po_sh = p.ws_sh;
    so.plse = nullptr;
    so.plse_sr = 0;
  } else {
    const int nrow = p.qrows * p.heads;
    const int64_t slot = (int64_t)w + b;
    so.po = p.part_o + slot * nrow * DV;
    so.po_sr = (int64_t)p.heads * DV;
    so.po_sh = DV;
    so.plse = p.part_lse + slot * nrow;
    so.plse_sr = p.heads;
  }
  return so;
}

// Calls f(req, a, e, L, so) for every token range [a, e) this workgroup owns.
//   fixed splits (num_splits > 0): grid (S, n_req); split s covers [s*per, min((s+1)*per, L)) with
//     per = ceil(ceil(L/S)/align)*align, as the reference's stage 1 (mla_decode_attention.py:389-396);
//     partials go to attn_logits [rows, heads, S, Dv+1].
//   balanced (num_splits == 0): workgroup w owns global PLAN_TILE-token tiles [w*chunk, (w+1)*chunk)
//     of the concatenated requests; a request it covers alone is finished in place, others leave a
//     partial in slot w + b.
template <int DV, int SW, class F>
__device__ __forceinline__ void for_each_segment(const KParams& p, F&& f) {
  // one call site of f, so the (large, inlined) segment body exists once per kernel
  const bool fixed = p.num_splits > 0;
  int b_lo, b_hi, lo = 0, hi = 0, c = 0;
  if (fixed) {
    b_lo = blockIdx.y;
    b_hi = b_lo + 1;
  } else {
    const BalRange r = balanced_range<SW>(p, blockIdx.x);
    lo = r.lo;
    hi = r.hi;
    if (lo >= hi) return;
    b_lo = r.b0;   // the request whose tiles contain lo (or an empty one right before it)
    c = r.c0;
    b_hi = p.n_req;
  }
  for (int b = b_lo; b < b_hi; ++b) {
    const int L = req_len(p, b);
    int a, e;
    SegOut so;
    if (fixed) {
      const int per = split_len(p, L);
      a = per * (int)blockIdx.x;
      e = a + per < L ? a + per : L;
      so = seg_out<DV>(p, b, p.num_splits == 1);
    } else {
      const int c0 = c, c1 = c + (L > 0 ? (L + PLAN_TILE - 1) / PLAN_TILE + SW : 0);
      c = c1;
      if (c0 >= hi) break;
      if (c1 <= lo) continue;
      const PieceTok pt = piece_tokens<SW>(L, c0, c1, lo, hi);
      a = pt.a;
      e = pt.e;
      so = seg_out<DV>(p, b, pt.whole);
    }
    if (e <= a) continue;
    f(b, a, e, L, so);
  }
}

// Cached rows on 16-byte boundaries (cache base, page stride and row stride): every kernel family
// stages them with 16-byte LDS-DMA loads. Rows on 4-byte boundaries only (the unpadded 12-head rows
// of the reference's numerics test) take the narrow-row instances, which stage 4 bytes per lane.
inline bool rows16(const qmla_decode_params* p) {
  const int eb = p->kv_dtype == QMLA_KV_FP8 ? 1 : 2;
  return ((uintptr_t)p->kv_cache & 15) == 0 && (p->page_stride * eb) % 16 == 0 && (p->token_stride * eb) % 16 == 0;
}

// ---- host-side interface of the warp-specialized translation unit (qmla_ws.hip) ----
int ws_select(const qmla_decode_params* p);
int ws_head_split(const qmla_decode_params* p);
int ws_launch(int inst, const qmla_decode_params* p, const KParams& k, int nwg, hipStream_t st);

// ---- host-side interface of the row-owner translation unit (qmla_ro.hip) ----
// Index of a compiled row-owner instance for these params (GLA-g2 on fp8 + log8 rows), or -1.
int ro_select(const qmla_decode_params* p);
int ro_launch(int inst, const qmla_decode_params* p, const KParams& k, int nwg, hipStream_t st);

// ---- host-side interface of the wide-row warp-specialized translation unit (qmla_wsb.hip) ----
// Index of a compiled instance for these params (bf16 rows, the deployed fp8 rows), or -1.
int wsb_select(const qmla_decode_params* p);
int wsb_launch(int inst, const qmla_decode_params* p, const KParams& k, int nwg, hipStream_t st);

// ---- host-side interface of the column-split translation unit (qmla_cs.hip) ----
// Index of a compiled column-split instance for these params, or -1.
int cs_select(const qmla_decode_params* p);
// Workgroups per token range (row splits along gridDim.z) of the selected instance, or 0.
int cs_row_splits(const qmla_decode_params* p);
// Launch the partial pass of column-split instance `inst` (grid per split mode).
int cs_launch(int inst, const qmla_decode_params* p, const KParams& k, int nwg, hipStream_t st);

}  // namespace qmla
