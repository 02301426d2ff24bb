// Warp-per-row family for gfx950: WarpPerRow, WarpPerRowFp4, WarpPerRowSmem,
// WarpPerRowSmemFp4 (reference src/device/csrspmm_warp_per_row*.cu).
//
// Mapping (wave64): a group of G lanes owns the output columns of a row;
// lane l of the group owns column chunks l, l+G, ..., each VEC floats wide
// (VEC = 4 is the float4 "Fp4" form: 16-byte global_load_dwordx4 gathers of
// B rows).  N = 128 with VEC = 4 gives 32-lane groups, two per wave; N = 256
// fills the wave.  Each lane keeps T chunk accumulators in registers, so A is
// read once per row (the reference re-reads A once per 32-column pass,
// csrspmm_warp_per_row.cu:34-43).
//
// Per output element the products are summed in CSR order with fma, the
// order of the reference kernels (csrspmm_warp_per_row.cu:37-43), so a row
// processed whole reproduces their accumulation.  The (col, val) pairs of a
// chunk of G nonzeros are loaded coalesced (one per lane) and broadcast to
// the group: by v_readlane / ds_bpermute in the register variants, through a
// per-wave LDS stage in the Smem variants.  U independent B-row gathers are
// issued before their fmas, keeping U x VEC x 4 bytes per lane in flight.
//
// Load balance (large problems, "plan" mode):
//  * plan_kernel, one thread per row, no atomics: merge-block starts, the
//    segment slots of long rows and, with column panels, the window table.
//  * with column panels, panel_window_kernel and panel_sched_kernel
//    (panels.hip) build this call's panel schedule.
//  * rowgroup_kernel: the first blocks take the panel pieces (when there
//    are panels), then the long-row segments (partial sums to the
//    workspace); the other blocks each take one merge block of consecutive
//    short rows and stream their contiguous nonzeros, so gathers stay in
//    flight across row boundaries and a row's accumulator is flushed
//    (epilogue + store) when the stream passes its end.  With column slices
//    the segment and merge blocks repeat per slice of columns; float4
//    slices replace the merge blocks by a band sweep (sweep_rows), whose
//    groups keep their rows for the whole slice and gather from B band
//    after band.
//  * combine_kernel: adds each split or panelized row's partials in a
//    fixed order.
// Everything is deterministic (no float atomics): results repeat bit for bit.

#include "common.hpp"


namespace csrspmm_hip {

namespace {

constexpr int kWaves = 4;  // waves per block (256 threads)

// Blocks of the combine kernel that scan the segment slots (grid-strided).
#ifndef CSRSPMM_COMBINE_SCAN_BLOCKS
#define CSRSPMM_COMBINE_SCAN_BLOCKS 4096
#endif
constexpr int kCombineScanBlocks = CSRSPMM_COMBINE_SCAN_BLOCKS;

// B-row gathers in flight per lane (unroll over nonzeros) for the float4
// single-chunk kernels; build-time tunable.
#ifndef CSRSPMM_VEC4_UNROLL
#define CSRSPMM_VEC4_UNROLL 4
#endif
constexpr int kVec4U = CSRSPMM_VEC4_UNROLL;

// B-row gathers in flight per lane in the long-row segment phase, whose
// groups each walk one long dependent chain; build-time tunable.
#ifndef CSRSPMM_SEG_UNROLL
#define CSRSPMM_SEG_UNROLL 4
#endif


// Pieces per group in one pieces block (a chunk is kPiecesPerGroup * GPB
// consecutive pieces of an XCD's list); build-time tunable.  The pieces
// assigned to an XCD's resident blocks span about kPiecesPerGroup panels on
// XL (~1,500 rows per panel), and their bands compete for its 4 MiB L2.
// Measured on MI355X, the pieces alone on XL: 2 per group 188 us at an L2
// hit rate of 0.70, 1 per group 161 us at 0.89; the whole call 376 -> 369 us.
#ifndef CSRSPMM_PIECES_PER_GROUP
#define CSRSPMM_PIECES_PER_GROUP 1
#endif
constexpr int kPiecesPerGroup = CSRSPMM_PIECES_PER_GROUP;

// Band sweep kernels: gathers in flight per lane in their long-row segments,
// and the least waves per SIMD they are compiled for; build-time tunable.
#ifndef CSRSPMM_SWEEP_SU
#define CSRSPMM_SWEEP_SU 4
#endif
#ifndef CSRSPMM_SWEEP_WPE
#define CSRSPMM_SWEEP_WPE 8
#endif

// Split rows summed in the main launch (Problem::seg_fuse); 0: always the
// combine launch.
#ifndef CSRSPMM_SEG_FUSE
#define CSRSPMM_SEG_FUSE 1
#endif

// B-row gathers in flight per lane in the pieces kernel; build-time tunable.
#ifndef CSRSPMM_PIECE_UNROLL
#define CSRSPMM_PIECE_UNROLL 4
#endif

__device__ __forceinline__ void wave_lds_sync() {
  // The LDS stage is private to the wave: order its writes against the
  // group's reads (and the next chunk's overwrite) without a block barrier.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ int clamp_nnz(int x, int nnz) { return min(max(x, 0), nnz); }

// B through a buffer resource (BUF kernels): a gather's byte offset
// row * ldb * 4 + column * 4 is one 32-bit v_mad_u32_u24 instead of 64-bit
// address arithmetic, and the hardware range-checks it against B's extent (an
// offset at or past the end reads 0 and fetches nothing).  The host picks BUF
// only when B's extent is below kBufOffPast and rows and row lengths fit 24
// bits (buf_gathers_ok), so a valid offset stays below kBufOffPast, and an
// entry past a chunk's count (offset kBufOffPast plus a column byte offset)
// lies past the end without wrapping.  A lane whose column lies past the
// block's columns adds kBufOffPast to a valid row offset, which stays past
// the end only while the row offset is below 2^32 - kBufOffPast (1 GiB):
// buf_gathers_ok allows a larger B only when no lane's column can be past
// the end.
constexpr unsigned kBufOffPast = 0xC0000000u;
struct BufB {
  __amdgpu_buffer_rsrc_t rsrc;
  unsigned rowbytes;
};
__device__ __forceinline__ BufB make_bufb(const Problem& p) {
  BufB bb;
  const long long bytes = p.K > 0 ? (long long)(p.K - 1) * p.ldb * 4 + (long long)p.N * 4 : 0;
  bb.rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.B), (short)0,
                                              (int)(bytes < (long long)kBufOffPast ? bytes : 0), 0x00020000);
  bb.rowbytes = (unsigned)(p.ldb * 4);
  return bb;
}
template <int VEC>
__device__ __forceinline__ typename Vec<VEC>::T ld_b_buf(const BufB& bb, unsigned off) {
  if constexpr (VEC == 4) {
    return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(bb.rsrc, (int)off, 0, 0));
  } else {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(bb.rsrc, (int)off, 0, 0));
  }
}

// True when this call's column panels took the long row starting at
// nonzero x0 (its segments are then skipped).
__device__ __forceinline__ bool is_panelized(const Problem& p, int x0) {
  if (p.dp.P <= 0) return false;
  const int id = (clamp_nnz(x0, p.nnz) + kPanelMinLen - 1) / kPanelMinLen;
  if (id >= p.dp.nwin) return false;
  const int pi = p.dp.pidx[id];
  return pi >= 0 && pi < p.dp.sched[0];
}

// Column bookkeeping of one panel of PW = G*VEC*T columns starting at c0;
// with BUF, B's buffer resource and each column's byte offset in a B row
// (past the buffer for a column at or beyond climit, so it fetches nothing).
template <int VEC, int G, int T, bool BUF>
struct Panel {
  const float* bcol[T];
  bool cval[T];
  int col[T];
  unsigned colbytes[T];
  BufB bb;
  __device__ __forceinline__ Panel(const Problem& p, int c0, int gl, int climit) {
    if constexpr (BUF) bb = make_bufb(p);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      col[t] = c0 + (gl + G * t) * VEC;
      cval[t] = col[t] < climit;  // VEC == 4 requires N % 4 == 0 (host-checked)
      bcol[t] = p.B + col[t];
      colbytes[t] = cval[t] ? (unsigned)col[t] * 4u : kBufOffPast;
    }
  }
};

// One chunk of up to G nonzeros [base, base + cnt): broadcast each (col, val)
// to the group, gather U B-row slices at a time, and hand every product to
// `consume(j, v, b)` in CSR order (j = nonzero index).
template <int VEC, int G, int T, int U, bool LDS, bool BUF, class Consume>
__device__ __forceinline__ void chunk_gather(const Problem& p, const Panel<VEC, G, T, BUF>& pn,
                                             int base, int cnt, int cj, float vj, int gl, int gbase,
                                             int2* stage, Consume&& consume) {
  using VT = typename Vec<VEC>::T;
  if constexpr (LDS) {
    stage[gbase + gl] = make_int2(cj, __float_as_int(vj));
    wave_lds_sync();
  }
  // (col, val) of entry kk of the chunk; kk < G
  auto pair = [&](int kk, int& c, float& v) {
    if constexpr (LDS) {
      const int2 e = stage[gbase + kk];
      c = e.x;
      v = __int_as_float(e.y);
    } else {
      c = group_bcast<G>(cj, gbase, kk);
      v = group_bcast<G>(vj, gbase, kk);
    }
  };
  if constexpr (BUF) {
    // Full batches of U need no per-entry masks (k + u < cnt <= G); the
    // last, partial batch gives its missing entries an offset past the
    // buffer and skips them, and reads their (col, val) from within the
    // group (index masked: U may exceed G, as in the scalar 4-lane kernels).
    int k = 0;
    for (; k + U <= cnt; k += U) {
      int c[U];
      float v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) pair(k + u, c[u], v[u]);
      VT b[U][T];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const unsigned roff = __umul24((unsigned)c[u], pn.bb.rowbytes);
#pragma unroll
        for (int t = 0; t < T; ++t) b[u][t] = ld_b_buf<VEC>(pn.bb, roff + pn.colbytes[t]);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) consume(base + k + u, v[u], b[u]);
    }
    if (k < cnt) {
      int c[U];
      float v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) pair((k + u) & (G - 1), c[u], v[u]);
      VT b[U][T];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const unsigned roff = (k + u) < cnt ? __umul24((unsigned)c[u], pn.bb.rowbytes) : kBufOffPast;
#pragma unroll
        for (int t = 0; t < T; ++t) b[u][t] = ld_b_buf<VEC>(pn.bb, roff + pn.colbytes[t]);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if ((k + u) < cnt) consume(base + k + u, v[u], b[u]);
      }
    }
  } else {
    for (int k = 0; k < cnt; k += U) {
      int c[U];
      float v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) pair((k + u) & (G - 1), c[u], v[u]);
      VT b[U][T];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool ok = (k + u) < cnt;
        const long long roff = (long long)c[u] * p.ldb;
#pragma unroll
        for (int t = 0; t < T; ++t) {
          b[u][t] = Vec<VEC>::zero();
          if (ok && pn.cval[t]) b[u][t] = ld_b<VEC>(pn.bcol[t] + roff);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if ((k + u) < cnt) consume(base + k + u, v[u], b[u]);
      }
    }
  }
  if constexpr (LDS) wave_lds_sync();
}

// Lane gl's (col, val) of the chunk of G nonzeros starting at j0 (0 past end).
__device__ __forceinline__ void load_chunk(const Problem& p, int j0, int end, int gl, int& cj,
                                           float& vj) {
  cj = 0;
  vj = 0.0f;
  if (j0 + gl < end) {
    cj = ld_stream(p.colidx + j0 + gl);
    vj = ld_stream(p.vals + j0 + gl);
  }
}

// Walks nonzeros [start, end) in chunks of G with the next chunk's (col, val)
// prefetched, calling consume(j, v, b[T]) for each in order; (cj, vj) is the
// caller's load of the first chunk.
template <int VEC, int G, int T, int U, bool LDS, bool BUF, class Consume>
__device__ __forceinline__ void stream_nonzeros_from(const Problem& p, const Panel<VEC, G, T, BUF>& pn,
                                                     int start, int end, int cj, float vj, int gl,
                                                     int gbase, int2* stage, Consume&& consume) {
  for (int base = start; base < end; base += G) {
    const int jn = base + G + gl;
    int cn = 0;
    float vn = 0.0f;
    if (jn < end) {
      cn = ld_stream(p.colidx + jn);
      vn = ld_stream(p.vals + jn);
    }
    chunk_gather<VEC, G, T, U, LDS, BUF>(p, pn, base, min(G, end - base), cj, vj, gl, gbase, stage,
                                    consume);
    cj = cn;
    vj = vn;
  }
}

template <int VEC, int G, int T, int U, bool LDS, bool BUF, class Consume>
__device__ __forceinline__ void stream_nonzeros(const Problem& p, const Panel<VEC, G, T, BUF>& pn,
                                                int start, int end, int gl, int gbase, int2* stage,
                                                Consume&& consume) {
  int cj;
  float vj;
  load_chunk(p, start, end, gl, cj, vj);
  stream_nonzeros_from<VEC, G, T, U, LDS, BUF>(p, pn, start, end, cj, vj, gl, gbase, stage, consume);
}

template <int VEC, int T>
__device__ __forceinline__ void store_row(const Problem& p, int row, const int (&col)[T],
                                          const bool (&cval)[T], typename Vec<VEC>::T (&acc)[T]) {
  float* crow = p.C + (long long)row * p.ldc;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    if (cval[t]) store_epi<VEC>(p, crow + col[t], acc[t]);
    acc[t] = Vec<VEC>::zero();
  }
}

// Short rows [rs, re) streamed: windows of up to G consecutive rows whose
// nonzeros form one contiguous range; a row longer than kLongRow ends the
// window and is skipped (its segments are summed elsewhere).
template <int VEC, int G, int T, int U, bool LDS, bool BUF>
__device__ __forceinline__ void stream_rows(const Problem& p, const Panel<VEC, G, T, BUF>& pn, int rs,
                                            int re, int gl, int gbase, int2* stage) {
  using VT = typename Vec<VEC>::T;
  const unsigned long long gmask = G == 64 ? ~0ULL : (((1ULL << G) - 1ULL) << gbase);
  while (rs < re) {
    const int nbm = min(G, re - rs);
    int lo = 0, hi = 0;
    if (gl < nbm) {
      lo = p.rowptr[rs + gl];
      hi = p.rowptr[rs + gl + 1];
    }
    const bool is_long = gl < nbm && !p.rows_whole && (hi - lo) > p.long_row;
    const unsigned long long bl = __ballot(is_long) & gmask;
    const int nb = bl ? (__ffsll((long long)bl) - 1 - gbase) : nbm;  // rows before the first long one
    if (nb > 0) {
      const int jb = group_bcast<G>(lo, gbase, 0);
      const int je = group_bcast<G>(hi, gbase, nb - 1);
      int cur = 0;
      int cur_end = group_bcast<G>(hi, gbase, 0);
      VT acc[T];
#pragma unroll
      for (int t = 0; t < T; ++t) acc[t] = Vec<VEC>::zero();
      stream_nonzeros<VEC, G, T, U, LDS, BUF>(
          p, pn, jb, je, gl, gbase, stage, [&](int j, float v, const VT(&b)[T]) {
            // rows ending before nonzero j are complete (je bounds cur < nb)
            while (j >= cur_end) {
              store_row<VEC, T>(p, rs + cur, pn.col, pn.cval, acc);
              ++cur;
              cur_end = group_bcast<G>(hi, gbase, cur);
            }
#pragma unroll
            for (int t = 0; t < T; ++t) acc[t] = fma_v(v, b[t], acc[t]);
          });
      for (; cur < nb; ++cur) store_row<VEC, T>(p, rs + cur, pn.col, pn.cval, acc);
    }
    rs += nb + (nb < nbm ? 1 : 0);
  }
}

// Band sweep of the short rows of one column slice, or of all N <= 128
// columns (float4, 16- or 32-lane groups, B through a buffer resource).  The
// group owns rows [unit R, unit R + R) and keeps their accumulators in
// registers through the whole slice.  All
// groups start together and walk B in bands of 2^sweep_shift rows: in band
// b each row takes its nonzeros whose columns fall in the band, so at any
// time the running groups gather from about one band, which stays in the
// L2s, instead of from all of B.  Column-sorted rows take their nonzeros in
// CSR order band after band, so every row is summed in CSR order, as the
// merge blocks sum it.  `bnd` (this group's LDS) first receives each row's
// band starts: bnd[r][q] = the first nonzero whose column lies in band q or
// later (the row end when there is none), from one pass over the row's
// columns.  A row with a column out of order or out of range takes all its
// nonzeros in band 0, in CSR order.  A row longer than long_row is skipped
// (its segments are summed elsewhere) unless the rows are summed whole.
template <int G, int R, bool LDS>
__device__ __forceinline__ void sweep_rows(const Problem& p, const Panel<4, G, 1, true>& pn, int unit,
                                           int gl, int gbase, int* bnd, int2* stage) {
  static_assert(G == 16 || G == 32, "sweep groups of 16 or 32 lanes");
  constexpr int NB1 = kSweepMaxBands + 1;
  const unsigned long long gmask = ((1ull << G) - 1ull) << gbase;
  const int nb = p.sweep_bands;
  const int sh = p.sweep_shift;
  bool keep[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = unit * R + r;
    int lo = 0, hi = 0;
    if (row < p.M) {
      lo = p.rowptr[row];
      hi = p.rowptr[row + 1];
    }
    keep[r] = row < p.M && (p.rows_whole || hi - lo <= p.long_row);
    const int x0 = clamp_nnz(lo, p.nnz);
    const int x1 = keep[r] ? max(clamp_nnz(hi, p.nnz), x0) : x0;
    int* bd = bnd + r * NB1;
    // positions x0 .. x1 (x1 closes the row as band nb); the previous
    // position's band is lane gl - 1's (lane 0: the carry)
    int carry = -1;
    bool bad = false;
    for (int c = x0; c <= x1; c += G) {
      const int j = c + gl;
      int q = nb;
      if (j < x1) {
        const int col = ld_stream(p.colidx + j);
        bad |= col < 0 || col >= p.K;
        q = min(max(col, 0) >> sh, nb - 1);
      }
      int qp = group_bcast<G>(q, gbase, (gl + G - 1) & (G - 1));
      const int ql = group_bcast<G>(q, gbase, G - 1);
      if (gl == 0) qp = carry;
      carry = ql;
      if (j <= x1) {
        bad |= qp > q;
        for (int t = qp + 1; t <= q; ++t) bd[t] = j;
      }
    }
    if (__ballot(bad) & gmask) {
      wave_lds_sync();
      for (int t = gl; t <= nb; t += G) bd[t] = t == 0 ? x0 : x1;
    }
  }
  wave_lds_sync();

  f4 acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = Vec<4>::zero();
  // (col, val) of lane gl's entry of band b's chunk at `base` for every row
  auto load_chunk_rows = [&](int b, int base, int (&c)[R], float (&v)[R]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int s0 = bnd[r * NB1 + b];
      const bool in = base + gl < bnd[r * NB1 + b + 1] - s0;
      c[r] = in ? ld_stream(p.colidx + s0 + base + gl) : 0;
      v[r] = in ? ld_stream(p.vals + s0 + base + gl) : 0.0f;
    }
  };
  // (A prefetch of the next band's first chunk during this band's gathers
  // measured 1-3% slower on MI355X.)
  for (int b = 0; b < nb; ++b) {
    int cnt[R];
#pragma unroll
    for (int r = 0; r < R; ++r) cnt[r] = bnd[r * NB1 + b + 1] - bnd[r * NB1 + b];
    for (int base = 0;; base += G) {
      bool more = false;
#pragma unroll
      for (int r = 0; r < R; ++r) more |= base < cnt[r];
      if (!__any(more)) break;
      int cj[R];
      float vj[R];
      load_chunk_rows(b, base, cj, vj);
      if constexpr (LDS) {
        // the LDS-staged variant: each row's chunk through the wave's stage
#pragma unroll
        for (int r = 0; r < R; ++r) stage[r * 64 + gbase + gl] = make_int2(cj[r], __float_as_int(vj[r]));
        wave_lds_sync();
      }
      // One gather per row in flight at a time: measured on MI355X (65536 x
      // 65536 x 256, 66 per row), 2 rows x 1 ran 286 us, 2 x 2 427 us, 1 x 2
      // 310 us, 1 x 4 477 us.  An entry past a row's count gets an offset
      // past the buffer (nothing fetched) and a value of 0, which leaves the
      // accumulator as it is.
      for (int k = 0; k < G; ++k) {
        bool any = false;
#pragma unroll
        for (int r = 0; r < R; ++r) any |= base + k < cnt[r];
        if (!__any(any)) break;
        f4 bv[R];
        float v[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          int c;
          if constexpr (LDS) {
            const int2 e = stage[r * 64 + gbase + k];
            c = e.x;
            v[r] = __int_as_float(e.y);
          } else {
            c = group_bcast<G>(cj[r], gbase, k);
            v[r] = group_bcast<G>(vj[r], gbase, k);
          }
          const unsigned off =
              base + k < cnt[r] ? __umul24((unsigned)c, pn.bb.rowbytes) + pn.colbytes[0] : kBufOffPast;
          bv[r] = ld_b_buf<4>(pn.bb, off);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = fma_v(v[r], bv[r], acc[r]);
      }
      if constexpr (LDS) wave_lds_sync();  // the chunk is read before the next overwrites it
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    f4 a[1] = {acc[r]};
    if (keep[r]) store_row<4, 1>(p, unit * R + r, pn.col, pn.cval, a);
  }
}

// Pieces of this call's column panels, run by the first blocks of the main
// launch.  Pieces block b takes chunk b / kXcds of XCD b mod kXcds's piece
// list: kPiecesPerGroup * GPB consecutive pieces, group g taking pieces
// g, g + GPB, ... of the chunk.  XCD x's list holds, panel by panel through
// its range [qa, qb), piece i = (panel qa + i / nl, panelized row i mod nl):
// the nonzeros of that row whose columns fall in the panel, summed into the
// partial (row, panel).  Block b runs on XCD b mod kXcds, and blocks are
// dispatched in order, so the running blocks of an XCD hold a short stretch
// of its list, within a panel or two, and gather from a band of B that stays
// in that XCD's L2; the hardware dispatcher balances the uneven pieces.  The
// grid covers nl_max rows (the host cannot know nl); chunks past the list
// exit at once, and they come last.  The short-row and segment blocks follow
// in the same grid and take over slots as the pieces run out.
template <int VEC, int G, int T, int U, bool LDS, bool BUF>
__device__ __forceinline__ void pieces_body(const Problem& p, int block, int gl, int gbase, int gid,
                                            int2* stage) {
  using VT = typename Vec<VEC>::T;
  constexpr int GPB = kWaves * (64 / G);
  constexpr int PW = G * VEC * T;
  constexpr int UP = CSRSPMM_PIECE_UNROLL < G ? CSRSPMM_PIECE_UNROLL : G;
  const DevPanels& d = p.dp;
  const int nl = d.sched[0];
  if (nl <= 0) return;
  const int x = block % kXcds;
  const int qa = d.sched[1 + x];
  const unsigned n_all = (unsigned)max(d.sched[2 + x] - qa, 0) * (unsigned)nl;
  const unsigned first = (unsigned)(block / kXcds) * (unsigned)(kPiecesPerGroup * GPB);
  if (first >= n_all) return;
  const unsigned n = min(n_all, first + (unsigned)(kPiecesPerGroup * GPB));
  const unsigned stride = (unsigned)GPB;
  unsigned i = first + (unsigned)gid;
  if (i >= n) return;
  const int P1 = d.P + 1;
  auto bounds = [&](unsigned k, int id, int& a, int& e) {
    const int* b = d.bnd + (long long)id * P1 + (qa + (int)(k / (unsigned)nl));
    a = min(max(b[0], 0), p.nnz);  // a malformed CSR cannot send the loads out of A
    e = min(max(b[1], a), p.nnz);
  };
  // Software pipeline: while piece i is summed, the bounds of piece i + stride
  // and the row id of piece i + 2 stride are in flight, and the first chunk
  // of piece i + stride is loaded before piece i's partial is stored.
  int a, e;
  bounds(i, d.list[i % (unsigned)nl], a, e);
  int id1 = i + stride < n ? d.list[(i + stride) % (unsigned)nl] : 0;
  int cj;
  float vj;
  load_chunk(p, a, e, gl, cj, vj);
  for (;;) {
    const unsigned i1 = i + stride;
    int a1 = 0, e1 = 0, id2 = 0;
    if (i1 < n) {
      bounds(i1, id1, a1, e1);
      if (i1 + stride < n) id2 = d.list[(i1 + stride) % (unsigned)nl];
    }
    const int q = qa + (int)(i / (unsigned)nl);
    float* prow = d.part + ((long long)(i % (unsigned)nl) * d.P + q) * p.ldp;
    const Panel<VEC, G, T, BUF> pn0(p, 0, gl, p.N);
    VT acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = Vec<VEC>::zero();
    stream_nonzeros_from<VEC, G, T, UP, LDS, BUF>(p, pn0, a, e, cj, vj, gl, gbase, stage,
                                             [&](int, float v, const VT(&bv)[T]) {
#pragma unroll
                                               for (int t = 0; t < T; ++t) acc[t] = fma_v(v, bv[t], acc[t]);
                                             });
    if (i1 < n) load_chunk(p, a1, e1, gl, cj, vj);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      if (pn0.cval[t]) *reinterpret_cast<VT*>(prow + pn0.col[t]) = acc[t];
    }
    // columns beyond the first PW (N > G * VEC * T): the rest of the piece, plainly
    for (int c0 = PW; c0 < p.N; c0 += PW) {
      const Panel<VEC, G, T, BUF> pn(p, c0, gl, p.N);
#pragma unroll
      for (int t = 0; t < T; ++t) acc[t] = Vec<VEC>::zero();
      stream_nonzeros<VEC, G, T, UP, LDS, BUF>(p, pn, a, e, gl, gbase, stage,
                                          [&](int, float v, const VT(&bv)[T]) {
#pragma unroll
                                            for (int t = 0; t < T; ++t) acc[t] = fma_v(v, bv[t], acc[t]);
                                          });
#pragma unroll
      for (int t = 0; t < T; ++t) {
        if (pn.cval[t]) *reinterpret_cast<VT*>(prow + pn.col[t]) = acc[t];
      }
    }
    if (i1 >= n) break;
    i = i1;
    a = a1;
    e = e1;
    id1 = id2;
  }
}

// Partials k = q, q + NG, q + 2*NG, ... (k < n) of one lane's four columns,
// added in that order; partial k sits at src + idx(k) * ldp, idx(k) =
// pieces[k] when a piece list is given, else k.  Partial rows are ldp = N
// rounded up to 4 floats long and 256-byte aligned, so they are read as
// float4 whatever the alignment of C.
template <int NG>
__device__ __forceinline__ f4 sum_strided(const float* src, const int* pieces, int n, int q,
                                          long long ldp, bool cv) {
  f4 acc = Vec<4>::zero();
  if (!cv) return acc;
  auto part = [&](int k) -> f4 {
    const long long idx = pieces ? (long long)pieces[k] : (long long)k;
    return *reinterpret_cast<const f4*>(src + idx * ldp);
  };
  int k = q;
  for (; k + 7 * NG < n; k += 8 * NG) {
    f4 a[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) a[u] = part(k + u * NG);
#pragma unroll
    for (int u = 0; u < 8; ++u) acc = add_v(acc, a[u]);
  }
  for (; k < n; k += NG) acc = add_v(acc, part(k));
  return acc;
}

// The value of lane (this lane ^ OFF), OFF in {8, 16, 32}: a DPP row_ror:8
// (rotating a 16-lane row by half of it is the xor), a ds_swizzle swapping the
// 16-lane halves of each 32-lane group (bit mode: and 0x1f, xor 0x10), and a
// ds_bpermute across the 32-lane halves, which no gfx9 DPP or swizzle crosses.
template <int OFF>
__device__ __forceinline__ float lane_xor(float v) {
  const int x = __builtin_bit_cast(int, v);
  int y;
  if constexpr (OFF == 8) {
    y = __builtin_amdgcn_update_dpp(0, x, 0x128 /* row_ror:8 */, 0xF, 0xF, false);
  } else if constexpr (OFF == 16) {
    y = __builtin_amdgcn_ds_swizzle(x, 0x401F);
  } else {
    static_assert(OFF == 32, "lane_xor: offsets 8, 16, 32");
    y = __builtin_amdgcn_ds_bpermute((lane_id() ^ 32) << 2, x);
  }
  return __builtin_bit_cast(float, y);
}

template <int OFF>
__device__ __forceinline__ f4 add_lane_xor(f4 v) {
  return f4{v.x + lane_xor<OFF>(v.x), v.y + lane_xor<OFF>(v.y), v.z + lane_xor<OFF>(v.z),
            v.w + lane_xor<OFF>(v.w)};
}

// Sum over the 64 / GC lane groups of a wave by a fixed xor tree (offsets GC,
// 2 GC, ... 32); every group ends with the total.  All lanes take part.
template <int GC>
__device__ __forceinline__ f4 wave_group_sum(f4 v) {
  static_assert(GC == 8 || GC == 16 || GC == 32 || GC == 64, "group widths of the combine");
  if constexpr (GC <= 8) v = add_lane_xor<8>(v);
  if constexpr (GC <= 16) v = add_lane_xor<16>(v);
  if constexpr (GC <= 32) v = add_lane_xor<32>(v);
  return v;
}

// Columns c .. c + 3 of a C row (those below N): one float4 store when C
// rows are 16-byte aligned (VEC == 4, N % 4 == 0), else one per column.
template <int VEC>
__device__ __forceinline__ void store_cols4(const Problem& p, float* cptr, int c, f4 v) {
  if constexpr (VEC == 4) {
    store_epi<4>(p, cptr, v);
  } else {
    store_epi<1>(p, cptr, v.x);
    if (c + 1 < p.N) store_epi<1>(p, cptr + 1, v.y);
    if (c + 2 < p.N) store_epi<1>(p, cptr + 2, v.z);
    if (c + 3 < p.N) store_epi<1>(p, cptr + 3, v.w);
  }
}

// Split rows summed in the main launch (Problem::seg_fuse).  A segment's
// partial row is stored, and the rows' partials are read back, with
// agent-scope atomic stores and loads (sc1: past this XCD's L2, to where
// every XCD sees them), and a segment's stores are complete (vmcnt 0) before
// it counts itself, so the last count of a row finds all its partials.
__device__ __forceinline__ void store_partial(float* dst, f4 v) {
#pragma unroll
  for (int i = 0; i < 4; ++i) __hip_atomic_store(dst + i, v[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_partial(float* dst, float v) {
  __hip_atomic_store(dst, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// sum_strided over the partial rows of one split row through a buffer
// resource on them, with agent-scope coherent (sc1) loads: the same adds in
// the same order.  Byte offsets fit 31 bits (launch_rowgroup_all fuses only
// when the whole partial buffer does).
constexpr int kCpolSc1 = 16;  // the sc1 cache-policy bit of buffer instructions
template <int NG>
__device__ __forceinline__ f4 sum_strided_coh(__amdgpu_buffer_rsrc_t rsrc, int c, int n, int q, long long ldp,
                                              bool cv) {
  f4 acc = Vec<4>::zero();
  if (!cv) return acc;
  auto part = [&](int k) -> f4 {
    const int off = (int)(((long long)k * ldp + c) * 4);
    return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, kCpolSc1));
  };
  int k = q;
  for (; k + 3 * NG < n; k += 4 * NG) {
    f4 a[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) a[u] = part(k + u * NG);
#pragma unroll
    for (int u = 0; u < 4; ++u) acc = add_v(acc, a[u]);
  }
  for (; k < n; k += NG) acc = add_v(acc, part(k));
  return acc;
}

// The split rows that this wave's groups counted last (lanes in `pend`, each
// holding row, segments n and first position x0), one after another with
// the whole wave, in the combine's lane layout and order (combine_kernel's
// slot scan: GC lanes a float4 chunk, 64 / GC groups adding strided
// partials, then the xor tree), so a fused row is bit for bit the combined
// one.
template <int VEC, int GC>
__device__ __forceinline__ void fused_rows(const Problem& p, unsigned long long pend, int row, int n, int x0) {
  constexpr int P = 64 / GC;
  const int lane = lane_id();
  const int q = lane / GC;
  const int gl = lane & (GC - 1);
  while (pend) {
    const int l = __ffsll((long long)pend) - 1;
    pend &= pend - 1;
    const int r = __builtin_amdgcn_readlane(row, l);
    const int nn = __builtin_amdgcn_readlane(n, l);
    float* base = p.partials + (long long)(__builtin_amdgcn_readlane(x0, l) >> p.seg_shift) * p.ldp;
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(base, (short)0, (int)((long long)nn * p.ldp * 4), 0x00020000);
    float* crow = p.C + (long long)r * p.ldc;
    for (int c0 = 0; c0 < p.N; c0 += GC * 4) {
      const int c = c0 + gl * 4;
      const bool cv = c < p.N;
      const f4 acc = wave_group_sum<GC>(sum_strided_coh<P>(rsrc, c, nn, q, p.ldp, cv));
      if (q == 0 && cv) store_cols4<VEC>(p, crow + c, c, acc);
    }
  }
}

// One block's share of the main launch, over the columns [c_lo, c_hi):
// block bid < seg_blocks takes long-row segment slots, the others merge
// blocks of short rows (or, without a plan, rows).
template <int VEC, int G, int T, int U, bool LDS, bool BUF, int SU, bool SWEEP, bool FUSE>
__device__ __forceinline__ void rowgroup_block(const Problem& p, int bid, int seg_blocks, int c_lo,
                                               int c_hi, int gl, int gbase, int gid, int2* stage,
                                               int* sweep_bnd) {
  using VT = typename Vec<VEC>::T;
  constexpr int GPB = kWaves * (64 / G);
  constexpr int PW = G * VEC * T;
  if (bid < seg_blocks) {
    // Long-row segments, one slot per group (grid-strided if the segment
    // blocks are capped).  FUSE: the group whose segment of a split row
    // counts last (over every column slice) notes the row in fuse_row, and
    // once the gathers are done its wave sums the rows its groups noted.
    constexpr int US = SU > U ? (SU < G ? SU : G) : U;
    auto slot = [&](int s, int& fuse_row, int& fuse_n, int& fuse_x0) {
      const int2 si = p.seg_info[s];
      if (si.x < 0 || si.x >= p.M) return;  // unused slot
      const int rs = p.rowptr[si.x];
      const int re = p.rowptr[si.x + 1];
      const int len = re - rs;
      if (len >= kPanelMinLen && is_panelized(p, rs)) return;  // summed by the pieces kernel
      const int nseg = seg_count(p, len);
      const int start = rs + seg_begin(len, nseg, si.y);
      const int end = rs + seg_begin(len, nseg, si.y + 1);
      // partial si.y of the row (si.y < the segments plan_kernel counted
      // from the clamped row range, so this stays inside the buffer)
      float* prow = p.partials + ((long long)(clamp_nnz(rs, p.nnz) >> p.seg_shift) + si.y) * p.ldp;
      for (int c0 = c_lo; c0 < c_hi; c0 += PW) {
        const Panel<VEC, G, T, BUF> pn(p, c0, gl, c_hi);
        VT acc[T];
#pragma unroll
        for (int t = 0; t < T; ++t) acc[t] = Vec<VEC>::zero();
        stream_nonzeros<VEC, G, T, US, LDS, BUF>(p, pn, start, end, gl, gbase, stage,
                                            [&](int, float v, const VT(&b)[T]) {
#pragma unroll
                                              for (int t = 0; t < T; ++t) acc[t] = fma_v(v, b[t], acc[t]);
                                            });
        if (nseg == 1) {  // the whole row: epilogue and store here
          store_row<VEC, T>(p, si.x, pn.col, pn.cval, acc);
        } else if constexpr (FUSE) {
#pragma unroll
          for (int t = 0; t < T; ++t) {
            if (pn.cval[t]) store_partial(prow + pn.col[t], acc[t]);
          }
        } else {
#pragma unroll
          for (int t = 0; t < T; ++t) {
            if (pn.cval[t]) *reinterpret_cast<VT*>(prow + pn.col[t]) = acc[t];
          }
        }
      }
      if constexpr (FUSE) {
        // The wait also keeps the compiler from holding the row's values
        // across the gathers above (they are read again).
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this group's partials are stored
        const int row = p.seg_info[s].x;
        const int r0 = p.rowptr[row];
        const int n = seg_count(p, p.rowptr[row + 1] - r0);
        if (n > 1) {
          // every segment of the row in every column slice counts once
          const int ns = p.sw > 0 ? (p.N + p.sw - 1) / p.sw : 1;
          const int x0 = clamp_nnz(r0, p.nnz);
          int seen = 0;
          if (gl == 0)
            seen = __hip_atomic_fetch_add(p.seg_cnt + (x0 >> p.slot_shift), 1, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
          seen = group_bcast<G>(seen, gbase, 0);
          if (seen == n * ns - 1) {
            fuse_row = row;
            fuse_n = n;
            fuse_x0 = x0;
          }
        }
      }
    };
    int fuse_row = -1, fuse_n = 0, fuse_x0 = 0;
    if constexpr (FUSE) {
      // one slot per group: a fused launch's segment blocks are not capped
      // (launch_rowgroup_all)
      const int s = bid * GPB + gid;
      if (s < p.nslots) slot(s, fuse_row, fuse_n, fuse_x0);
      // the whole wave, its groups' rows one after another (GC as launch_combine picks it)
      const unsigned long long pend = __ballot(fuse_row >= 0 && gl == 0);
      if (pend) {
        const int chunks = (p.N + 3) / 4;
        if (chunks <= 8) {
          fused_rows<VEC, 8>(p, pend, fuse_row, fuse_n, fuse_x0);
        } else if (chunks <= 16) {
          fused_rows<VEC, 16>(p, pend, fuse_row, fuse_n, fuse_x0);
        } else if (chunks <= 32) {
          fused_rows<VEC, 32>(p, pend, fuse_row, fuse_n, fuse_x0);
        } else {
          fused_rows<VEC, 64>(p, pend, fuse_row, fuse_n, fuse_x0);
        }
      }
    } else {
      for (int s = bid * GPB + gid; s < p.nslots; s += seg_blocks * GPB) slot(s, fuse_row, fuse_n, fuse_x0);
    }
    return;
  }

  const int unit = (bid - seg_blocks) * GPB + gid;
  if constexpr (SWEEP) {
    // The band sweep of a column slice (or of all N <= 128 columns):
    // kSweepRows rows per group.
    static_assert(VEC == 4 && (G == 16 || G == 32) && T == 1 && BUF,
                  "the sweep runs float4 groups of up to 128 columns");
    const Panel<VEC, G, T, BUF> pn(p, c_lo, gl, c_hi);
    sweep_rows<G, kSweepRows, LDS>(p, pn, unit, gl, gbase, sweep_bnd + gid * kSweepRows * (kSweepMaxBands + 1),
                                   stage);
    return;
  }
  if (p.plan) {
    // One merge block of short rows.
    if (unit >= p.nblocks) return;
    const int rs = max(0, p.block_start[unit]);
    const int re = min(p.M, p.block_start[unit + 1]);
    for (int c0 = c_lo; c0 < c_hi; c0 += PW) {
      const Panel<VEC, G, T, BUF> pn(p, c0, gl, c_hi);
      stream_rows<VEC, G, T, U, LDS, BUF>(p, pn, rs, re, gl, gbase, stage);
    }
    return;
  }

  // No plan: one row per group, summed whole.
  const int row = unit;
  if (row >= p.M) return;
  const int start = p.rowptr[row];
  const int end = p.rowptr[row + 1];
  for (int c0 = c_lo; c0 < c_hi; c0 += PW) {
    const Panel<VEC, G, T, BUF> pn(p, c0, gl, c_hi);
    VT acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = Vec<VEC>::zero();
    stream_nonzeros<VEC, G, T, U, LDS, BUF>(p, pn, start, end, gl, gbase, stage,
                                       [&](int, float v, const VT(&b)[T]) {
#pragma unroll
                                         for (int t = 0; t < T; ++t) acc[t] = fma_v(v, b[t], acc[t]);
                                       });
    store_row<VEC, T>(p, row, pn.col, pn.cval, acc);
  }
}

// The main launch with column panels holds piece_blocks pieces blocks (a
// multiple of kXcds) and the blocks of the other roles (segments, merge
// blocks).  The pieces gather from an L2-resident band and are bound by L2
// bandwidth; the other roles gather at random and are bound by L2 misses.
// Run back to back on XL they take 161 + 182 us; interleaved, they overlap.
// Grid block b belongs to group b / kXcds (one block per XCD); the groups
// cycle through kInterPieces groups of pieces blocks, then kInterRest groups
// of the other roles, until one role runs out, and the rest of the grid is
// the remaining role.  Pieces block i keeps running on XCD i mod kXcds.
// Measured on MI355X per call (float4 columns; ratio pieces : other):
//   XL         pieces first 369.5 us, 1:1 419.7, 2:1 349.2, 3:2 346.7,
//              4:3 345.3, 5:4 344.9, 3:1 387.2, 4:1 362.3
//   XL-98      1073.2 us -> 1002.7 (4:3)
//   power-law rows, K = 131072, N = 128: 198.4 -> 192.5 us (4:3)
// A cycle of 4 groups (3:1, and 1:1 at 2) put the other roles' blocks on the
// same CUs of each XCD every time; 4:3 cycles through 7.  Scalar-column
// calls keep the pieces first: interleaved, XL WarpPerRow went 514 -> 523 us.
constexpr int kInterPieces = 4;
constexpr int kInterRest = 3;
__device__ __forceinline__ void interleave_roles(int b, int piece_blocks, int total, int& piece,
                                                 int& other) {
  const int pg = piece_blocks / kXcds;
  const int rg = (total - piece_blocks) / kXcds;
  const int g = b / kXcds, x = b % kXcds;
  constexpr int kCycle = kInterPieces + kInterRest;
  const int cycles = min(pg / kInterPieces, rg / kInterRest);
  if (g < cycles * kCycle) {
    const int c = g / kCycle, k = g % kCycle;
    if (k < kInterPieces) {
      piece = (c * kInterPieces + k) * kXcds + x;
    } else {
      piece = -1;
      other = (c * kInterRest + (k - kInterPieces)) * kXcds + x;
    }
    return;
  }
  // past the cycles: the remaining pieces blocks, then the remaining others
  const int t = (g - cycles * kCycle) * kXcds + x;
  const int pdone = cycles * kInterPieces * kXcds;
  if (pdone + t < piece_blocks) {
    piece = pdone + t;
  } else {
    piece = -1;
    other = cycles * kInterRest * kXcds + (pdone + t - piece_blocks);
  }
}

// PIECES: compiled with the panel pieces (launched only for calls with
// column panels).  The kernels of calls without them are compiled without
// that code, which as dead code cost the scalar N <= 64 kernel 9% on R-MAT
// and the scalar N = 128 / 256 kernels 3-18% on the reference's sweep shapes.
// FUSE: the segment blocks sum the split rows themselves (Problem::seg_fuse),
// in instances of their own, so that the other kernels keep their registers.
template <int VEC, int G, int T, int U, bool LDS, bool PIECES, int SU, bool BUF, bool SWEEP, bool FUSE = false>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(SWEEP ? CSRSPMM_SWEEP_WPE : 1))) void rowgroup_kernel(Problem p, int piece_blocks,
                                                                int seg_blocks, int slice_blocks,
                                                                int slice0) {
  constexpr int GPW = 64 / G;  // groups per wave
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gl = lane & (G - 1);
  const int gbase = lane & ~(G - 1);
  const int gid = wave * GPW + lane / G;  // group index within block

  // the LDS variants' per-wave stage: 64 (col, val) pairs, one row's chunk
  // each for the sweep's kSweepRows rows
  constexpr int kStage = 64 * (SWEEP ? kSweepRows : 1);
  __shared__ int2 stage_all[LDS ? kWaves * kStage : 1];
  int2* stage = stage_all + (LDS ? wave * kStage : 0);
  // band starts of the sweep's rows, kSweepRows x (kSweepMaxBands + 1) per group
  __shared__ int sweep_bnd[SWEEP ? kWaves * GPW * kSweepRows * (kSweepMaxBands + 1) : 1];

  int bid = (int)blockIdx.x - piece_blocks;
  if constexpr (PIECES) {
    int piece = -1;
    if constexpr (VEC == 4) {
      interleave_roles((int)blockIdx.x, piece_blocks, (int)gridDim.x, piece, bid);
    } else if ((int)blockIdx.x < piece_blocks) {
      piece = (int)blockIdx.x;
    }
    if (piece >= 0) {
      pieces_body<VEC, G, T, U, LDS, BUF>(p, piece, gl, gbase, gid, stage);
      return;
    }
  }
  // Column slices: the blocks of slice sl cover columns [c_lo, c_hi), and a
  // launch holds one slice or all of them in slice order (launch_rg).
  int c_lo = 0, c_hi = p.N;
  if (p.sw > 0) {
    int local;
    if (p.xslice) {  // all slices in this launch, interleaved block by block
      const int ns = (p.N + p.sw - 1) / p.sw;
      local = bid % ns;
      bid /= ns;
    } else {
      local = bid / slice_blocks;  // bid counts from this launch's first slice, slice0
      bid -= local * slice_blocks;  // now in [0, slice_blocks)
    }
    c_lo = (slice0 + local) * p.sw;
    c_hi = min(p.N, c_lo + p.sw);
  }
  if constexpr (!PIECES) {
    // The segment blocks come after the merge blocks of their slice in the
    // grid (rowgroup_block numbers them first): on a matrix without long
    // rows they only find empty slots, and first they held dispatch slots
    // the merge blocks were waiting for.  Measured on MI355X per call
    // (bit-identical): large 4 x 74.2 -> 72.3 us, medium main kernel 40.7 ->
    // 40.2 us, with a base-size workspace (no panels, no shares) R-MAT
    // WarpPerRowSmem 590 -> 552 us and WarpPerRowFp4 613 -> 579, XL-98
    // 1816 -> 1795; XL WarpPerRowFp4 without panels 631 -> 651.  The pieces
    // kernels interleave the roles instead (interleave_roles).
    if (seg_blocks > 0) {
      const int units = slice_blocks - seg_blocks;
      bid = bid >= units ? bid - units : bid + seg_blocks;
    }
  }
  rowgroup_block<VEC, G, T, U, LDS, BUF, SU, SWEEP, FUSE>(p, bid, seg_blocks, c_lo, c_hi, gl, gbase, gid, stage,
                                                     sweep_bnd);
}

// The combine checks the row blocks' flags (Problem::need) only without
// column panels or XCD shares, which come with long rows: there the check
// would only add its loads (XL: combine 10.6 -> 12.0 us, plan_kernel 6.3 ->
// 6.9).
__device__ __forceinline__ bool need_checked(const Problem& p) {
  return p.need != nullptr && p.dp.P == 0 && !p.shares;
}

// Table entries of one row r: the merge-block starts [b_lo, b_hi], the
// segment slots [s0, s1) (the first nseg hold segments) and the windows
// [w0, w1), each range walked from `first` in steps of `step`.
__device__ __forceinline__ void plan_row_entries(const Problem& p, int r, int b_lo, int b_hi, int s0,
                                                 int s1, int nseg, int w0, int w1, int x0, int x1,
                                                 int first, int step) {
  for (int b = b_lo + first; b <= b_hi; b += step) p.block_start[b] = r;
  for (int s = s0 + first; s < s1; s += step)
    p.seg_info[s] = (s - s0) < nseg ? make_int2(r, s - s0) : make_int2(-1, 0);
  if (p.seg_fuse && first == 0 && nseg >= 2 && s0 < s1) p.seg_cnt[s0] = 0;
  // the first window of a long row is the row's id
  for (int w = w0 + first; w < w1; w += step) {
    const int id = (w == w0 && x1 - x0 >= kPanelMinLen) ? 1 : 0;
    p.dp.win[w] = make_int4(r, x0, x1, id);
    p.dp_flag[w] = (unsigned char)id;
  }
}

// A row with more table entries than this has them written by its whole
// wave, 64 per store instruction, instead of by its own lane one at a time:
// a long row covers hundreds of merge blocks, and one lane holds at most 63
// stores in flight.  Below it, the lanes write their rows in parallel (the
// wave-wide path takes the rows one after another).
#ifndef CSRSPMM_PLAN_SOLO_ENTRIES
#define CSRSPMM_PLAN_SOLO_ENTRIES 32
#endif
constexpr int kPlanSoloEntries = CSRSPMM_PLAN_SOLO_ENTRIES;

// Column boundaries of the XCD shares (the first block of plan_kernel, 256
// threads, next to the row blocks): the columns at kShareSamples hashed
// positions of colidx, counted in kShareBins bins of 2^hs columns;
// boundary x (x = 1 .. 7) is the first column of the first bin whose
// inclusive count reaches x / kXcds of the sample, so each XCD range carries
// about an eighth of it.  Boundary 0 is 0 and boundary kXcds is K.  Only the
// locality depends on them.  (Computing them in every block of plan_kernel
// from the same sample took 16.7 M L2 requests on R-MAT: plan_kernel 13 ->
// 223 us; in block 0, which holds the first and often longest rows, 12 ->
// 24 us.)
__device__ __forceinline__ void share_cut(const Problem& p) {
  __shared__ int hist[kShareBins];
  constexpr int kPer = kShareSamples / 256;
  constexpr int kBinsPerLane = kShareBins / 64;
  const int t = (int)threadIdx.x;
  for (int i = t; i < kShareBins; i += 256) hist[i] = 0;
  int hs = 0;
  while (((long long)(p.K - 1) >> hs) >= kShareBins) ++hs;
  // positions from a multiplicative hash of the sample index: evenly spaced
  // ones fall on the same place in every row when the spacing is a multiple
  // of the row length (uniform rows of 200 over 52 M nonzeros: every sample
  // a row's smallest column, and one XCD range held 99% of the nonzeros)
  int cv[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const unsigned long long i = (unsigned long long)(u * 256 + t) + 1;
    const unsigned long long h = (i * 0x9E3779B97F4A7C15ull) >> 32;
    cv[u] = p.nnz > 0 ? p.colidx[(int)(h % (unsigned long long)p.nnz)] : -1;
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kPer; ++u)
    if (cv[u] >= 0 && cv[u] < p.K) atomicAdd(&hist[cv[u] >> hs], 1);
  __syncthreads();
  if (t >= 64) return;
  int h[kBinsPerLane];
  int mine = 0;
#pragma unroll
  for (int b = 0; b < kBinsPerLane; ++b) {
    h[b] = hist[t * kBinsPerLane + b];
    mine += h[b];
  }
  int incl = mine;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(incl, off);
    if (t >= off) incl += o;
  }
  const long long total = __shfl(incl, 63);
  int run = incl - mine;
  int below[kXcds - 1];
#pragma unroll
  for (int x = 0; x < kXcds - 1; ++x) below[x] = 0;
#pragma unroll
  for (int b = 0; b < kBinsPerLane; ++b) {
    run += h[b];
#pragma unroll
    for (int x = 0; x < kXcds - 1; ++x) below[x] += (long long)run * kXcds < (long long)(x + 1) * total;
  }
#pragma unroll
  for (int x = 0; x < kXcds - 1; ++x)
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) below[x] += __shfl_xor(below[x], off);
  if (t == 0) {
#pragma unroll
    for (int x = 0; x < kXcds - 1; ++x) {
      const long long c = total > 0 ? (long long)below[x] << hs : (long long)p.K * (x + 1) / kXcds;
      p.shr_cb[x] = (int)min(c, (long long)p.K);
    }
  }
}

// The boundaries 1 .. kXcds - 1 plan_kernel wrote, made non-decreasing and
// clamped to [0, K].
__device__ __forceinline__ void share_cols(const Problem& p, int (&cb)[kXcds - 1]) {
  int prev = 0;
#pragma unroll
  for (int x = 0; x < kXcds - 1; ++x) {
    prev = min(max(p.shr_cb[x], prev), p.K);
    cb[x] = prev;
  }
}

// One thread per row r in [0, M]: the merge-block starts that fall on r, the
// segment slots r owns and, with column panels, the windows that begin in r.
// Every entry the main kernel reads is written here on each call, from
// rowptr alone (no atomics); with panels, the first row block also zeroes
// the sampled panel loads that panel_window_kernel adds to.  With XCD shares
// the grid has one more block, the first, which only writes the shares'
// column boundaries (share_cut) while the row blocks run.
__global__ __launch_bounds__(256) void plan_kernel(Problem p) {
  const int first = p.shares ? 1 : 0;  // blocks before the row blocks
  if ((int)blockIdx.x < first) {
    share_cut(p);
    return;
  }
  const int rblock = (int)blockIdx.x - first;
  const int stride = ((int)gridDim.x - first) * blockDim.x;
  const int mshift = __builtin_ctz((unsigned)p.mblk);  // mblk is a power of two
  const int lane = lane_id();
  if (p.dp.P > 0 && rblock == 0)
    for (int q = (int)threadIdx.x; q < p.dp.P; q += blockDim.x) p.dp.sched[kPanelHist + q] = 0;
  int need = 0;  // a row of this block needs the combine
  // block-uniform trip count, so every wave reaches the ballot below whole
  for (int base = rblock * blockDim.x; base <= p.M; base += stride) {
    const int r = base + (int)threadIdx.x;
    int b_lo = 0, b_hi = -1, s0 = 0, s1 = 0, nseg = 0, w0 = 0, w1 = 0, x0 = 0, x1 = 0;
    if (r <= p.M) {
      x0 = clamp_nnz(p.rowptr[r], p.nnz);
      // merge blocks b with F(r-1) < b*mblk <= F(r) start at row r
      const long long F = (long long)r + x0;
      const long long Fprev = r > 0 ? (long long)(r - 1) + clamp_nnz(p.rowptr[r - 1], p.nnz) : -1;
      b_lo = Fprev < 0 ? 0 : (int)((Fprev >> mshift) + 1);
      b_hi = (int)min(F >> mshift, (long long)p.nblocks - 1);
      if (r == p.M) {
        p.block_start[p.nblocks] = p.M;
      } else {
        // slots [x0 / S, x1 / S) belong to row r; a long row uses the first nseg
        x1 = clamp_nnz(p.rowptr[r + 1], p.nnz);
        s0 = x0 >> p.slot_shift;
        s1 = min(max(s0, x1 >> p.slot_shift), p.nslots);
        nseg = seg_count(p, x1 - x0);
        need |= nseg >= 2 || (p.shares && nseg >= 1) || (p.dp.P > 0 && x1 - x0 >= kPanelMinLen);
        if (p.dp.P > 0) {
          // windows w whose first position w * kPanelMinLen lies in this row
          w0 = (x0 + kPanelMinLen - 1) / kPanelMinLen;
          w1 = max(w0, min((x1 + kPanelMinLen - 1) / kPanelMinLen, p.dp.nwin));
        }
      }
    }
    const int entries = max(b_hi - b_lo + 1, 0) + (s1 - s0) + (w1 - w0);
    const bool solo = entries <= kPlanSoloEntries;
    if (solo) plan_row_entries(p, r, b_lo, b_hi, s0, s1, nseg, w0, w1, x0, x1, 0, 1);
    unsigned long long heavy = __ballot(!solo);
    while (heavy) {
      const int l = __ffsll((long long)heavy) - 1;
      heavy &= heavy - 1;
      plan_row_entries(p, __builtin_amdgcn_readlane(r, l), __builtin_amdgcn_readlane(b_lo, l),
                       __builtin_amdgcn_readlane(b_hi, l), __builtin_amdgcn_readlane(s0, l),
                       __builtin_amdgcn_readlane(s1, l), __builtin_amdgcn_readlane(nseg, l),
                       __builtin_amdgcn_readlane(w0, l), __builtin_amdgcn_readlane(w1, l),
                       __builtin_amdgcn_readlane(x0, l), __builtin_amdgcn_readlane(x1, l), lane, 64);
    }
  }
  if (need_checked(p)) {
    need = __syncthreads_or(need);
    if (threadIdx.x == 0 && rblock < p.need_blocks) p.need[rblock] = (unsigned char)(need != 0);
  }
}

// XCD shares (Problem::shares).  The first slot s of a split row (fewer
// than kShareSplitSegs segments) keeps, at shr_pb + 8 s, the offsets
// [0 .. 6] = o_1 .. o_7 from the row start at which the parts of column
// ranges 1 .. 7 begin (o_0 = 0, o_8 = the row length; o_x counts the row's
// nonzeros whose column lies below boundary x).  Slot s holding segment k of
// a longer row keeps at [7] the range holding the column at the segment's
// middle, the XCD that sums the whole segment.  For a sorted row part x
// holds the columns of range x; for any row the parts partition its
// positions, since the boundaries (made non-decreasing) make o_x
// non-decreasing in x.

// Segment k of a long row [rs, re): its positions [start, end).
__device__ __forceinline__ void segment_range(const Problem& p, int rs, int re, int k, int& start,
                                              int& end, int& nseg) {
  const int len = re - rs;
  nseg = seg_count(p, len);
  start = rs + seg_begin(len, nseg, k);
  end = rs + seg_begin(len, nseg, k + 1);
}

// Slots per wave of share_bounds_kernel, and slots whose columns load
// together; build-time tunable.  Measured on MI355X (R-MAT N = 64), slots x
// batch: 16 x 4 37.5 us, 32 x 2 40.0, 16 x 2 30.3, 8 x 2 27.3, 4 x 2 29.9,
// 4 x 1 23.0, 2 x 1 26.7, 1 x 1 32.5: short waves, many of them.
#ifndef CSRSPMM_SHARE_BOUND_SLOTS
#define CSRSPMM_SHARE_BOUND_SLOTS 4
#endif
#ifndef CSRSPMM_SHARE_BOUND_BATCH
#define CSRSPMM_SHARE_BOUND_BATCH 1
#endif
constexpr int kShareBoundSlots = CSRSPMM_SHARE_BOUND_SLOTS;

// The share table (shr_pb) of every slot, after plan_kernel: one wave per
// kShareBoundSlots slots, balanced by nonzeros rather than rows (R-MAT's
// long rows crowd a few row blocks).  Lane t loads slot t's metadata (two
// rounds for all of them); then the slots to record, four at a time, load
// their columns in rounds of 512 positions each (a split row's, or a whole
// segment's middle one), and count them against the boundaries by ballots.
__global__ __launch_bounds__(256) void share_bounds_kernel(Problem p) {
  constexpr int S = kShareBoundSlots;
  constexpr int kB = CSRSPMM_SHARE_BOUND_BATCH;
  constexpr int kC = 8;  // chunks of 64 positions per slot and round
  static_assert(S <= 64, "one slot per lane");
  const int lane = lane_id();
  const int s0 = ((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6)) * S;
  int cb[kXcds - 1];
  share_cols(p, cb);
  // lane t < S: slot s0 + t
  int2 si = make_int2(-1, 0);
  if (lane < S && s0 + lane < p.nslots) si = p.seg_info[s0 + lane];
  if (si.x >= p.M) si.x = -1;
  // split: -1 nothing to record, 0 a segment kept whole (its middle
  // position in st), 1 the first slot of a split row (its positions
  // [st, en) are the whole row)
  int st = 0, en = 0, split = -1;
  if (si.x >= 0) {
    const int rs = clamp_nnz(p.rowptr[si.x], p.nnz);
    const int re = max(clamp_nnz(p.rowptr[si.x + 1], p.nnz), rs);
    int nseg, a, e;
    segment_range(p, rs, re, si.y, a, e, nseg);
    if (nseg < kShareSplitSegs) {
      split = si.y == 0 && nseg > 0 ? 1 : -1;
      st = rs;
      en = re;
    } else if (si.y < nseg) {
      split = 0;
      st = (a + e) >> 1;
      en = st + 1;
    }
  }
  unsigned long long todo = __ballot(split >= 0);
  while (todo) {
    int l[kB], a[kB], e[kB], sp[kB];
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      l[b] = todo ? __ffsll((long long)todo) - 1 : -1;
      if (todo) todo &= todo - 1;
      a[b] = l[b] >= 0 ? __builtin_amdgcn_readlane(st, l[b]) : 0;
      e[b] = l[b] >= 0 ? __builtin_amdgcn_readlane(en, l[b]) : 0;
      sp[b] = l[b] >= 0 ? __builtin_amdgcn_readlane(split, l[b]) : -1;
    }
    int cnt[kB][kXcds - 1];
#pragma unroll
    for (int b = 0; b < kB; ++b)
#pragma unroll
      for (int x = 0; x < kXcds - 1; ++x) cnt[b][x] = 0;
    int mx = 0;  // the longest of the batch's ranges
#pragma unroll
    for (int b = 0; b < kB; ++b) mx = max(mx, e[b] - a[b]);
    for (int off = 0; off < mx; off += kC * 64) {
      int cv[kB][kC];
#pragma unroll
      for (int b = 0; b < kB; ++b)
#pragma unroll
        for (int u = 0; u < kC; ++u) {
          const int j = a[b] + off + u * 64 + lane;
          cv[b][u] = j < e[b] ? p.colidx[j] : 0x7fffffff;
        }
#pragma unroll
      for (int b = 0; b < kB; ++b)
#pragma unroll
        for (int u = 0; u < kC; ++u)
#pragma unroll
          for (int x = 0; x < kXcds - 1; ++x) cnt[b][x] += __popcll(__ballot(cv[b][u] < cb[x]));
    }
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      if (sp[b] < 0 || lane != 0) continue;
      int* dst = reinterpret_cast<int*>(p.shr_pb) + 8LL * (s0 + l[b]);
      if (sp[b] == 0) {
        // a whole segment: the range of its middle column (one position)
        int x = 0;
#pragma unroll
        for (int i = 0; i < kXcds - 1; ++i) x += 1 - cnt[b][i];
        dst[7] = x;
      } else {
        int4* d4 = reinterpret_cast<int4*>(dst);
        d4[0] = make_int4(cnt[b][0], cnt[b][1], cnt[b][2], cnt[b][3]);
        d4[1] = make_int4(cnt[b][4], cnt[b][5], cnt[b][6], -1);
      }
    }
  }
}

// B-row gathers in flight per lane in the scalar-column share_kernel's
// pieces (at least the variant's own; float4 ones keep theirs), and the
// slots one group of it takes (one per lane, at most G); build-time tunable.
#ifndef CSRSPMM_SHARE_U
#define CSRSPMM_SHARE_U 16
#endif
#ifndef CSRSPMM_SHARE_LANES
#define CSRSPMM_SHARE_LANES 64
#endif

// The long rows of a call with XCD shares, over the columns of the slices
// [slice0, slice0 + gridDim.x / share_blocks): block b runs on XCD
// x = b mod kXcds.  Group g of XCD x's blocks (g = (b / kXcds) * GPB +
// group, ng groups in all) takes G slots, lane l slot g + l * ng, so that a
// long row's neighbouring segments (which fall in one column range) go to
// different groups.  Each lane loads its slot's metadata (three rounds for
// the group); then the group walks its slots with something to do in lane
// order, the next one's first chunk of (col, val) loaded while the current
// one is summed: at a split row's first slot, part x of the row (zero when
// empty) into its shr_part row, or, for a segment kept whole whose middle
// column lies in range x, the whole segment into its segment partial.  Launched before the
// main kernel of the same slices, which then holds no segment blocks.
template <int VEC, int G, int T, int US, bool LDS, bool BUF>
__global__ __launch_bounds__(kWaves * 64) void share_kernel(Problem p, int share_blocks, int slice0) {
  using VT = typename Vec<VEC>::T;
  constexpr int GPW = 64 / G;
  constexpr int GPB = kWaves * GPW;
  constexpr int PW = G * VEC * T;
  constexpr int UP = (VEC == 4 || US >= CSRSPMM_SHARE_U) ? US : (CSRSPMM_SHARE_U < G ? CSRSPMM_SHARE_U : G);
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gl = lane & (G - 1);
  const int gbase = lane & ~(G - 1);
  const int gid = G == 64 ? wave : wave * GPW + lane / G;
  const unsigned long long gmask = G == 64 ? ~0ULL : (((1ULL << G) - 1ULL) << gbase);
  __shared__ int2 stage_all[LDS ? kWaves * 64 : 1];
  int2* stage = stage_all + (LDS ? wave * 64 : 0);

  int bid = (int)blockIdx.x;
  int c_lo = 0, c_hi = p.N;
  if (p.sw > 0) {
    const int local = bid / share_blocks;
    bid -= local * share_blocks;
    c_lo = (slice0 + local) * p.sw;
    c_hi = min(p.N, c_lo + p.sw);
  }
  constexpr int SL = CSRSPMM_SHARE_LANES < G ? CSRSPMM_SHARE_LANES : G;  // slots per group
  const int x = (int)(blockIdx.x % kXcds);  // share_blocks is a multiple of kXcds
  const int ng = share_blocks / kXcds * GPB;
  const int s = gl < SL ? ((bid / kXcds) * GPB + gid) + gl * ng : 0x7fffffff;

  // this lane's slot: the positions [pa, pe) and the partial row (-1:
  // nothing to do; <= -2: segment partial -2 - prow)
  int pa = 0, pe = 0;
  long long prow = -1;
  int2 si = s < p.nslots ? p.seg_info[s] : make_int2(-1, 0);  // (s past nslots beyond SL lanes)
  if (si.x >= p.M) si.x = -1;
  if (si.x >= 0) {
    const int rs = clamp_nnz(p.rowptr[si.x], p.nnz);
    const int re = max(clamp_nnz(p.rowptr[si.x + 1], p.nnz), rs);
    int start, end, nseg;
    segment_range(p, rs, re, si.y, start, end, nseg);
    const int* pb = reinterpret_cast<const int*>(p.shr_pb) + 8LL * s;
    if (nseg >= kShareSplitSegs) {
      if (si.y < nseg && pb[7] == x) {
        pa = start;
        pe = end;
        prow = -2 - ((long long)(rs >> p.seg_shift) + si.y);
      }
    } else if (si.y == 0 && nseg > 0) {
      const int len = re - rs;
      const int lo = x == 0 ? 0 : min(max(pb[x - 1], 0), len);
      const int hi = x == kXcds - 1 ? len : min(max(pb[x], lo), len);
      pa = rs + lo;
      pe = rs + hi;
      prow = (long long)(rs >> kShareIdxShift) + x;
    }
  }
  unsigned long long todo = __ballot(prow != -1) & gmask;
  // the first piece's first chunk
  int l = todo ? __ffsll((long long)todo) - 1 - gbase : -1;
  int a = l >= 0 ? group_bcast<G>(pa, gbase, l) : 0;
  int e = l >= 0 ? group_bcast<G>(pe, gbase, l) : 0;
  int cj;
  float vj;
  load_chunk(p, a, e, gl, cj, vj);
  while (l >= 0) {
    todo &= todo - 1;
    const long long pr = ((long long)group_bcast<G>((int)(prow >> 32), gbase, l) << 32) |
                         (unsigned)group_bcast<G>((int)prow, gbase, l);
    // the next piece and its first chunk
    const int ln = todo ? __ffsll((long long)todo) - 1 - gbase : -1;
    const int an = ln >= 0 ? group_bcast<G>(pa, gbase, ln) : 0;
    const int en = ln >= 0 ? group_bcast<G>(pe, gbase, ln) : 0;
    int cn;
    float vn;
    load_chunk(p, an, en, gl, cn, vn);
    float* dst = pr >= 0 ? p.shr_part + pr * p.ldp : p.partials + (-2 - pr) * p.ldp;
    for (int c0 = c_lo; c0 < c_hi; c0 += PW) {
      const Panel<VEC, G, T, BUF> pn(p, c0, gl, c_hi);
      VT acc[T];
#pragma unroll
      for (int u = 0; u < T; ++u) acc[u] = Vec<VEC>::zero();
      if (c0 != c_lo) load_chunk(p, a, e, gl, cj, vj);
      stream_nonzeros_from<VEC, G, T, UP, LDS, BUF>(p, pn, a, e, cj, vj, gl, gbase, stage,
                                                    [&](int, float v, const VT(&b)[T]) {
#pragma unroll
                                                      for (int u = 0; u < T; ++u) acc[u] = fma_v(v, b[u], acc[u]);
                                                    });
#pragma unroll
      for (int u = 0; u < T; ++u) {
        if (pn.cval[u]) *reinterpret_cast<VT*>(dst + pn.col[u]) = acc[u];
      }
    }
    l = ln;
    a = an;
    e = en;
    cj = cn;
    vj = vn;
  }
}


// Table slots one wave of the combine scan reads at once.  A split row (two
// segments or more) owns two slots or more, so a wave meets at most
// kScanSlots / 2 rows to sum (with XCD shares, kScanSlots rows).
constexpr int kScanSlots = 16;

// Whether any row block of plan_kernel flagged a row for the combine (every
// wave reads the flags, 16 a load, and all reach the same answer).
__device__ __forceinline__ bool combine_needed(const Problem& p, int lane) {
  if (!need_checked(p)) return true;
  const uint4* f4 = reinterpret_cast<const uint4*>(p.need);
  bool any = false;
  for (int i = lane; i * 16 < p.need_blocks; i += 64) {
    const uint4 x = f4[i];
    const int valid = min(p.need_blocks - i * 16, 16);  // bytes past need_blocks are padding
    const unsigned w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int nb = min(max(valid - 4 * j, 0), 4);
      const unsigned m = nb >= 4 ? 0xffffffffu : (1u << (8 * nb)) - 1u;
      any |= (w[j] & m) != 0;
    }
  }
  return __ballot(any) != 0;
}

template <int VEC, int GC>
__global__ __launch_bounds__(kWaves * 64) void combine_kernel(Problem p, int scan_blocks) {
  constexpr int P = 64 / GC;
  const int lane = lane_id();
  const int q = lane / GC;
  const int gl = lane & (GC - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (!combine_needed(p, lane)) return;  // no split, shared or panelized row
  if ((int)blockIdx.x < scan_blocks) {
    const int nchunks = div_up(p.nslots, kScanSlots);
    for (int ch = blockIdx.x * kWaves + wave; ch < nchunks; ch += scan_blocks * kWaves) {
      const int s = ch * kScanSlots + lane;
      int2 si = make_int2(-1, 1);
      if (lane < kScanSlots && s < p.nslots) si = p.seg_info[s];
      int nseg = 0, x0 = 0, len = 0;
      if (si.x >= 0 && si.x < p.M && si.y == 0) {
        x0 = clamp_nnz(p.rowptr[si.x], p.nnz);
        len = max(clamp_nnz(p.rowptr[si.x + 1], p.nnz) - x0, 0);
        nseg = seg_count(p, len);
        // one segment: stored by the segment phase; panelized: summed from
        // pieces; split by XCD: summed from its parts whatever nseg
        if (!p.shares && (nseg < 2 || (len >= kPanelMinLen && is_panelized(p, x0)))) nseg = 0;
      }
      unsigned long long rows = __ballot(nseg > 0);
      if (p.shares) {
        // Rows split by XCD, P at a time: lane group q takes the q-th and
        // adds its kXcds part rows from x0 >> kShareIdxShift (zero where a
        // part is empty) in range order, all loads in flight.
        unsigned long long srows = __ballot(nseg > 0 && nseg < kShareSplitSegs);
        rows &= ~srows;
        while (srows) {
          unsigned long long m = srows;
          for (int i = 0; i < q; ++i) m &= m - 1;
          const int lq = m ? __ffsll((long long)m) - 1 : -1;
#pragma unroll
          for (int i = 0; i < P; ++i) srows &= srows - 1;
          const int src = lq >= 0 ? lq : 0;
          const int row = __shfl(si.x, src);
          const int rx0 = __shfl(x0, src);
          if (lq < 0) continue;
          const float* base = p.shr_part + (long long)(rx0 >> kShareIdxShift) * p.ldp;
          float* crow = p.C + (long long)row * p.ldc;
          for (int c0 = 0; c0 < p.N; c0 += GC * 4) {
            const int c = c0 + gl * 4;
            const bool cv = c < p.N;
            const f4 acc = sum_strided<1>(base + c, nullptr, kXcds, 0, p.ldp, cv);
            if (cv) store_cols4<VEC>(p, crow + c, c, acc);
          }
        }
      }
      while (rows) {
        const int l = __ffsll((long long)rows) - 1;
        rows &= rows - 1;
        const int row = __builtin_amdgcn_readlane(si.x, l);
        const int n = __builtin_amdgcn_readlane(nseg, l);
        // the row's partials x0 / seg .. + n - 1
        const float* base = p.partials + (long long)(__builtin_amdgcn_readlane(x0, l) >> p.seg_shift) * p.ldp;
        float* crow = p.C + (long long)row * p.ldc;
        for (int c0 = 0; c0 < p.N; c0 += GC * 4) {
          const int c = c0 + gl * 4;
          const bool cv = c < p.N;
          const f4 acc = wave_group_sum<GC>(sum_strided<P>(base + c, nullptr, n, q, p.ldp, cv));
          if (q == 0 && cv) store_cols4<VEC>(p, crow + c, c, acc);
        }
      }
    }
    return;
  }
  const int i = (int)blockIdx.x - scan_blocks;
  __shared__ f4 wave_sum[kWaves][GC];
  int row, npc;
  const int* pieces;
  const float* part;
  if (p.dp.P > 0) {
    // this call's panelized row i: partials (i, 0 .. P-1), in column order
    if (i >= p.dp.sched[0]) return;
    row = p.dp.win[p.dp.list[i]].x;
    if (row < 0 || row >= p.M) return;  // only for a malformed rowptr
    npc = p.dp.P;
    pieces = nullptr;
    part = p.dp.part + (long long)i * p.dp.P * p.ldp;
  } else {
    if (i >= p.npan) return;
    row = p.pan_rows[i];
    npc = p.pan_ptr[i + 1] - p.pan_ptr[i];
    pieces = p.pan_piece + p.pan_ptr[i];
    part = p.pan_part;
  }
  float* crow = p.C + (long long)row * p.ldc;
  for (int c0 = 0; c0 < p.N; c0 += GC * 4) {
    const int c = c0 + gl * 4;
    const bool cv = c < p.N;
    const f4 acc = wave_group_sum<GC>(
        sum_strided<kWaves * P>(part + c, pieces, npc, wave * P + q, p.ldp, cv));
    if (q == 0) wave_sum[wave][gl] = acc;
    __syncthreads();
    if (wave == 0 && q == 0 && cv) {
      f4 t = wave_sum[0][gl];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) t = add_v(t, wave_sum[w][gl]);
      store_cols4<VEC>(p, crow + c, c, t);
    }
    __syncthreads();
  }
}

// The lane groups cover ceil(N / 4) float4 column chunks.
template <int VEC>
void launch_combine(const Problem& p, hipStream_t s) {
  const int chunks = (p.N + 3) / 4;
  const int scan_blocks =
      std::min(kCombineScanBlocks, div_up_host(div_up_host(p.nslots, kScanSlots), kWaves));
  const int blocks = scan_blocks + (p.dp.P > 0 ? p.dp.nl_max : p.npan);
  if (blocks == 0) return;
  if (chunks <= 8) {
    hipLaunchKernelGGL((combine_kernel<VEC, 8>), dim3(blocks), dim3(kWaves * 64), 0, s, p, scan_blocks);
  } else if (chunks <= 16) {
    hipLaunchKernelGGL((combine_kernel<VEC, 16>), dim3(blocks), dim3(kWaves * 64), 0, s, p, scan_blocks);
  } else if (chunks <= 32) {
    hipLaunchKernelGGL((combine_kernel<VEC, 32>), dim3(blocks), dim3(kWaves * 64), 0, s, p, scan_blocks);
  } else {
    hipLaunchKernelGGL((combine_kernel<VEC, 64>), dim3(blocks), dim3(kWaves * 64), 0, s, p, scan_blocks);
  }
}

// SU: B-row gathers in flight per lane in the long-row segments (at least U).
// BUF: B gathered through a buffer resource (buf_gathers_ok must hold).
// SWEEP: the short rows of each slice in a band sweep (p.sweep_bands > 0).
// p.seg_fuse launches the FUSE instance of the kernel without pieces.
template <int VEC, int G, int T, int U, bool LDS, int SU = CSRSPMM_SEG_UNROLL, bool BUF = false,
          bool SWEEP = false>
hipError_t launch_rg(const Problem& p, hipStream_t s) {
  constexpr int GPB = kWaves * (64 / G);
  const int units = SWEEP ? div_up_host(p.M, kSweepRows) : p.plan ? p.nblocks : p.M;
  const int unit_blocks = div_up_host(units, GPB);
  // With XCD shares the segments run in share_kernel, launched before each
  // main launch over the same slices, and the main launch has no segment
  // blocks.
  const bool shares = p.plan && p.nslots > 0 && p.shares;
  const int seg_blocks =
      (p.plan && p.nslots > 0 && !shares) ? std::min(kSegBlocksMax, div_up_host(p.nslots, GPB)) : 0;
  const int share_blocks =
      shares ? kXcds * div_up_host(div_up_host(p.nslots, std::min(G, CSRSPMM_SHARE_LANES)), GPB) : 0;
  constexpr int US = SU > U ? (SU < G ? SU : G) : U;
  int piece_blocks = 0;
  // Column panels reach the float4 kernels and the scalar ones of N > 64
  // (per_call_panels, from N = 128).
  constexpr bool kCanPanel = VEC == 4 || T >= 2;
  // the segments would skip rows that no piece sums
  if (!kCanPanel && p.dp.P > 0) return hipErrorInvalidValue;
  if (kCanPanel && p.dp.P > 0) {
    // chunks of the longest XCD list possible: ceil(P / kXcds) panels x nl_max rows
    const long long per_xcd = (long long)div_up_host(p.dp.P, kXcds) * p.dp.nl_max;
    const long long chunks = (per_xcd + (long long)kPiecesPerGroup * GPB - 1) / ((long long)kPiecesPerGroup * GPB);
    if (chunks * kXcds > 0x7fffffffLL / 2) return hipErrorInvalidValue;
    piece_blocks = (int)(chunks * kXcds);
  }
  const int slice_blocks = unit_blocks + seg_blocks;
  const int nslices = p.sw > 0 ? div_up_host(p.N, p.sw) : 1;
  // Slices in one launch (their blocks in slice order) or one launch per slice.
  const int per_launch = (p.sw > 0 && p.slice_launch) ? 1 : nslices;
  // Unused LDS that leaves room for only `cap` blocks per CU (a multiple of
  // 512 bytes, the allocation unit, per block with the static stage).
  const int cap = SWEEP ? 0 : slice_blocks_per_cu(p.K, p.sw, p.slice_launch);
  constexpr int kStaticLds = (LDS ? kWaves * 64 : 1) * (int)sizeof(int2);
  const int pad_lds = cap > 0 ? (kLdsPerCu / cap) / 512 * 512 - kStaticLds : 0;
  for (int s0 = 0; s0 < nslices; s0 += per_launch) {
    if (share_blocks > 0) {
      const long long sblocks = (long long)per_launch * share_blocks;
      if (sblocks > 0x7fffffffLL) return hipErrorInvalidValue;
      hipLaunchKernelGGL((share_kernel<VEC, G, T, US, LDS, BUF>), dim3((unsigned)sblocks), dim3(kWaves * 64), 0,
                         s, p, share_blocks, s0);
    }
    const long long blocks = (long long)piece_blocks + (long long)per_launch * slice_blocks;
    if (blocks == 0) continue;
    if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
    if (piece_blocks > 0) {
      hipLaunchKernelGGL((rowgroup_kernel<VEC, G, T, U, LDS, kCanPanel, SU, BUF, false>), dim3((unsigned)blocks),
                         dim3(kWaves * 64), pad_lds, s, p, piece_blocks, seg_blocks, slice_blocks,
                         s0);
    } else if (p.seg_fuse) {
      hipLaunchKernelGGL((rowgroup_kernel<VEC, G, T, U, LDS, false, SU, BUF, SWEEP, true>), dim3((unsigned)blocks),
                         dim3(kWaves * 64), pad_lds, s, p, 0, seg_blocks, slice_blocks, s0);
    } else {
      hipLaunchKernelGGL((rowgroup_kernel<VEC, G, T, U, LDS, false, SU, BUF, SWEEP>), dim3((unsigned)blocks),
                         dim3(kWaves * 64), pad_lds, s, p, 0, seg_blocks, slice_blocks, s0);
    }
  }
  return hipGetLastError();
}

}  // namespace

static inline int pow2_ceil(int x) {
  int v = 1;
  while (v < x) v <<= 1;
  return v;
}

// Unsliced float4 calls: the group width from N.
// Unsliced float4 calls of up to 128 columns sweep too when B exceeds
// CSRSPMM_SWEEP_UNSLICED_MB and the max_row_nnz hint rules out skewed rows
// (longest row at most long_row or 4x the mean).  Measured on MI355X per
// call, bit-identical: uniform rows with the hint, 32768^2 x 128 with 40 per
// row 77.1 -> 48.8 us, 65536^2 x 64 with 32 per row 67.0 -> 49.1 us,
// 16384^2 x 128 with 20 per row 24.0 -> 21.7 us, medium (82 per row, 8 MiB)
// 49.5 -> 50.8 us; power-law rows (mean 32, the hint excludes them) lost
// 8-19% swept.
#ifndef CSRSPMM_SWEEP_UNSLICED_MB
#define CSRSPMM_SWEEP_UNSLICED_MB 4
#endif
template <bool LDS, bool BUF>
static hipError_t dispatch_vec4_cols(const Problem& p, hipStream_t s) {
  constexpr int SU = CSRSPMM_SEG_UNROLL;
  const int nv = (p.sw > 0 ? std::min(p.sw, p.N) : p.N) / 4;
  const int G = nv >= 64 ? 64 : (pow2_ceil(nv) < 4 ? 4 : pow2_ceil(nv));
  if constexpr (BUF) {
    const long long mean4 = p.M > 0 ? 4LL * p.nnz / p.M : 0;
    if ((G == 16 || G == 32) && p.dp.P == 0 && p.row_hint >= 0 &&
        p.row_hint <= std::max<long long>(p.long_row, mean4) &&
        (long long)p.K * p.N * 4 > ((long long)CSRSPMM_SWEEP_UNSLICED_MB << 20) &&
        sweep_applies(p.plan, p.M, p.K, p.nnz, G * 4)) {
      Problem q = p;
      sweep_geometry(p.K, G * 4, q.sweep_shift, q.sweep_bands);
      if (q.sweep_bands >= 2) {
        if (G == 16) return launch_rg<4, 16, 1, kVec4U, LDS, CSRSPMM_SWEEP_SU, true, true>(q, s);
        return launch_rg<4, 32, 1, kVec4U, LDS, CSRSPMM_SWEEP_SU, true, true>(q, s);
      }
    }
  }
  if (G < 64) {
    switch (G) {
      case 4: return launch_rg<4, 4, 1, kVec4U, LDS, SU, BUF>(p, s);
      case 8: return launch_rg<4, 8, 1, kVec4U, LDS, SU, BUF>(p, s);
      case 16: return launch_rg<4, 16, 1, kVec4U, LDS, SU, BUF>(p, s);
      default: return launch_rg<4, 32, 1, kVec4U, LDS, SU, BUF>(p, s);
    }
  }
  const int t = (nv + 63) / 64;
  if (t <= 1) return launch_rg<4, 64, 1, kVec4U, LDS, SU, BUF>(p, s);
  // Beyond 512 columns a planned call loops over 512-column panels; one
  // with rows summed whole (no plan) takes 1024 columns a pass, since each
  // pass walks a row's chain again.  Measured on MI355X per call,
  // bit-identical, 512 against 1024 columns a pass: 4096^2 x 1024 with 300
  // per row 392 -> 287 us, 128 per row 154 -> 138, 8192 x 2048 x 2048 with
  // 64 per row 269 -> 232 (213 -> 188 with the hint); rows summed whole,
  // 2048 x 4096 x 1024 with 200 per row 61.0 against 64.1 us.
  if (t <= 2 || p.plan) return launch_rg<4, 64, 2, 4, LDS, SU, BUF>(p, s);
  return launch_rg<4, 64, 4, 2, LDS, SU, BUF>(p, s);  // N > 1024 loops over 1024-column panels
}

// B can be gathered through a buffer resource: every row and row length fits
// 24 bits (one v_mad_u32_u24 per offset), B's extent stays below
// kBufOffPast, and either it stays within 1 GiB or no lane of any group owns
// a column past the block's columns (a power of two of at least 4 vec
// columns per block, which the column slices divide): a masked lane's
// offset, row offset + kBufOffPast, then cannot wrap into the buffer.
static bool buf_gathers_ok(const Problem& p, int vec) {
  if (p.K <= 0 || p.K >= (1 << 24) || p.ldb * 4 >= (1LL << 24)) return false;
  const long long bytes = (long long)(p.K - 1) * p.ldb * 4 + (long long)p.N * 4;
  if (bytes >= (long long)kBufOffPast) return false;
  if (bytes <= (1LL << 30)) return true;
  const int cols = p.sw > 0 ? p.sw : p.N;
  return (cols & (cols - 1)) == 0 && cols >= 4 * vec && (p.sw == 0 || p.N % p.sw == 0);
}

// The kernel shape comes from the columns one block covers: a column slice,
// or all N.
//
// Float4 calls gather B through a buffer resource when it fits
// (buf_gathers_ok).  Measured on MI355X against 64-bit global loads, with
// bit-identical results: XL 393.6 -> 376.3 us per call (VALU instructions
// 133 M -> 59 M, L2 hit rate 0.50 -> 0.56, fetched bytes -12%), the
// mean-98 power-law config 1085 -> 1071 us, medium 48.5 -> 45.1 us.  On
// column slices (those the band sweep does not take): power-law rows (mean
// 32) at 32768^2 x 256 290 -> 199 us, uniform rows 4096 x 65536 x 256 with
// 32 per row 41.7 -> 35.8, 8192 x 65536 x 1024 with 50 per row 257 -> 238,
// 32768^2 x 256 with 24 per row 84.1 -> 80.1; R-MAT N = 256 and 512 -1% and
// -0.3%; 131072^2 and power-law rows at K = 65536-131072 within 0.3%.  (The
// uniform 65536 x 256 config, sliced without the sweep, had gone 381 -> 423
// us with it, its L2 hit rate falling 0.48 -> 0.39; it sweeps now.)
template <bool LDS>
static hipError_t dispatch_vec4(const Problem& p, hipStream_t s) {
  // A column slice (64 columns: 16-lane groups) keeps 8 gathers in flight per
  // lane in its segments, twice the unsliced kernels'.  Measured on MI355X,
  // power-law rows (mean 32, rows up to 16k) at N = 256: K = 32768 341 ->
  // 276 us, K = 65536 325 -> 304; the 66-per-row uniform and R-MAT N = 512
  // configs within 1%.  Unsliced 16-lane calls keep 4 (XL at N = 64 lost 7%).
  static_assert(kSliceWidth == 64, "a slice's float4 chunks fill 16-lane groups");
  if (p.sw == kSliceWidth) {
    // The short rows of each slice are swept band by band (sweep_rows); the
    // LDS-staged variant passes each chunk through its stage.
    // (XCD slices keep each band in one XCD's L2 without it.)
    if (!p.xslice && sweep_applies(p.plan, p.M, p.K, p.nnz, p.sw) && buf_gathers_ok(p, 4)) {
      Problem q = p;
      sweep_geometry(p.K, p.sw, q.sweep_shift, q.sweep_bands);
      return launch_rg<4, 16, 1, kVec4U, LDS, CSRSPMM_SWEEP_SU, true, true>(q, s);
    }
    if (buf_gathers_ok(p, 4)) return launch_rg<4, 16, 1, kVec4U, LDS, 8, true>(p, s);
    return launch_rg<4, 16, 1, kVec4U, LDS, 8>(p, s);
  }
  if (buf_gathers_ok(p, 4)) return dispatch_vec4_cols<LDS, true>(p, s);
  return dispatch_vec4_cols<LDS, false>(p, s);
}

template <bool LDS, bool BUF>
static hipError_t dispatch_vec1_cols(const Problem& p, hipStream_t s) {
  constexpr int SU = CSRSPMM_SEG_UNROLL;
  const int n = p.sw > 0 ? std::min(p.sw, p.N) : p.N;
  const int G = n >= 64 ? 64 : (pow2_ceil(n) < 4 ? 4 : pow2_ceil(n));
  if (G < 64) {
    switch (G) {
      case 4: return launch_rg<1, 4, 1, 8, LDS, SU, BUF>(p, s);
      case 8: return launch_rg<1, 8, 1, 8, LDS, SU, BUF>(p, s);
      case 16: return launch_rg<1, 16, 1, 8, LDS, SU, BUF>(p, s);
      default: return launch_rg<1, 32, 1, 8, LDS, SU, BUF>(p, s);
    }
  }
  const int t = (n + 63) / 64;
  if (t <= 1) return launch_rg<1, 64, 1, 8, LDS, SU, BUF>(p, s);
  if (t <= 2) return launch_rg<1, 64, 2, 8, LDS, SU, BUF>(p, s);
  if (t <= 4) return launch_rg<1, 64, 4, 8, LDS, SU, BUF>(p, s);
  return launch_rg<1, 64, 8, 4, LDS, SU, BUF>(p, s);  // N > 512 loops over 512-column panels
}

// Scalar-column calls gather B through a buffer resource when it fits
// (buf_gathers_ok), sliced or not.  Measured on MI355X against 64-bit global
// loads, per call, bit-identical: XL WarpPerRow 510 -> 394 us and
// WarpPerRowSmem 416 -> 357; medium WarpPerRow 84 -> 59 and WarpPerRowSmem
// 67 -> 59; R-MAT N = 32 (Auto) 388 -> 307; sliced, large WarpPerRow 690 ->
// 535 and WarpPerRowSmem 575 -> 525, R-MAT N = 512 WarpPerRow 5122 -> 4753;
// R-MAT N = 64 (Auto) within 0.6%.
template <bool LDS>
static hipError_t dispatch_vec1(const Problem& p, hipStream_t s) {
  if (buf_gathers_ok(p, 1)) return dispatch_vec1_cols<LDS, true>(p, s);
  return dispatch_vec1_cols<LDS, false>(p, s);
}

// plan_kernel's grid: blocks of 256 rows (grid-strided beyond 4096), and
// with XCD shares one more block for their column boundaries.
static int plan_blocks(const Problem& p) {
  return plan_row_blocks(p.M) + (p.shares ? 1 : 0);
}

hipError_t launch_share_bounds(const Problem& p, hipStream_t s) {
  const int waves = div_up_host(p.nslots, kShareBoundSlots);
  if (waves <= 0) return hipSuccess;
  hipLaunchKernelGGL(share_bounds_kernel, dim3(div_up_host(waves, 4)), dim3(256), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_plan_tables(const Problem& p, hipStream_t s) {
  hipLaunchKernelGGL(plan_kernel, dim3(plan_blocks(p)), dim3(256), 0, s, p);
  if (p.dp.P > 0) return launch_panel_schedule(p, s);
  if (p.plan && p.nslots > 0 && p.shares) return launch_share_bounds(p, s);
  return hipGetLastError();
}

static hipError_t dispatch_main(const Problem& p, int vec, bool lds, hipStream_t s) {
  if (vec == 4) return lds ? dispatch_vec4<true>(p, s) : dispatch_vec4<false>(p, s);
  return lds ? dispatch_vec1<true>(p, s) : dispatch_vec1<false>(p, s);
}

static hipError_t launch_rowgroup_all(const Problem& p_in, int vec, bool lds, hipStream_t s) {
  // A per-call plan without column panels, XCD shares or stored panels sums
  // its split rows in the main launch (Problem::seg_fuse), when every slot
  // has a group of its own (the segment blocks, at least kWaves slots each,
  // are not capped); a stored plan has no per-call plan_kernel to zero the
  // counters, and keeps the combine.  Measured on MI355X per call (rocprof
  // sums, bit-identical to the combine): medium 49.4 -> 44.6 us (the combine
  // launch, which found no split row, gone), large 300.4 -> 300.0 us; XL
  // without its column panels (thousands of split rows) 645 -> 654 us.  The
  // rows' sums one lane group at a time, with a load in flight, had cost
  // that call 58 us.
  Problem p = p_in;
  p.seg_fuse = CSRSPMM_SEG_FUSE && p.plan && !p.plan_ready && p.nslots > 0 && !p.no_split && !p.shares &&
               p.npan == 0 && p.dp.P == 0 && p.seg_cnt != nullptr &&
               (long long)p.nslots <= (long long)kSegBlocksMax * kWaves &&
               (long long)(p.nnz >> p.seg_shift) * p.ldp * 4 < (1LL << 31);
  if (p.plan && !p.plan_ready) hipLaunchKernelGGL(plan_kernel, dim3(plan_blocks(p)), dim3(256), 0, s, p);
  hipError_t e;
  if (p.dp.P > 0 && !p.dp_ready) {
    e = launch_panel_schedule(p, s);
    if (e != hipSuccess) return e;
  }
  const bool shares = p.plan && p.nslots > 0 && p.shares;
  if (shares && !p.dp_ready) {
    e = launch_share_bounds(p, s);
    if (e != hipSuccess) return e;
  }
  e = dispatch_main(p, vec, lds, s);
  if (e != hipSuccess) return e;
  if (p.plan && !p.seg_fuse && ((p.nslots > 0 && !p.no_split) || shares || p.npan > 0 || p.dp.P > 0)) {
    if (vec == 4) {
      launch_combine<4>(p, s);
    } else {
      launch_combine<1>(p, s);
    }
    e = hipGetLastError();
  }
  return e;
}

hipError_t launch_rowgroup(const Problem& p, int vec, bool lds, hipStream_t s) {
  if (p.M == 0 || p.N == 0) return hipSuccess;
  timing_before_main(s);
  const hipError_t e = launch_rowgroup_all(p, vec, lds, s);
  timing_after_main(s);
  return e;
}

}  // namespace csrspmm_hip
