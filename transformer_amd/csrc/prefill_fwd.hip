// Causal flash-attention forward over the decoupled-RoPE MLA heads (gfx950).
//
// Computes, per (batch b, head h):
//   S = (q_nope k_nope^T + q_rope k_rope^T) * scale,  S[i][j] = -inf if causal and
//   j > i + q_offset;  O = softmax(S) V;  LSE = log(sum_j exp S[i][j]).
// This is F.scaled_dot_product_attention(cat[q_nope,q_rope], cat[k_nope,k_rope], v,
// is_causal=True) at transformer.py:311-314 (q_offset = 0), and the absorbed branch's
// bottom-right mask triu(diagonal = pos_offset + 1) at transformer.py:273-281.
//
// Work decomposition: one workgroup = NW waves (NW = 4) = a q-tile of 32 NW query rows of
// one (b, h), two such workgroups per CU; each wave owns 32 query rows and keeps its Q
// fragment in registers.  A workgroup runs two mirrored q-tiles of its (b, h) (equal causal
// work for every workgroup).  The key loop walks 32-key tiles that buffer loads write
// straight into LDS (no staging registers): a ring of four stages, each tile's loads issued
// three steps ahead, one barrier per tile.  Each step overlaps the score MFMAs of the next
// tile with the softmax of the current one.
//
// Per 32-key tile and wave:
//   S^T (32 x 32)  = K (32 x DQK) . Q^T (DQK x 32)     DQK/16 MFMA 32x32x16
//   O^T (128 x 32) += V^T (128 x 32) . P^T (32 x 32)   4 x 2  MFMA 32x32x16
// Computing S^T rather than S puts one query row per lane (column of the MFMA
// output), so the running max / sum / rescale of the online softmax are per-lane
// scalars; the row max needs one cross-lane exchange (lanes l and l ^ 32).
// P^T goes straight from the S^T accumulators into the PV MFMA's B operand; V^T comes
// from row-major V through ds_read_b64_tr_b16.
#include <type_traits>

#include "mla_common.h"

namespace mla {

struct FwdParams {
  const bf16 *qn, *qr, *kn, *kr, *v;
  bf16* o;
  float* lse;
  int B, H, Tq, Tk, n_qt;
  mla_strides qn_s, qr_s, kn_s, kr_s, v_s, o_s;
  float scale_log2;  // scale * log2(e)
  int causal;
  int64_t q_offset;
  // key split (small grids): each pair of q-tiles is cut into S segments of its key tiles; a
  // q-tile whose keys span several segments leaves one partial per segment (O normalised
  // within the segment, fp32, and its log2 LSE) in ws_o / ws_lse for fwd_merge_kernel
  int S;
  float* ws_o;
  float* ws_lse;
  // RoPE folded into the Q load (rope_cos non-null): q_rope holds the unrotated rope slice and
  // query row t is rotated at position q_pos_offset + t by the bf16 tables; the rotated slice is
  // also stored to qr_out when that is non-null (for the backward)
  const bf16 *rope_cos, *rope_sin;
  int64_t q_pos_offset;
  bf16* qr_out;
  mla_strides qro_s;
};

// LDS tiles, rows unpadded (a direct-to-LDS load writes 64 lanes x 16 bytes contiguously),
// chunks XOR-swizzled per row.  A stage holds one 32-key tile: K_nope [32][DN] (DN = 128:
// 256-byte rows; DN = 64: 128-byte rows), K_rope [32][64] (128-byte rows), then V [32][128]
// (256-byte rows).  Four stages form a ring.
template <int DN>
struct FwdCfg {
  static constexpr int DR = 64, DV = 128, DQK = DN + DR;
#ifndef FWD_NW
#define FWD_NW 4
#endif
  static constexpr int NW = FWD_NW;            // waves per workgroup, 32 query rows each
  static constexpr int BM = 32 * NW, BN = 32;  // query rows per workgroup, keys per tile
  static constexpr int KS = DQK / 16;   // MFMA k-steps of S^T
  static constexpr int KNS = DN / 16;   // of which over the nope dims
  static constexpr int KN_RB = DN * 2;  // K_nope row bytes
  static constexpr int OFF_KR = BN * KN_RB;
  static constexpr int K_STAGE = OFF_KR + BN * 128;
  static constexpr int V_STAGE = BN * 256;
  static constexpr int STAGE = K_STAGE + V_STAGE;  // K tile, then V tile
  // tile t sits in stage t % 4; its loads are issued AHEAD steps before it is consumed
  static constexpr int NSTAGE = 4, AHEAD = NSTAGE - 1;
  // 1 KiB direct-to-LDS loads per tile and region (wave w issues loads w, w + NW, ...)
  static constexpr int T_KN = BN * KN_RB / 1024, T_KR = BN * 128 / 1024, T_V = BN * 256 / 1024;
  static_assert(NW % 4 == 0, "the K_nope load swizzle assumes NW % 4 == 0");
};

// Chunk swizzles (a row's 16-byte chunk c sits at position c ^ f(row)):
//  - 256-byte rows read by rows (K_nope, DN = 128): f = row mod 16, so the 16 rows that one
//    16-lane group reads at one chunk fall on 16 distinct 16-byte bank groups;
//  - 128-byte rows read by rows (K_rope, K_nope for DN = 64): f = (row ^ row / 8) mod 8,
//    distinct over any 8 consecutive rows and, paired with row parity, over 16;
//  - V (256-byte rows, transpose reads of 4 rows x 4 chunks per 32 lanes): f = 4 (row mod 4).
__device__ __forceinline__ int swz256(int r) { return r & 15; }
__device__ __forceinline__ int swz128(int r) { return (r ^ (r >> 3)) & 7; }
__device__ __forceinline__ int swzv(int r) { return 4 * (r & 3); }

// growth of a row's running max (log2 units) that triggers a rescale of O (safe form)
constexpr float kFwdRescale = 8.0f;
// a row sum beyond this (or not finite) under the fixed reference max sends the q-tile to
// the safe form; p <= 2^127 per key keeps every finite sum of the fast form exact up to it
constexpr float kFwdSumLimit = 0x1p120f;

// Maps the linear workgroup id to (b, h) and its pair of q-tiles.  A workgroup runs q-tiles
// n_qt - 1 - r and r of one (b, h) back to back: with causal masking the pair always
// totals the same number of key tiles (balanced workgroups, no tail of short tiles) and
// the second tile's first K/V tiles are loaded while the first one's output is stored.
// Workgroups are dispatched round-robin over the 8 XCDs (id % 8); renumbering so each XCD receives a contiguous range keeps the K/V of a (b, h) in that
// XCD's L2.
__device__ __forceinline__ void fwd_tile_coords(const FwdParams& p, int& b, int& h, int& qa, int& qb_, int& n_items) {
  const int n = gridDim.x;
  int id = blockIdx.x;
  if ((n & 7) == 0) id = (id & 7) * (n >> 3) + (id >> 3);
  const int n_pairs = (p.n_qt + 1) >> 1;
  const int bh = id / n_pairs;
  const int r = id - bh * n_pairs;
  qa = p.n_qt - 1 - r;  // the longer tile first
  qb_ = r;
  n_items = qa == qb_ ? 1 : 2;
  b = bh / p.H;
  h = bh - b * p.H;
}

// Key tiles (32 keys) that q-tile qt of BM rows sees: all of Tk, or up to its last row's causal
// limit (qt + 1) BM - 1 + q_offset.
__host__ __device__ __forceinline__ int fwd_qtile_tiles(int qt, int BM, int Tk, int causal, int64_t q_offset) {
  int64_t kv_end = Tk;
  if (causal) {
    const int64_t lim = (int64_t)qt * BM + BM + q_offset;
    if (lim < kv_end) kv_end = lim;
  }
  return (int)((kv_end + 31) / 32);
}

// The key split of a pair of q-tiles (qa = n_qt - 1 - r, qb = r): their key tiles, qa's then
// qb's, N = n_a + n_b in all, cut into S segments [c_s, c_{s+1}), c_s = floor(s N / S).
// Segment s holds tiles of qa if c_s < n_a and tiles of qb if c_{s+1} > n_a.  A q-tile's
// partials are the segments that hold its tiles: qa's are slots 0 .. parts_a - 1,
// parts_a = ceil(n_a S / N); qb's are slots S - parts_b .. S - 1, parts_b = S + 1 -
// ceil((n_a + 1) S / N).
struct FwdSplit {
  int qa, qb, n_a, n_b, N;
};
__host__ __device__ __forceinline__ FwdSplit fwd_split_of_pair(int r, int n_qt, int BM, int Tk, int causal,
                                                                int64_t q_offset) {
  FwdSplit f;
  f.qa = n_qt - 1 - r;
  f.qb = r;
  f.n_a = fwd_qtile_tiles(f.qa, BM, Tk, causal, q_offset);
  f.n_b = f.qa == f.qb ? 0 : fwd_qtile_tiles(f.qb, BM, Tk, causal, q_offset);
  f.N = f.n_a + f.n_b;
  return f;
}
__host__ __device__ __forceinline__ int fwd_seg_start(int s, int N, int S) { return (int)((int64_t)s * N / S); }
// partials of q-tile qt (a member of its pair) and the first slot they use
__host__ __device__ __forceinline__ void fwd_qtile_parts(int qt, int n_qt, int BM, int Tk, int causal, int64_t q_offset,
                                                          int S, int& parts, int& first) {
  const int r = qt < n_qt - 1 - qt ? qt : n_qt - 1 - qt;
  const FwdSplit f = fwd_split_of_pair(r, n_qt, BM, Tk, causal, q_offset);
  if (qt == f.qa) {
    parts = (int)(((int64_t)f.n_a * S + f.N - 1) / f.N);
    first = 0;
  } else {
    parts = S + 1 - (int)(((int64_t)(f.n_a + 1) * S + f.N - 1) / f.N);
    first = S - parts;
  }
}

// instruction classes of __builtin_amdgcn_sched_group_barrier
constexpr int kSgValu = 0x002, kSgMfma = 0x008, kSgDsRead = 0x100;
#ifndef S_AHEAD
#define S_AHEAD 3  // S^T A fragments in flight ahead of their MFMA
#endif
#ifndef PV_AHEAD
#define PV_AHEAD 2  // V^T fragments (two transpose reads each) in flight ahead of their MFMA
#endif

template <int DN, int QB, bool PT, bool SP>
__global__ __launch_bounds__(64 * FWD_NW, QB == 1 ? 2 : 1) void prefill_fwd_kernel(FwdParams p) {
  using C = FwdCfg<DN>;
  constexpr int BM = 32 * QB * C::NW;  // query rows per q-tile: QB blocks of 32 per wave
  // separate objects, so the compiler sees that reads of one stage do not wait for loads
  // into another
  __shared__ __attribute__((aligned(1024))) unsigned char stage0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char stage1[C::STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char stage2[C::STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char stage3[C::STAGE];
  auto stage = [&](auto s_tag) -> unsigned char* {
    constexpr int S = decltype(s_tag)::value % C::NSTAGE;
    return S == 0 ? stage0 : S == 1 ? stage1 : S == 2 ? stage2 : stage3;
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;

  // the workgroup's items: q-tile it_qt[i], key tiles [it_lo[i], it_hi[i]), it_parts[i] partials
  // of that q-tile (1: no split, the item writes O)
  int b, h, n_items, seg = 0;
  int it_qt[2], it_lo[2] = {0, 0}, it_hi[2], it_parts[2] = {1, 1};
  if constexpr (!SP) {
    fwd_tile_coords(p, b, h, it_qt[0], it_qt[1], n_items);  // p.n_qt counts BM-row q-tiles
    it_hi[0] = fwd_qtile_tiles(it_qt[0], BM, p.Tk, p.causal, p.q_offset);
    it_hi[1] = fwd_qtile_tiles(it_qt[1], BM, p.Tk, p.causal, p.q_offset);
  } else {
    // consecutive ids are the segments of one pair: with the XCD renumbering they share an XCD
    const int n = gridDim.x;
    int id = blockIdx.x;
    if ((n & 7) == 0) id = (id & 7) * (n >> 3) + (id >> 3);
    const int n_pairs = (p.n_qt + 1) >> 1;
    const int pid = id / p.S;
    seg = id - pid * p.S;
    const int bh = pid / n_pairs;
    const int r = pid - bh * n_pairs;
    b = bh / p.H;
    h = bh - b * p.H;
    const FwdSplit f = fwd_split_of_pair(r, p.n_qt, BM, p.Tk, p.causal, p.q_offset);
    const int c0 = fwd_seg_start(seg, f.N, p.S), c1 = fwd_seg_start(seg + 1, f.N, p.S);
    // item A: tiles of qa in the segment (if any); item B: tiles of qb (if any)
    const bool has_a = c0 < f.n_a, has_b = f.n_b > 0 && c1 > f.n_a;
    int parts_a, first_a, parts_b, first_b;
    fwd_qtile_parts(f.qa, p.n_qt, BM, p.Tk, p.causal, p.q_offset, p.S, parts_a, first_a);
    fwd_qtile_parts(f.qb, p.n_qt, BM, p.Tk, p.causal, p.q_offset, p.S, parts_b, first_b);
    const int lo_b = max(c0, f.n_a) - f.n_a, hi_b = c1 - f.n_a;
    it_qt[0] = has_a ? f.qa : f.qb;
    it_lo[0] = has_a ? c0 : lo_b;
    it_hi[0] = has_a ? min(c1, f.n_a) : hi_b;
    it_parts[0] = has_a ? parts_a : parts_b;
    it_qt[1] = f.qb;
    it_lo[1] = lo_b;
    it_hi[1] = hi_b;
    it_parts[1] = parts_b;
    n_items = has_a && has_b ? 2 : 1;
  }
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  __builtin_assume(w >= 0 && w < C::NW);
  const int l32 = lane & 31;
  const int g = lane >> 5;
  const int q_off = (int)p.q_offset;  // the host keeps q_offset < 2^30
  const bf16* kn_b = p.kn + (int64_t)b * p.kn_s.b + (int64_t)h * p.kn_s.h;
  const bf16* kr_b = p.kr + (int64_t)b * p.kr_s.b + (int64_t)h * p.kr_s.h;
  const bf16* v_b = p.v + (int64_t)b * p.v_s.b + (int64_t)h * p.v_s.h;
  // key row strides (elements; the host keeps them below 2^24)
  const int kn_st = (int)p.kn_s.t, kr_st = (int)p.kr_s.t, v_st = (int)p.v_s.t;

  // Rows past the descriptor's range are never loaded.  Their scores are masked by a select,
  // whatever the stage holds, but their V rows meet p = 0 in the P V product and must be finite:
  // when a tile can end inside its 32 rows, the V parts of the stages are zeroed once (rows that
  // earlier tiles left in a stage are finite data).  Whole-range descriptors end at Tk only; per-tile
  // descriptors also end at a q-tile's last visible key, which a causal q_offset that is not a
  // multiple of 32 puts inside a tile.
  if (p.Tk % C::BN != 0 || (PT && p.causal && p.q_offset % C::BN != 0)) {
    const u32x4 z{0u, 0u, 0u, 0u};
    for (int i = tid; i < C::V_STAGE / 16; i += 64 * C::NW) {
      sts16(stage0 + C::K_STAGE + 16 * i, z);
      sts16(stage1 + C::K_STAGE + 16 * i, z);
      sts16(stage2 + C::K_STAGE + 16 * i, z);
      sts16(stage3 + C::K_STAGE + 16 * i, z);
    }
  }

  // The wave's loads of one K and V tile, n = 0 .. NL - 1: K_nope loads first, then K_rope,
  // then V; load n of a region is that region's 1 KiB load I = w + NW k.  Load I covers
  // rows RPI I .. RPI I + RPI - 1 (RPI = 1024 / row bytes); lane l writes LDS position
  // l % (row chunks) of row RPI I + l / (row chunks), which holds logical chunk
  // position ^ f(row).  Each load has a loop-invariant per-lane byte offset relative to the
  // tile's first key.
  constexpr int MK_KN = (C::T_KN + C::NW - 1) / C::NW, MK_KR = (C::T_KR + C::NW - 1) / C::NW,
                MK_V = (C::T_V + C::NW - 1) / C::NW;
  constexpr int NL = MK_KN + MK_KR + MK_V;
  static_assert(NL <= 6, "six load offsets are kept");
  auto load_voff = [&](int n) -> uint32_t {
    if (n < MK_KN) {
      const int I = w + C::NW * n;
      if (DN == 128) {
        const int r = 4 * I + (lane >> 4);
        return (uint32_t)(r * kn_st * 2 + ((lane & 15) ^ swz256(r)) * 16);
      }
      const int r = 8 * I + (lane >> 3);
      return (uint32_t)(r * kn_st * 2 + ((lane & 7) ^ swz128(r)) * 16);
    }
    if (n < MK_KN + MK_KR) {
      const int r = 8 * (w + C::NW * (n - MK_KN)) + (lane >> 3);
      return (uint32_t)(r * kr_st * 2 + ((lane & 7) ^ swz128(r)) * 16);
    }
    const int r = 4 * (w + C::NW * (n - MK_KN - MK_KR)) + (lane >> 4);
    return (uint32_t)(r * v_st * 2 + ((lane & 15) ^ swzv(r)) * 16);
  };
  const uint32_t vl0 = load_voff(0), vl1 = NL > 1 ? load_voff(1) : 0u, vl2 = NL > 2 ? load_voff(2) : 0u,
                 vl3 = NL > 3 ? load_voff(3) : 0u, vl4 = NL > 4 ? load_voff(4) : 0u,
                 vl5 = NL > 5 ? load_voff(5) : 0u;
  // The loads of the K and V tile at kv0 into a stage: the same number per wave for every
  // tile (a tile past the end of the q-tile's keys, tk = 0, loads nothing but keeps the
  // count).  One descriptor per operand, based at the tile's first key and ending at the
  // last valid one (tk): lanes past it load nothing.  issue(n) issues the wave's load n
  // (n is a constant after unrolling), so that callers can spread them between MFMAs.
  // LDS destination of the wave's loads into each stage: the stage plus 1 KiB per wave (load
  // I = w + NW k of a region lands at region + 1 KiB I)
  const uint32_t wl = 1024u * (uint32_t)w;
  const uint32_t lb0 = lds_addr(stage0) + wl, lb1 = lds_addr(stage1) + wl, lb2 = lds_addr(stage2) + wl,
                 lb3 = lds_addr(stage3) + wl;
  auto stage_lds = [&](auto s_tag) -> uint32_t {
    constexpr int S = decltype(s_tag)::value % C::NSTAGE;
    return S == 0 ? lb0 : S == 1 ? lb1 : S == 2 ? lb2 : lb3;
  };
  struct TileLoads {
    buf_rsrc rkn, rkr, rv;
    uint32_t lb;
    uint32_t okn, okr, ov;  // byte offset of the tile's first key row in each operand
  };
  // Whole-range descriptors (PT = false): one per operand for the workgroup's (b, h), rows
  // [0, Tk), built once; a tile adds its first row's byte offset to the per-lane offsets, and a
  // tile that loads nothing gets an offset past the range (the host keeps every range below
  // 2^31 bytes).  Rows of a q-tile's last tile past its last visible key are then loaded as
  // ordinary finite data and masked.  Per-tile descriptors (PT = true, ranges of 2^31 bytes or
  // more) are rebuilt for every tile, based at its first key and ending at its last valid one.
  const buf_rsrc rkn_all = make_rsrc(kn_b, PT ? 0u : rows_bytes(p.Tk, kn_st, C::KN_RB));
  const buf_rsrc rkr_all = make_rsrc(kr_b, PT ? 0u : rows_bytes(p.Tk, kr_st, 128));
  const buf_rsrc rv_all = make_rsrc(v_b, PT ? 0u : rows_bytes(p.Tk, v_st, 256));
  constexpr uint32_t kNoRows = 0x80000000u;
  auto tile_loads = [&](int kv0, uint32_t lb, int tk) {
    if constexpr (PT) {
      const int nv = min(tk - kv0, C::BN);
      return TileLoads{make_rsrc(kn_b + (int64_t)kv0 * kn_st, rows_bytes(nv, kn_st, C::KN_RB)),
                       make_rsrc(kr_b + (int64_t)kv0 * kr_st, rows_bytes(nv, kr_st, 128)),
                       make_rsrc(v_b + (int64_t)kv0 * v_st, rows_bytes(nv, v_st, 256)), lb, 0u, 0u, 0u};
    } else {
      const bool none = kv0 >= tk;
      const uint32_t r0 = (uint32_t)kv0 * 2u;
      return TileLoads{rkn_all, rkr_all, rv_all, lb, none ? kNoRows : r0 * (uint32_t)kn_st,
                       none ? kNoRows : r0 * (uint32_t)kr_st, none ? kNoRows : r0 * (uint32_t)v_st};
    }
  };
  // load n of the wave's tile loads, n a constant: its region, descriptor and LDS offset
  auto issue_c = [&](const TileLoads& tl, auto n_tag) {
    constexpr int n = decltype(n_tag)::value;
    const uint32_t vo = n == 0 ? vl0 : n == 1 ? vl1 : n == 2 ? vl2 : n == 3 ? vl3 : n == 4 ? vl4 : vl5;
    if constexpr (n < MK_KN) {
      if (w + C::NW * n < C::T_KN) dma16_at<1024 * C::NW * n>(tl.rkn, vo + tl.okn, tl.lb);
    } else if constexpr (n < MK_KN + MK_KR) {
      if (w + C::NW * (n - MK_KN) < C::T_KR) dma16_at<C::OFF_KR + 1024 * C::NW * (n - MK_KN)>(tl.rkr, vo + tl.okr, tl.lb);
    } else if constexpr (n < NL) {
      if (w + C::NW * (n - MK_KN - MK_KR) < C::T_V)
        dma16_at<C::K_STAGE + 1024 * C::NW * (n - MK_KN - MK_KR)>(tl.rv, vo + tl.ov, tl.lb);
    }
  };
  // the same for n known only after unrolling (the switch folds away)
  auto issue = [&](const TileLoads& tl, int n) {
    switch (n) {
      case 0: issue_c(tl, std::integral_constant<int, 0>{}); break;
      case 1: issue_c(tl, std::integral_constant<int, 1>{}); break;
      case 2: issue_c(tl, std::integral_constant<int, 2>{}); break;
      case 3: issue_c(tl, std::integral_constant<int, 3>{}); break;
      case 4: issue_c(tl, std::integral_constant<int, 4>{}); break;
      case 5: issue_c(tl, std::integral_constant<int, 5>{}); break;
      default: break;
    }
  };
  auto load_tile = [&](int kv0, uint32_t lb, int tk) {
    const TileLoads tl = tile_loads(kv0, lb, tk);
#pragma unroll
    for (int n = 0; n < NL; ++n) issue(tl, n);
  };
  // loads this wave issues per tile
  auto n_loads = [&](int total) { return w < total ? (total - w + C::NW - 1) / C::NW : 0; };
  const int loads = n_loads(C::T_KN) + n_loads(C::T_KR) + n_loads(C::T_V);

  // LDS byte offsets (within a stage) of this lane's operands.
  // S^T A operand, k-step ks: row l32, chunk 2 ks' + g of its region.  With power-of-two
  // rows, row * RB + 16 (c ^ f) = (row * RB + 16 f) ^ 16 c.
  const int a_kn = DN == 128 ? (l32 * 256 + 16 * (g ^ swz256(l32))) : (l32 * 128 + 16 * (g ^ swz128(l32)));
  const int a_kr = C::OFF_KR + l32 * 128 + 16 * (g ^ swz128(l32));
  // V^T operand through ds_read_b64_tr_b16: lane r of a 16-lane group addresses key
  // (block start) + 4 g + r / 4, dv columns 32 mb + 16 ((lane >> 4) & 1) + 4 (r % 4).
  const int l16 = lane & 15;
  const int vt_row = 4 * g + (l16 >> 2);
  const int vt_base = vt_row * 256 + 16 * ((2 * ((lane >> 4) & 1) + ((l16 & 3) >> 1)) ^ swzv(vt_row)) + 8 * (l16 & 1);

  // ---- Q^T fragments (B operand of S^T = K Q^T) of the wave's QB row blocks: block qb is
  // rows 32 (QB w + qb) + [0, 32) of the q-tile, dims 16 ks + 8 g + [0, 8)
  bf16x8 qf[QB][C::KS];
  // Q loads of q-tile qt.  With the RoPE fold the rotation waits for its data, so it runs later
  // (rotate_q, just before the q-tile's first scores), after the q-tile's first K/V tile loads
  // are issued; its table rows are loaded there too (held from here they would have to live
  // through the previous q-tile's epilogue).
  int q_rot_tile = 0;
  auto load_q = [&](int qt) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int q_row = qt * BM + 32 * (QB * w + qb) + l32;
      const int q_ld = q_row < p.Tq ? q_row : p.Tq - 1;  // clamped row for loads
      const bf16* qn = p.qn + (int64_t)b * p.qn_s.b + (int64_t)q_ld * p.qn_s.t + (int64_t)h * p.qn_s.h;
      const bf16* qr = p.qr + (int64_t)b * p.qr_s.b + (int64_t)q_ld * p.qr_s.t + (int64_t)h * p.qr_s.h;
#pragma unroll
      for (int ks = 0; ks < C::KS; ++ks) {
        const int d = 16 * ks + 8 * g;
        qf[qb][ks] = as_bf16x8(d < DN ? ldg16(qn + d) : ldg16(qr + (d - DN)));
      }
    }
    q_rot_tile = qt;
  };
  // The rotation of the loaded rope slice; with `store` (the item that starts the q-tile, when
  // qr_out is set) the rotated slice also goes to qr_out.  The lane holds rope dims 16 k + 8 g +
  // [0, 8) (k-steps KNS + k, k = 0..3): dims f and f + 32 (k and k + 2) are a rotation pair,
  // f = 16 k + 8 g + e, k = 0, 1.
  auto rotate_q = [&](bool store) {
    if (!p.rope_cos) return;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int q_row = q_rot_tile * BM + 32 * (QB * w + qb) + l32;
      const int64_t pos = p.q_pos_offset + (q_row < p.Tq ? q_row : p.Tq - 1);
      // cos, then sin, of freqs 8 g + [0, 8) and 16 + 8 g + [0, 8)
      const u32x4 c0 = ldg16(p.rope_cos + pos * 32 + 8 * g), c1 = ldg16(p.rope_cos + pos * 32 + 16 + 8 * g);
      const u32x4 s0 = ldg16(p.rope_sin + pos * 32 + 8 * g), s1 = ldg16(p.rope_sin + pos * 32 + 16 + 8 * g);
      rope_rotate8(qf[qb][C::KNS], qf[qb][C::KNS + 2], c0, s0);
      rope_rotate8(qf[qb][C::KNS + 1], qf[qb][C::KNS + 3], c1, s1);
      if (store && p.qr_out && q_row < p.Tq) {
        bf16* qo = p.qr_out + (int64_t)b * p.qro_s.b + (int64_t)q_row * p.qro_s.t + (int64_t)h * p.qro_s.h;
#pragma unroll
        for (int k = 0; k < 4; ++k) stg16(qo + 16 * k + 8 * g, as_u32x4(qf[qb][C::KNS + k]));
      }
    }
  };
  // first loads of an item (key tiles [lo, hi) of a q-tile whose keys end at kv_end): tiles
  // lo .. lo + AHEAD - 1
  auto first_tiles = [&](int lo, int hi, int kv_end) {
    const int tk = min(p.Tk, kv_end);
    load_tile(lo * C::BN, stage_lds(S0{}), lo < hi ? tk : 0);
    load_tile((lo + 1) * C::BN, stage_lds(S1{}), lo + 1 < hi ? tk : 0);
    load_tile((lo + 2) * C::BN, stage_lds(S2{}), lo + 2 < hi ? tk : 0);
  };
  static_assert(C::AHEAD == 3, "first_tiles issues AHEAD tiles");
  // exclusive end of the keys that q-tile qt sees
  auto key_end = [&](int qt) {
    int kv_end = p.Tk;
    if (p.causal) {
      const int64_t lim = (int64_t)qt * BM + BM + p.q_offset;
      if (lim < kv_end) kv_end = (int)lim;
    }
    return kv_end;
  };
  auto start_item = [&](int i) {
    const int qt = i == 0 ? it_qt[0] : it_qt[1];
    load_q(qt);
    first_tiles(i == 0 ? it_lo[0] : it_lo[1], i == 0 ? it_hi[0] : it_hi[1], key_end(qt));
  };

  __syncthreads();  // the zeros are in place before any load lands
  start_item(0);

  for (int item = 0; item < n_items; ++item) {
  const int qt = item == 0 ? it_qt[0] : it_qt[1];
  const int t_lo = item == 0 ? it_lo[0] : it_lo[1];  // the item's key tiles [t_lo, t_hi)
  const int t_hi = item == 0 ? it_hi[0] : it_hi[1];
  const int q0 = qt * BM;
  const int qw0 = q0 + 32 * QB * w;  // first query row of this wave; block qb starts 32 qb further

  // ---- key range of the workgroup and of this wave
  const int kv_end = key_end(qt);
  int wave_last = p.Tk - 1;  // last key any row of this wave can see
  if (p.causal) {
    const int64_t wl = (int64_t)qw0 + 32 * QB - 1 + p.q_offset;
    if (wl < wave_last) wave_last = (int)wl;
  }
  const int n_tiles = t_hi - t_lo;  // steps of the item
  const int n_vis = min(t_hi, wave_last / C::BN + 1);  // tiles (absolute index) below it have a key this wave sees

  f32x16 oacc[QB][4];
  float m_run[QB], l_run[QB];  // per row block: log2 reference max of the lane's row; its share of the sum

  // Tile loop, software-pipelined: step j computes the scores of tile j + 1 while it turns
  // the scores of tile j into P and accumulates P V.  Tile t sits in stage t % 4 and its
  // loads are issued in step t - 3; one barrier per step.
  // Fast form (SAFE = false): the reference max is the first tile's row max (key 0 is
  // visible to every row) and never moves, so later tiles need no max, no rescale and no
  // branch on the scores.  p = 2^(s - m) stays finite unless a later score exceeds the
  // first tile's max by more than ~127 (log2); the workgroup then votes and recomputes the
  // q-tile with the safe form, which moves the reference max lazily (when it grows by more
  // than kFwdRescale) and rescales O and l.
  // With a multiple of NSTAGE tiles the steps past the end load the next q-tile's first
  // AHEAD tiles (its own first steps then find them in place).
  const int kv_end_next = item + 1 < n_items ? key_end(it_qt[1]) : 0;
  const int lo_next = it_lo[1], hi_next = it_hi[1];
  const bool prefetch = item + 1 < n_items && n_tiles % C::NSTAGE == 0;
  // the first tile whose scores this wave must mask: one crossing its causal diagonal
  // (32 j + 31 > qw0 + q_offset) or reaching past Tk (32 j + 32 > Tk); tiles [1, mask_from)
  // are fully visible to every row of the wave and skip the mask and the max
  int mask_from = p.Tk / C::BN;
  if (p.causal) mask_from = min(mask_from, (qw0 + q_off + 1) / C::BN);

  auto run_tiles = [&](auto safe_tag) {
    constexpr bool SAFE = decltype(safe_tag)::value;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) oacc[qb][mb] = f32x16{};
      m_run[qb] = -INFINITY;
      l_run[qb] = 0.f;
    }
    // S^T of the tile being consumed and of the next one: tiles alternate between sA and sB
    f32x16 sA[QB], sB[QB];

    // S^T (32 x 32) of one K tile: one chain of KS MFMAs; the A fragments are read ahead of
    // their use as the group barriers of the caller's region pin it
    auto scores = [&](const unsigned char* kst, f32x16 (&out)[QB], int b_kn, int b_kr) {
      bf16x8 a[C::KS];
#pragma unroll
      for (int ks = 0; ks < C::KS; ++ks) {
        const int off = ks < C::KNS ? b_kn ^ (32 * ks) : b_kr ^ (32 * (ks - C::KNS));
        a[ks] = as_bf16x8(lds16(kst + off));
      }
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) out[qb] = f32x16{};
#pragma unroll
      for (int ks = 0; ks < C::KS; ++ks)
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) out[qb] = mfma32(a[ks], qf[qb][ks], out[qb]);
    };

    // One step: tile j's P and P V, and the scores of tile j + 1.  Every wave runs it for
    // every tile (one code path keeps the accumulators in place): a tile that no row of the
    // wave can see (j >= n_vis) is masked to p = 0 and skips its P V MFMAs; scores of a tile
    // past the end read a stage of stale finite data and go unused.
    auto body = [&](int j, const unsigned char* vcur, const unsigned char* knext, f32x16 (&sacc)[QB],
                    f32x16 (&snext)[QB], const TileLoads& tl) {
      const int kv0 = j * C::BN;
      // masking and the max are needed only on the first tile and from mask_from on
      if (SAFE || j == t_lo || j >= mask_from) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          const int qb0 = qw0 + 32 * qb;  // first row of the block
          // mask only the tiles that cross the causal diagonal or the end of the keys
          const bool need_mask = (p.causal && kv0 + C::BN - 1 > qb0 + q_off) || kv0 + C::BN > p.Tk;
          if (need_mask) {
            // key kv is visible to this lane's row iff kv < lim (lim <= Tk)
            const int lim = p.causal ? min(p.Tk, qb0 + l32 + q_off + 1) : p.Tk;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int kv = kv0 + 8 * (r >> 2) + 4 * g + (r & 3);
              sacc[qb][r] = kv < lim ? sacc[qb][r] : -INFINITY;
            }
          }
          if (SAFE || j == t_lo) {
            float mx = max3f(sacc[qb][0], sacc[qb][1], sacc[qb][2]);
#pragma unroll
            for (int r = 3; r < 15; r += 2) mx = max3f(mx, sacc[qb][r], sacc[qb][r + 1]);
            float mloc = fmaxf(mx, sacc[qb][15]);
            mloc = xor32_max(mloc) * p.scale_log2;  // scale > 0 commutes with max
            if (!SAFE) {
              m_run[qb] = mloc;
            } else if (__any(mloc > m_run[qb] + kFwdRescale)) {
              const float m_new = mloc > m_run[qb] + kFwdRescale ? mloc : m_run[qb];
              const float alpha = fast_exp2(m_run[qb] - m_new);  // 1 for rows that keep m_run (incl. -inf)
              m_run[qb] = m_new;
              l_run[qb] *= alpha;
#pragma unroll
              for (int mb = 0; mb < 4; ++mb) oacc[qb][mb] *= alpha;
            }
          }
        }
      }
      float neg_m[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) neg_m[qb] = m_run[qb] == -INFINITY ? 0.f : -m_run[qb];

      // the per-k-step read addresses (base ^ constant) are loop-invariant: the compiler keeps
      // them in registers
      const int b_kn = a_kn, b_kr = a_kr, b_vt = vt_base;
      bf16x8 pb[QB][2];

      // Phase 1 carries the dependency chain from one tile to the next (scores, then the
      // exponentials): it runs at raised wave priority, so the other wave of the SIMD fills
      // the gaps rather than delaying it.
      __builtin_amdgcn_s_setprio(1);
      // Phase 1, in chunks (in the key-split form no instruction crosses a chunk boundary): chunk n reads
      // the A fragment of k-step n + S_AHEAD, issues score MFMA n of tile j + 1 and, in the
      // last 8 chunks, turns two scores of tile j into p = 2^(s * scale - m), so the
      // exponentials run while the MFMAs do (starting them after the first KS - 8 MFMAs
      // measured 1-1.5 % faster than in the first 8 chunks).
      {
        auto ka = [&](int ks) {
          const int off = ks < C::KNS ? b_kn ^ (32 * ks) : b_kr ^ (32 * (ks - C::KNS));
          return as_bf16x8(lds16(knext + off));
        };
        bf16x8 a[C::KS];
#pragma unroll
        for (int ks = 0; ks < S_AHEAD; ++ks) a[ks] = ka(ks);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) snext[qb] = f32x16{};
        uint32_t pkw[QB][8];
#pragma unroll
        for (int n = 0; n < C::KS; ++n) {
          if (n + S_AHEAD < C::KS) a[n + S_AHEAD] = ka(n + S_AHEAD);
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) snext[qb] = mfma32(a[n], qf[qb][n], snext[qb]);
          if (n < NL) issue(tl, n);  // the next tile's loads ride between the MFMAs
          static_assert(C::KS >= 8, "the 8 pairs of scores need 8 chunks");
          if (n >= C::KS - 8) {
            const int pi = n - (C::KS - 8);  // pair of scores (rows 2 pi, 2 pi + 1)
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
              const float p0 = fast_exp2(__builtin_fmaf(sacc[qb][2 * pi], p.scale_log2, neg_m[qb]));
              const float p1 = fast_exp2(__builtin_fmaf(sacc[qb][2 * pi + 1], p.scale_log2, neg_m[qb]));
              l_run[qb] += p0 + p1;
              pkw[qb][pi] = pack_bf16x2(p0, p1);
            }
          }
          // chunk boundaries: kept in the key-split form (3.7 % faster with them at B = 1, T = 2048);
          // the unsplit form schedules across them (1.5 % faster at config 3, the same at config 1)
          if constexpr (SP) __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          pb[qb][0] = as_bf16x8(u32x4{pkw[qb][0], pkw[qb][1], pkw[qb][2], pkw[qb][3]});
          pb[qb][1] = as_bf16x8(u32x4{pkw[qb][4], pkw[qb][5], pkw[qb][6], pkw[qb][7]});
        }
      }

      __builtin_amdgcn_s_setprio(0);
      // Phase 2: O^T (128 x 32) += V^T (128 x 32) P^T (32 x 32), chunk n reading the V^T
      // fragment PV_AHEAD MFMAs ahead.  K slot (g, e) <-> key 16 s + 8 (e / 4) + 4 g + e % 4,
      // matching the S^T accumulator rows; rows 16 s (+ 8) keep row % 4, so only the dv
      // block mb changes the swizzle.
      {
        typedef short s16x4 __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
        auto vtr = [&](int n) {  // n = 4 s + mb
          const int off = (b_vt ^ (64 * (n & 3))) + 16 * (n >> 2) * 256;
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vcur + off));
          const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vcur + off + 8 * 256));
          const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
          return as_bf16x8(u32x4{l2[0], l2[1], h2[0], h2[1]});
        };
        bf16x8 vt[8];
        if (j < n_vis) {  // every p of an invisible tile is 0
#pragma unroll
        for (int n = 0; n < PV_AHEAD; ++n) vt[n] = vtr(n);
#pragma unroll
        for (int n = 0; n < 8; ++n) {
          if (n + PV_AHEAD < 8) vt[n + PV_AHEAD] = vtr(n + PV_AHEAD);
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) oacc[qb][n & 3] = mfma32(vt[n], pb[qb][n >> 2], oacc[qb][n & 3]);
          __builtin_amdgcn_sched_barrier(0);
        }
        }
      }
    };

    // step j: tile j's stage holds its V, tile j + 1's stage its K.  Entering step j, the
    // loads of tiles j + 1 and j + 2 may be in flight (LOADS each, in issue order): waiting
    // until at most LOADS remain lands tile j + 1; after the barrier every wave is done
    // with tile j - 1, whose stage receives tile j + AHEAD.
    auto step = [&](int j, auto par_tag) {
      constexpr int P = decltype(par_tag)::value;
      unsigned char* vcur = stage(par_tag) + C::K_STAGE;
      const unsigned char* knext = stage(std::integral_constant<int, P + 1>{});
      const uint32_t fill = stage_lds(std::integral_constant<int, P + C::AHEAD>{});
      static_assert(C::AHEAD == 3, "the wait leaves one tile's loads in flight");
      wait_vmem(loads);
      __syncthreads();
      // tile t of this q-tile; past the end, the next q-tile's tile t - n_tiles when
      // prefetching (its stage is then (t - n_tiles) % NSTAGE, where that q-tile starts)
      const int t = j + C::AHEAD;
      int kv0t = (t_lo + t) * C::BN, tk = t < n_tiles ? kv_end : 0;
      if (t >= n_tiles && prefetch) {
        const int tn = lo_next + t - n_tiles;
        kv0t = tn * C::BN;
        tk = tn < hi_next ? kv_end_next : 0;
      }
      const TileLoads tl = tile_loads(kv0t, fill, tk);
      if constexpr (P % 2 == 0) body(t_lo + j, vcur, knext, sA, sB, tl);
      else body(t_lo + j, vcur, knext, sB, sA, tl);
    };

    // prologue: scores of tile 0 (tiles 0 .. AHEAD - 1 are in flight)
    wait_vmem(2 * loads);
    __syncthreads();
    if constexpr (!SAFE) rotate_q(t_lo == 0);  // once per q-tile item (the safe redo keeps Q)
    scores(stage(S0{}), sA, a_kn, a_kr);
    __builtin_amdgcn_sched_group_barrier(kSgDsRead, S_AHEAD, 0);
#pragma unroll
    for (int n = 0; n < C::KS - S_AHEAD; ++n) {
      __builtin_amdgcn_sched_group_barrier(kSgMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSgDsRead, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kSgMfma, S_AHEAD, 0);

    using S3 = std::integral_constant<int, 3>;
    for (int j = 0; j < n_tiles; j += 4) {
      step(j, S0{});
      if (j + 1 < n_tiles) step(j + 1, S1{});
      if (j + 2 < n_tiles) step(j + 2, S2{});
      if (j + 3 < n_tiles) step(j + 3, S3{});
    }
  };

  run_tiles(std::false_type{});
  {
    // workgroup vote: did any row's sum leave the finite range of the fixed reference?
    // The vote slots sit in stage 3, which loads in flight of the next q-tile's tiles
    // 0 .. 2 do not touch; empty loads past the end land first.
    int* vote = reinterpret_cast<int*>(stage3);
    bool bad = false;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) bad |= !(xor32_sum(l_run[qb]) <= kFwdSumLimit);
    const bool any_bad = __any(bad);  // a wave-wide vote: every lane takes part
    if (!prefetch) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (lane == 0) vote[w] = any_bad ? 1 : 0;
    __syncthreads();
    int any = 0;
#pragma unroll
    for (int i = 0; i < C::NW; ++i) any |= vote[i];
    const bool redo = any != 0;
    if (redo) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // prefetched tiles land before reloading
      first_tiles(t_lo, t_hi, kv_end);
      run_tiles(std::true_type{});
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();  // every wave is done with the stages before the next q-tile's loads
    }
  }
  // the next q-tile's first loads (its tiles are already in flight when prefetched) overlap
  // this one's epilogue
  if (item + 1 < n_items) {
    if (prefetch) load_q(it_qt[1]);
    else start_item(1);
  }
  // a q-tile whose keys span several segments leaves its partial in the workspace
  const int parts = item == 0 ? it_parts[0] : it_parts[1];
  const bool partial = SP && parts > 1;

  // ---- epilogue: normalise and store O [q][d] and LSE
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int q_row = qw0 + 32 * qb + l32;  // this lane's query in block qb
    const float l_tot = xor32_sum(l_run[qb]);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    // Lane (l32, g) holds dv 32 mb + 8 i + 4 g + [0, 4) of its query; swapping the upper
    // half-wave's even-i runs with the lower half-wave's odd-i runs (v_permlane32_swap) gives
    // every lane 16 contiguous bytes: dv 32 mb + 16 k + 8 g + [0, 8), k = 0, 1.  Each 32-column
    // block is packed and stored before the next (few registers live beside the next q-tile's Q).
    const bool row_ok = q_row < p.Tq;
    // the partial of segment seg: rows of q-tile qt in slot seg (dv contiguous, fp32), log2 LSE
    const int64_t ws_row = ((((int64_t)b * p.H + h) * p.n_qt + qt) * p.S + seg) * BM + (q_row - q0);
    if (!partial) {
      bf16* op = p.o + (int64_t)b * p.o_s.b + (int64_t)q_row * p.o_s.t + (int64_t)h * p.o_s.h;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        u32x4 ost[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          uint32_t x[2], y[2];
#pragma unroll
          for (int d = 0; d < 2; ++d) {
            x[d] = pack_bf16x2(oacc[qb][mb][8 * k + 2 * d] * inv, oacc[qb][mb][8 * k + 2 * d + 1] * inv);
            y[d] = pack_bf16x2(oacc[qb][mb][8 * k + 4 + 2 * d] * inv, oacc[qb][mb][8 * k + 4 + 2 * d + 1] * inv);
            const auto r = __builtin_amdgcn_permlane32_swap(x[d], y[d], false, false);
            x[d] = r[0];
            y[d] = r[1];
          }
          ost[k] = u32x4{x[0], x[1], y[0], y[1]};
        }
        if (row_ok) {
#pragma unroll
          for (int k = 0; k < 2; ++k) stg16(op + 32 * mb + 16 * k + 8 * g, ost[k]);
        }
      }
    } else if (row_ok) {
      float* wp = p.ws_o + ws_row * 128;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i)  // dv 32 mb + 8 i + 4 g + [0, 4)
          *reinterpret_cast<f32x4*>(wp + 32 * mb + 8 * i + 4 * g) =
              f32x4{oacc[qb][mb][4 * i] * inv, oacc[qb][mb][4 * i + 1] * inv, oacc[qb][mb][4 * i + 2] * inv,
                    oacc[qb][mb][4 * i + 3] * inv};
    }
    if (row_ok) {
      if (g == 0) {
        const float lse2 = l_tot > 0.f ? m_run[qb] + fast_log2(l_tot) : -INFINITY;
        if (partial) p.ws_lse[ws_row] = lse2;
        else p.lse[((int64_t)b * p.H + h) * p.Tq + q_row] = lse2 * kLn2;
      }
    }
  }
  }  // item
}

// Row blocks per wave.  QB = 2 (64 rows per wave, one wave per SIMD, every K/V fragment
// read feeds two MFMAs) is correct but measured 13-25 % slower than QB = 1 (two waves per
// SIMD hide each other's latencies); it stays available as a build option.
#ifndef FWD_QB
#define FWD_QB 1
#endif
// Combines the partials of the q-tiles that a key split cut: per row, the max of the partials'
// log2 LSE m, weights w_s = 2^(lse_s - m), O = sum_s w_s O_s / sum_s w_s in slot (key) order,
// LSE = (m + log2 sum_s w_s) ln 2.  Sixteen threads per row, 8 dv each; a workgroup covers 16
// rows of one q-tile.
template <int BM>
__global__ __launch_bounds__(256) void fwd_merge_kernel(FwdParams p) {
  constexpr int RPW = 16;  // rows per workgroup
  const int chunk = blockIdx.x % (BM / RPW);
  const int tile = blockIdx.x / (BM / RPW);  // ((b H + h) n_qt + qt)
  const int qt = tile % p.n_qt;
  const int bh = tile / p.n_qt;
  int parts, first;
  fwd_qtile_parts(qt, p.n_qt, BM, p.Tk, p.causal, p.q_offset, p.S, parts, first);
  if (parts <= 1) return;  // that q-tile wrote O itself
  const int r = chunk * RPW + (int)(threadIdx.x >> 4);
  const int q_row = qt * BM + r;
  if (q_row >= p.Tq) return;
  const int d0 = 8 * (int)(threadIdx.x & 15);
  const int64_t row0 = ((int64_t)tile * p.S + first) * BM + r;  // workspace row of the first slot
  constexpr int MAXS = 8;
  float ls[MAXS];
  f32x4 ov[MAXS][2];
#pragma unroll
  for (int i = 0; i < MAXS; ++i) {  // parts is uniform over the workgroup: the loads issue together
    if (i < parts) {
      const int64_t row = row0 + (int64_t)i * BM;
      ls[i] = p.ws_lse[row];
      ov[i][0] = *reinterpret_cast<const f32x4*>(p.ws_o + row * 128 + d0);
      ov[i][1] = *reinterpret_cast<const f32x4*>(p.ws_o + row * 128 + d0 + 4);
    }
  }
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < MAXS; ++i)
    if (i < parts) m = fmaxf(m, ls[i]);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float wsum = 0.f;
  if (m != -INFINITY) {
#pragma unroll
    for (int i = 0; i < MAXS; ++i) {
      if (i < parts) {
        const float wgt = fast_exp2(ls[i] - m);  // 0 for a partial that saw no key
        wsum += wgt;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[e] += wgt * ov[i][0][e];
          acc[4 + e] += wgt * ov[i][1][e];
        }
      }
    }
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  u32x4 out;
#pragma unroll
  for (int e = 0; e < 4; ++e) out[e] = pack_bf16x2(acc[2 * e] * inv, acc[2 * e + 1] * inv);
  const int b = bh / p.H, h = bh - (bh / p.H) * p.H;
  stg16(p.o + (int64_t)b * p.o_s.b + (int64_t)q_row * p.o_s.t + (int64_t)h * p.o_s.h + d0, out);
  if ((threadIdx.x & 15) == 0)
    p.lse[(int64_t)bh * p.Tq + q_row] = wsum > 0.f ? (m + fast_log2(wsum)) * kLn2 : -INFINITY;
}

// Segments per pair of q-tiles: 1 (no split) when the pairs alone give every CU a workgroup
// (> 128 pairs); else enough to reach ~256 workgroups (one per CU: a workgroup's fixed cost
// of ~6 us for its Q and first tiles, its q-tile switch and its stores is exposed at small
// grids, and two per CU measured slower), at most 8 and at least 8 key tiles per segment of
// the longest pair.
template <int DN>
static int fwd_split_count(const FwdParams& prm) {
  constexpr int BM = 32 * FWD_QB * FwdCfg<DN>::NW;
  const int n_qt = (prm.Tq + BM - 1) / BM;
  const int64_t units = (int64_t)prm.B * prm.H * ((n_qt + 1) / 2);
  if (units <= 0 || units > 128) return 1;
  const FwdSplit f = fwd_split_of_pair(0, n_qt, BM, prm.Tk, prm.causal, prm.q_offset);
  int S = (int)(256 / units);
  S = min(S, 8);
  S = min(S, f.N / 8);
  return S < 2 ? 1 : S;
}
template <int DN>
static size_t fwd_workspace_bytes(const FwdParams& prm) {
  constexpr int BM = 32 * FWD_QB * FwdCfg<DN>::NW;
  const int S = fwd_split_count<DN>(prm);
  if (S <= 1) return 0;
  const int64_t rows = (int64_t)prm.B * prm.H * ((prm.Tq + BM - 1) / BM) * S * BM;
  return (size_t)(rows * 512 + rows * 4);  // fp32 partials, then log2 LSEs
}

template <int DN>
static int launch_fwd(FwdParams prm, hipStream_t s, void* ws, size_t ws_bytes) {
  constexpr int QB = FWD_QB;
  constexpr int BM = 32 * QB * FwdCfg<DN>::NW;
  prm.n_qt = (prm.Tq + BM - 1) / BM;
  // whole-range descriptors need each operand's rows [0, Tk) below 2^31 bytes
  auto range_ok = [&](const mla_strides& st, int row_bytes) {
    return prm.Tk <= 0 || ((int64_t)(prm.Tk - 1) * st.t * 2 + row_bytes) < (1ll << 31);
  };
  const bool pt = !(range_ok(prm.kn_s, 2 * DN) && range_ok(prm.kr_s, 128) && range_ok(prm.v_s, 256));
  const size_t need = fwd_workspace_bytes<DN>(prm);
  const dim3 blk(64 * FwdCfg<DN>::NW);
  if (!pt && need > 0 && ws && ws_bytes >= need) {
    prm.S = fwd_split_count<DN>(prm);
    const int64_t rows = (int64_t)prm.B * prm.H * prm.n_qt * prm.S * BM;
    prm.ws_o = (float*)ws;
    prm.ws_lse = (float*)((char*)ws + rows * 512);
    const int64_t n = (int64_t)prm.B * prm.H * ((prm.n_qt + 1) / 2) * prm.S;
    MLA_CHECK(n < (1ll << 31), MLA_ERR_INVALID_ARG, "mla_prefill_fwd: grid too large");
    prefill_fwd_kernel<DN, QB, false, true><<<dim3((unsigned)n), blk, 0, s>>>(prm);
    MLA_TRY(launch_status("mla_prefill_fwd"));
    const int64_t nm = (int64_t)prm.B * prm.H * prm.n_qt * (BM / 16);
    fwd_merge_kernel<BM><<<dim3((unsigned)nm), dim3(256), 0, s>>>(prm);
    return launch_status("mla_prefill_fwd (split merge)");
  }
  prm.S = 1;
  prm.ws_o = nullptr;
  prm.ws_lse = nullptr;
  const int64_t n = (int64_t)prm.B * prm.H * ((prm.n_qt + 1) / 2);
  MLA_CHECK(n < (1ll << 31), MLA_ERR_INVALID_ARG, "mla_prefill_fwd: grid too large");
  if (pt) prefill_fwd_kernel<DN, QB, true, false><<<dim3((unsigned)n), blk, 0, s>>>(prm);
  else prefill_fwd_kernel<DN, QB, false, false><<<dim3((unsigned)n), blk, 0, s>>>(prm);
  return launch_status("mla_prefill_fwd");
}

}  // namespace mla

using namespace mla;

static FwdParams fwd_params(const mla_prefill_fwd_args* a);

extern "C" int mla_prefill_fwd(const mla_prefill_fwd_args* a, void* stream) {
  const char* op = "mla_prefill_fwd";
  MLA_CHECK(a, MLA_ERR_INVALID_ARG, "%s: null args", op);
  MLA_TRY(check_scale(op, a->scale));
  MLA_CHECK(a->d_rope == 64 && a->d_v == 128 && (a->d_nope == 128 || a->d_nope == 64), MLA_ERR_UNSUPPORTED,
            "%s: head dims (nope %lld, rope %lld, v %lld) not built; supported nope in {64,128}, rope 64, v 128",
            op, (long long)a->d_nope, (long long)a->d_rope, (long long)a->d_v);
  MLA_CHECK(a->B >= 0 && a->H >= 0 && a->Tq >= 0 && a->Tk >= 0, MLA_ERR_INVALID_ARG, "%s: negative size", op);
  MLA_CHECK(a->B < (1 << 20) && a->H < (1 << 16) && a->Tq < (1 << 30) && a->Tk < (1 << 30), MLA_ERR_INVALID_ARG,
            "%s: size out of range", op);
  if (a->B == 0 || a->H == 0 || a->Tq == 0) return MLA_OK;
  MLA_CHECK(a->Tk > 0, MLA_ERR_INVALID_ARG, "%s: Tk must be positive", op);
  MLA_CHECK(!a->causal || a->q_offset >= 0, MLA_ERR_INVALID_ARG, "%s: q_offset must be >= 0", op);
  MLA_CHECK(a->q_offset < (1 << 30), MLA_ERR_INVALID_ARG, "%s: q_offset out of range", op);
  MLA_CHECK(a->k_nope_stride.t < (1 << 24) && a->k_rope_stride.t < (1 << 24) && a->v_stride.t < (1 << 24),
            MLA_ERR_INVALID_ARG, "%s: key/value row strides must be below 2^24 elements", op);
  MLA_TRY(check_operand(op, "q_nope", a->q_nope, a->q_nope_stride));
  MLA_TRY(check_operand(op, "q_rope", a->q_rope, a->q_rope_stride));
  MLA_TRY(check_operand(op, "k_nope", a->k_nope, a->k_nope_stride));
  MLA_TRY(check_operand(op, "k_rope", a->k_rope, a->k_rope_stride));
  MLA_TRY(check_operand(op, "v", a->v, a->v_stride));
  MLA_TRY(check_operand(op, "o", a->o, a->o_stride));
  MLA_CHECK(a->lse, MLA_ERR_INVALID_ARG, "%s: lse is null", op);
  MLA_CHECK(!a->rope_cos == !a->rope_sin, MLA_ERR_INVALID_ARG, "%s: rope_cos and rope_sin go together", op);
  if (a->rope_cos) {
    MLA_CHECK(((uintptr_t)a->rope_cos & 15) == 0 && ((uintptr_t)a->rope_sin & 15) == 0, MLA_ERR_INVALID_ARG,
              "%s: RoPE tables must be 16-byte aligned", op);
    MLA_CHECK(a->q_pos_offset >= 0 && a->q_pos_offset + a->Tq <= a->rope_rows, MLA_ERR_INVALID_ARG,
              "%s: query positions %lld..%lld exceed the RoPE table (%lld rows)", op, (long long)a->q_pos_offset,
              (long long)(a->q_pos_offset + a->Tq - 1), (long long)a->rope_rows);
    if (a->q_rope_out) MLA_TRY(check_operand(op, "q_rope_out", a->q_rope_out, a->q_rope_out_stride));
  } else {
    MLA_CHECK(!a->q_rope_out, MLA_ERR_INVALID_ARG, "%s: q_rope_out needs the RoPE tables", op);
  }
  const FwdParams prm = fwd_params(a);
  hipStream_t s = (hipStream_t)stream;
  return a->d_nope == 128 ? launch_fwd<128>(prm, s, a->workspace, a->workspace_bytes)
                          : launch_fwd<64>(prm, s, a->workspace, a->workspace_bytes);
}

extern "C" size_t mla_prefill_fwd_workspace_bytes(const mla_prefill_fwd_args* a) {
  if (!a || a->B <= 0 || a->H <= 0 || a->Tq <= 0 || a->Tk <= 0 || a->B >= (1 << 20) || a->H >= (1 << 16) ||
      a->Tq >= (1 << 30) || a->Tk >= (1 << 30) || a->q_offset < 0 || a->q_offset >= (1 << 30) ||
      (a->d_nope != 128 && a->d_nope != 64))
    return 0;
  const FwdParams prm = fwd_params(a);
  return a->d_nope == 128 ? fwd_workspace_bytes<128>(prm) : fwd_workspace_bytes<64>(prm);
}

static FwdParams fwd_params(const mla_prefill_fwd_args* a) {
  FwdParams prm;
  prm.qn = (const bf16*)a->q_nope;
  prm.qr = (const bf16*)a->q_rope;
  prm.kn = (const bf16*)a->k_nope;
  prm.kr = (const bf16*)a->k_rope;
  prm.v = (const bf16*)a->v;
  prm.o = (bf16*)a->o;
  prm.lse = a->lse;
  prm.B = (int)a->B;
  prm.H = (int)a->H;
  prm.Tq = (int)a->Tq;
  prm.Tk = (int)a->Tk;
  prm.n_qt = 0;  // set by launch_fwd for its q-tile height
  prm.qn_s = a->q_nope_stride;
  prm.qr_s = a->q_rope_stride;
  prm.kn_s = a->k_nope_stride;
  prm.kr_s = a->k_rope_stride;
  prm.v_s = a->v_stride;
  prm.o_s = a->o_stride;
  prm.scale_log2 = a->scale * kLog2e;
  prm.causal = a->causal ? 1 : 0;
  prm.q_offset = a->q_offset;
  prm.S = 1;
  prm.ws_o = nullptr;
  prm.ws_lse = nullptr;
  prm.rope_cos = (const bf16*)a->rope_cos;
  prm.rope_sin = (const bf16*)a->rope_sin;
  prm.q_pos_offset = a->q_pos_offset;
  prm.qr_out = (bf16*)a->q_rope_out;
  prm.qro_s = a->q_rope_out_stride;
  return prm;
}
