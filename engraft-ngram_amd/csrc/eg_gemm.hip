// The PLE block's projections (engraft/replica/layers.py:594-606: key = emb
// w_key^T and value = emb w_value^T, as two column groups over the same A in
// one launch, and their backward d_emb = d_key w_key + d_value w_value as two
// K segments with the weights' transposes kept row-major):
//
//   C[M, N] (+)= A[M, K] B[N, K]^T  (+ A2[M, K2] B2[N, K2]^T)
//
// in two arithmetics.
//
// gemm_x3_kernel, fp32 on the bf16 matrix cores: each fp32 operand is split
// once (eg_split_bf16) into bf16 planes hi = rne(x) and lo = rne(x - hi)
// (x - hi is exact in fp32), and C accumulates hi*hi + hi*lo + lo*hi in fp32
// on v_mfma_f32_32x32x16_bf16.  hi + lo keeps 16 of fp32's 24 mantissa bits,
// so each product carries a relative error up to ~3 x 2^-18 (fp32's own is
// 2^-24): about 1e-5 of the result on random data, at the bf16 rate.
//
// gemm_f32_kernel, fp32 arithmetic on the fp32 matrix cores
// (v_mfma_f32_32x32x2_f32): the products of an fp32 matmul, each operand
// read once as fp32.
//
// Tiling, both: 256 x 256 output tiles, one workgroup a CU; K in steps of 32
// through a two-stage LDS ring filled by direct-to-LDS loads
// (global_load_lds_dwordx4: lane i of a wavefront writes 16 bytes at the
// wavefront's LDS base + 16 i), so the next step's loads are in flight during
// the current step's MFMAs without passing through registers.
// gemm_x3: eight wavefronts of 128 x 64 outputs (4 x 2 MFMA tiles of 32 x 32),
// 128 KB of LDS (four bf16 planes a stage), software-pipelined: a half step's
// fragments are read during the other half step's MFMAs, one barrier a step.
// On the key projection (M 2048, N 10240, K 2560) 290 us against 319 us for
// the 128 x 128 tiles of four wavefronts it replaces (two workgroups a CU,
// the last round in K quarters), and the backward's d_emb 400 against 470 us;
// sixteen wavefronts of 64 x 64 or eight of 64 x 128 ran 1-4 % slower, four
// of 128 x 128 (one a SIMD, the accumulators in the accumulation registers,
// a third less LDS read a step) 8-13 % slower on the bf16x3 and bf16x6 shapes, the
// same tile without the pipelining 2 % slower, with 2-way LDS bank conflicts
// on the fragment reads 2-3 % slower; the reads interleaved one by one with
// the MFMAs, or the wave priority raised over the MFMA passes, within 1 %.  Measured earlier on the 128 x 128 tile
// and dropped: three stages, scheduling hints, register-staged loads into a
// padded LDS tile (20 % slower).  Counters on the key projection: the matrix
// cores busy 55 % of the cycles (SQ_VALU_MFMA_BUSY_CYCLES) at a shader clock
// of ~1.8 GHz under this load.  gemm_f32: sixteen wavefronts of 64 x 64, 128 KB of
// LDS: 88.8 % of the fp32 MFMA peak where the tiles fill whole rounds,
// against 83.3 % for 128 x 128 tiles of four.
//
// The last round.  When the tile count leaves the last round (one tile a CU)
// partly empty, the (tile, K step) units of that round's tiles are cut into
// one contiguous range a CU, each range's parts (one or two tiles) go to a
// workspace, and sk_sum_kernel adds each tile's parts in K order into C, so
// the result does not depend on scheduling.  On MI355X (256 CUs): the fp32
// key + value's 400 tiles run as 256 whole and 144 in 256 ranges of 45 of a
// tile's 80 K steps (1040 us against 1249 us whole and 1126 us with the 144
// in sevenths), the backward's 80 tiles of 400 K steps in 256 ranges of 125
// (1018 us against 1091 us in thirds); the bf16x3 key projection's 320 tiles
// as 256 whole and 64 in 256 ranges of 20.  An explicit k_slices cuts every
// tile into that many equal pieces instead (piece_sum_kernel adds them).
//
// Workgroups are dispatched round-robin over the 8 XCDs; the whole tiles are
// remapped so that each XCD takes a contiguous run of tiles, grouped 8 row
// tiles deep, whose A and B panels its own L2 shares.
#include "eg_common.h"

#include <algorithm>
#include <mutex>
#include <utility>
#include <vector>

namespace eg {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kGroupM = 8;
constexpr int kXcds = 8;
constexpr int kBK = 32;
constexpr int kStages = 2;

// gemm_x3's tile: 256 x 256 outputs of 2 x 4 wavefronts of 128 x 64; two
// stages of four 256 x 32 bf16 planes, 128 KB of LDS
constexpr int kX3BM = 256, kX3BN = 256, kX3WM = 2, kX3WN = 4;

// What both kernels share: output, tiles and the whole-tile / piece split.
struct Plan {
  int64_t kt0;            // K steps of segment 0
  int64_t kt_total;
  int64_t kt_per_piece;
  int dp_tiles;           // blocks [0, dp_tiles) run whole tiles (logical tiles 0 .. dp_tiles-1)
  int pieces;             // pieces per remaining tile; block dp_tiles + q runs piece q
  int sk_groups;          // > 0: the remaining tiles' K steps in sk_groups contiguous ranges instead
  int64_t sk_units;       //      (tiles - dp_tiles) x kt_total (tile, K step) units split among them
  float* c[2];            // per column group
  int64_t ldc[2];
  float* ws;              // [tiles - dp_tiles][pieces][tile] partial products, or [2 sk_groups][tile]
  int64_t m, n[2];
  int tiles_m, tiles_n0, tiles_n;
  int accumulate;         // 1: C += result
};

struct GemmSeg {
  const __bf16* a_hi;
  const __bf16* a_lo;
  const __bf16* b_hi[2];  // per column group
  const __bf16* b_lo[2];
  int64_t lda, ldb[2];    // in bf16, multiples of 8
  int64_t ktiles;         // K / 32
};

struct GemmArgs {
  GemmSeg seg[2];
  int n_seg;
  Plan p;
};

struct F32Seg {
  const float* a;
  const float* b[2];      // per column group
  int64_t lda, ldb[2];    // in floats, multiples of 4
  int64_t ktiles;         // K / 32
};

struct F32Args {
  F32Seg seg[2];
  int n_seg;
  Plan p;
};

// hi = rne(x), lo = rne(x - hi) for 4 values.
__device__ inline void split4(const float4 v, bf16x4& hi, bf16x4& lo) {
  hi[0] = (__bf16)v.x;
  hi[1] = (__bf16)v.y;
  hi[2] = (__bf16)v.z;
  hi[3] = (__bf16)v.w;
  lo[0] = (__bf16)(v.x - (float)hi[0]);
  lo[1] = (__bf16)(v.y - (float)hi[1]);
  lo[2] = (__bf16)(v.z - (float)hi[2]);
  lo[3] = (__bf16)(v.w - (float)hi[3]);
}

// x [rows, cols] (row stride ld) -> hi, lo [rows, kp] with kp = cols rounded up
// to 32 and the padding zero; blockIdx.y walks rows, each thread 4 values.
// With a third plane lo2 (bf16x6's split): hi, mid = lo as above, and
// lo2 = rne(x - hi - lo) (both differences exact in fp32).
template <bool VEC, bool THREE>
__global__ __launch_bounds__(256) void split_kernel(const float* __restrict__ x, int64_t rows, int64_t cols,
                                                    int64_t ld, int64_t kp, __bf16* __restrict__ hi,
                                                    __bf16* __restrict__ lo, __bf16* __restrict__ lo2) {
  const int64_t c = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (c >= kp) return;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const float* src = x + r * ld + c;
    float4 v;
    if (VEC && c + 3 < cols) {
      v = *(const float4*)src;
    } else {
      v.x = c + 0 < cols ? src[0] : 0.0f;
      v.y = c + 1 < cols ? src[1] : 0.0f;
      v.z = c + 2 < cols ? src[2] : 0.0f;
      v.w = c + 3 < cols ? src[3] : 0.0f;
    }
    bf16x4 h, l;
    split4(v, h, l);
    *(bf16x4*)(hi + r * kp + c) = h;
    *(bf16x4*)(lo + r * kp + c) = l;
    if constexpr (THREE) {
      bf16x4 l2;
      l2[0] = (__bf16)((v.x - (float)h[0]) - (float)l[0]);
      l2[1] = (__bf16)((v.y - (float)h[1]) - (float)l[1]);
      l2[2] = (__bf16)((v.z - (float)h[2]) - (float)l[2]);
      l2[3] = (__bf16)((v.w - (float)h[3]) - (float)l[3]);
      *(bf16x4*)(lo2 + r * kp + c) = l2;
    }
  }
}

// Logical tile -> (row tile, column tile): groups of kGroupM row tiles, each
// group walked column tile by column tile.
__device__ inline void grouped(int logical, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int in_group = kGroupM * tiles_n;
  const int g = logical / in_group;
  const int first_m = g * kGroupM;
  const int gsize = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
  const int r = logical % in_group;
  tm = first_m + r % gsize;
  tn = r / gsize;
}

// The block's work: a whole tile (piece < 0) or piece `piece` of a tile of the
// last round, its K steps [kv0, kv1), and where its output goes.
struct Work {
  int64_t m0, n0, kv0, kv1;
  int grp, piece;
};

// Block b of nb whole-tile blocks -> logical tile: block b runs on XCD b % 8,
// and each XCD takes a contiguous run of tiles.
__device__ inline int xcd_order(int b, int nb) {
  const int x = b % kXcds, i = b / kXcds;
  const int per = nb / kXcds, extra = nb % kXcds;
  return x * per + (x < extra ? x : extra) + i;
}

// The work of one tile (logical index) over K steps [kv0, kv1).
template <int BM, int BN>
__device__ inline Work tile_work(const Plan& p, int logical, int64_t kv0, int64_t kv1, int piece) {
  Work w;
  int tm, tn;
  grouped(logical, p.tiles_m, p.tiles_n, tm, tn);
  w.grp = tn < p.tiles_n0 ? 0 : 1;
  w.m0 = (int64_t)tm * BM;
  w.n0 = (int64_t)(w.grp ? tn - p.tiles_n0 : tn) * BN;
  w.kv0 = kv0;
  w.kv1 = kv1;
  w.piece = piece;
  return w;
}

// Range s of the last round's (tile, K step) units: [U s / G, U (s + 1) / G).
__device__ inline int64_t sk_start(const Plan& p, int64_t s) { return p.sk_units * s / p.sk_groups; }

// D of a 32 x 32 MFMA tile: lane l holds column l % 32 and rows
// 8 (r / 4) + 4 (l / 32) + r % 4; wavefront (wm, wn) holds TI x TJ such
// tiles, the block of 32 TI x 32 TJ outputs at (32 TI wm, 32 TJ wn) of the
// tile.  A whole tile goes to C (bounded by m and n, added to when
// accumulating); a piece to its BM x BN workspace slot.
template <int BM, int BN, int TI, int TJ>
__device__ inline void store_acc(const Plan& p, const Work& w, const f32x16 (&acc)[TI][TJ], int wm, int wn,
                                 int lane) {
  // the store addresses depend on the lane only; an opaque copy of it keeps the
  // compiler from computing them once ahead of a loop over tiles and holding
  // them (in scratch) across the K loops
  asm volatile("" : "+v"(lane));
  const int r0 = wm * 32 * TI, c0 = wn * 32 * TJ;
  if (w.piece >= 0) {
    float* t = p.ws + (int64_t)w.piece * (BM * BN);
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const int lc = c0 + j * 32 + (lane & 31);
#pragma unroll
        for (int r = 0; r < 16; ++r)
          t[(r0 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * BN + lc] = acc[i][j][r];
      }
    return;
  }
  float* out = p.c[w.grp];
  const int64_t ld = p.ldc[w.grp], n_grp = p.n[w.grp];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int64_t col = w.n0 + c0 + j * 32 + (lane & 31);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = w.m0 + r0 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < p.m && col < n_grp) {
          float* q = out + row * ld + col;
          *q = p.accumulate ? *q + acc[i][j][r] : acc[i][j][r];
        }
      }
    }
}

__device__ inline int swz(int row, int chunk) { return chunk ^ ((row >> 2) & 3); }
__device__ inline int swz8(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

// s_waitcnt vmcnt(0), leaving the other counters alone.
__device__ inline void wait_vm0() { __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); }
// s_waitcnt vmcnt(N) (N < 16) and s_waitcnt lgkmcnt(0), each alone.
template <int N>
__device__ inline void wait_vm() {
  static_assert(N >= 0 && N < 16, "vmcnt field");
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8) | N);
}
__device__ inline void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xf | (7 << 4) | (3 << 14)); }

// Both GEMM kernels walk their blocks the same way: every block covers a range
// [u0, u1) of (tile, K step) units from tile `base` on.  A whole tile is
// [0, kt) of its own tile; piece q of the equal cuts is its K steps of tile
// dp_tiles + q / pieces; with ranges (sk_groups > 0), range s of the last
// round covers units [start(s), start(s + 1)) of the tiles from dp_tiles on.
// A range is shorter than a tile's K steps (the last round has fewer tiles
// than there are ranges), so it meets one or two tiles, t0 and t1 = t0 + 1
// from base, and the block runs the two parts one after the other.  A part of
// a tile goes to workspace slot `slot0` + (its tile - t0).  (Written out in
// each kernel: as a shared helper the fp32 kernel ran 10 % slower.)
#define EG_GEMM_WALK(...)                                                                               \
  const Plan& p = args.p;                                                                               \
  const int64_t kt = p.kt_total;                                                                        \
  const int b = (int)blockIdx.x;                                                                        \
  int base, slot0 = 0;                                                                                  \
  int64_t u0 = 0, u1 = kt;                                                                              \
  if (b < p.dp_tiles) {                                                                                 \
    base = xcd_order(b, p.dp_tiles);                                                                    \
  } else if (p.sk_groups == 0) {                                                                        \
    const int q = b - p.dp_tiles;                                                                       \
    base = p.dp_tiles + q / p.pieces;                                                                   \
    u0 = (int64_t)(q % p.pieces) * p.kt_per_piece;                                                      \
    u1 = u0 + p.kt_per_piece < kt ? u0 + p.kt_per_piece : kt;                                           \
    slot0 = q;                                                                                          \
  } else {                                                                                              \
    const int s = b - p.dp_tiles;                                                                       \
    base = p.dp_tiles;                                                                                  \
    u0 = sk_start(p, s);                                                                                \
    u1 = sk_start(p, s + 1);                                                                            \
    slot0 = 2 * s;                                                                                      \
  }                                                                                                     \
  if (u0 >= u1 && !(u0 == 0 && kt == 0)) return; /* an empty range (no K steps still stores zeros) */  \
  const int64_t t0 = kt > 0 ? u0 / kt : 0, t1 = kt > 0 ? (u1 - 1) / kt : 0;                            \
  _Pragma("unroll 1") for (int64_t t = t0; t <= t1; ++t) {                                              \
    const int64_t k0 = (u0 > t * kt ? u0 : t * kt) - t * kt;                                            \
    const int64_t k1 = (u1 < (t + 1) * kt ? u1 : (t + 1) * kt) - t * kt;                                \
    /* whole: a tile of the full rounds, or one that a range covers from end to end */                  \
    const bool whole = (b < p.dp_tiles || p.sk_groups > 0) && k0 == 0 && k1 == kt;                      \
    const Work w = tile_work<BM, BN>(p, base + (int)t, k0, k1, whole ? -1 : slot0 + (int)(t - t0));     \
    __VA_ARGS__;                                                                                        \
  }

// The products a bf16 GEMM launch adds, over the hi and lo planes it loads
// (a pass: A's lo or hi plane times B's lo or hi plane), the small ones first:
//   PR 3 (bf16x3): lo*hi, hi*lo, hi*hi;
//   PR 4: lo*lo, lo*hi, hi*lo, hi*hi (bf16x6 on the hi and mid planes);
//   PR 2: lo*hi, hi*lo (bf16x6 on the hi and lo planes), passes 1 and 2 of PR 4,
//   which is how gemm_x6_kernel runs them (pass set 4 with a run-time mask).
template <int PR>
__device__ constexpr bool pass_alo(int pass) {
  return PR == 4 ? pass < 2 : pass == 0;
}
template <int PR>
__device__ constexpr bool pass_blo(int pass) {
  return PR == 4 ? (pass == 0 || pass == 2) : pass == 1;
}

// gemm_x3: one tile's (or piece's) K steps [w.kv0, w.kv1) and its store.
// BM x BN tile of WMW x WNW wavefronts, each 32 TI x 32 TJ outputs (TI x TJ
// MFMA tiles).  A stage holds the four bf16 planes ah, al (BM rows) and bh, bl
// (BN rows) of 32 k each, 64 B rows, one after the other; the 16-byte chunk c
// of plane row r sits in slot c ^ ((r >> 2) & 3): a fragment read (16 lanes
// at one chunk of 16 consecutive rows per LDS cycle) then touches 16
// distinct 16-byte bank groups (the counter SQ_LDS_BANK_CONFLICT read half of
// SQ_LDS_IDX_ACTIVE with c ^ ((r >> 1) & 3); 2-3 % faster without the
// conflicts).  A direct-to-LDS load fills 16
// rows of a plane (1 KB), so load q of a stage lands at 16 q rows from the
// stage's start.
// A segment's pass set: PR passes of pass_alo / pass_blo; with RT, only the
// passes whose bit is set in a uniform run-time mask run.
template <int PR, bool RT>
struct PassSet {
  static constexpr int value = PR;
  static constexpr bool masked = RT;
};

template <int BM, int BN, int WMW, int WNW, int PR0, int PR1>
__device__ inline void x3_tile(const GemmArgs& args, const Work& w, __bf16* lds) {
  constexpr int NW = WMW * WNW, TI = BM / WMW / 32, TJ = BN / WNW / 32;
  constexpr int LA = BM / 16, LB = BN / 16;         // loads per A / B plane
  constexpr int LPW = 2 * (LA + LB) / NW;           // loads per wavefront per stage
  constexpr int STAGE = 2 * (BM + BN) * kBK;        // bf16
  static_assert(LA % NW == 0 && LB % NW == 0, "a wavefront's j-th load stays in one plane");
  const Plan& p = args.p;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r0 = (wave / WNW) * (BM / WMW), c0 = (wave % WNW) * (BN / WNW);
  const int grp = w.grp;
  const int64_t n_grp = p.n[grp];

  f32x16 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // this wavefront's loads per stage: load q = wave + NW j covers plane
  // plane_of(j) (0 ah, 1 al, 2 bh, 3 bl), rows 16 (q - the plane's first load)
  // .. +15; lane i fills row 16 (..) + i / 4, slot i % 4.  Rows past m or n read
  // row m-1 or n-1: their products only reach outputs that are not stored.
  auto plane_of = [](int j) { return NW * j < LA ? 0 : NW * j < 2 * LA ? 1 : NW * j < 2 * LA + LB ? 2 : 3; };
  auto first_of = [](int pl) { return pl == 0 ? 0 : pl == 1 ? LA : pl == 2 ? 2 * LA : 2 * LA + LB; };
  const int uwave = __builtin_amdgcn_readfirstlane(wave);

  // the block's K steps of segment s, whose products are pass set PR
  auto seg_steps = [&](const int s, auto pass_set, const uint32_t live) {
    constexpr int PR = decltype(pass_set)::value, NP = PR;  // passes (products) a half step
    auto on = [&](int pass) { return !decltype(pass_set)::masked || ((live >> pass) & 1u); };
    const int64_t seg0 = s ? p.kt0 : 0, seg1 = s ? p.kt_total : p.kt0;
    const int64_t lo = w.kv0 > seg0 ? w.kv0 : seg0, hi = w.kv1 < seg1 ? w.kv1 : seg1;
    if (lo >= hi) return;
    const GemmSeg& sg = args.seg[s];
    // a load's address: the plane's base (uniform) + a 32-bit byte offset
    // (the host keeps every plane under 4 GiB), one VGPR a load
    // (from an opaque copy of the lane: computed here for the segment, not once
    // for the tile and held across the K loops, which spilled)
    int ln = lane;
    asm volatile("" : "+v"(ln));
    uint32_t off[LPW];
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      const int pl = plane_of(j), q = uwave + NW * j, row = 16 * (q - first_of(pl)) + (ln >> 2);
      const bool is_a = pl < 2;
      const int64_t gr = (is_a ? w.m0 : w.n0) + row, lim = is_a ? p.m : n_grp;
      const int64_t rr = gr < lim ? gr : lim - 1;
      off[j] = (uint32_t)((rr * (pl < 2 ? sg.lda : sg.ldb[grp]) + swz(row, ln & 3) * 8) * 2);
    }
    auto issue = [&](int64_t kt) {  // K step kt of the segment
      __bf16* st = lds + (kt & 1) * STAGE;
#pragma unroll
      for (int j = 0; j < LPW; ++j) {
        const int pl = plane_of(j), q = uwave + NW * j;
        const __bf16* base = pl == 0 ? sg.a_hi : pl == 1 ? sg.a_lo : pl == 2 ? sg.b_hi[grp] : sg.b_lo[grp];
        __builtin_amdgcn_global_load_lds((const void*)((const char*)(base + kt * kBK) + off[j]),
                                         (__attribute__((address_space(3))) void*)(st + 16 * q * kBK), 16, 0, 0);
      }
    };
    // load j alone: the half step after the barrier issues them one at a time
    // between its MFMAs
    auto issue_one = [&](int64_t kt, int j) {
      __bf16* st = lds + (kt & 1) * STAGE;
      const int pl = plane_of(j), q = uwave + NW * j;
      const __bf16* base = pl == 0 ? sg.a_hi : pl == 1 ? sg.a_lo : pl == 2 ? sg.b_hi[grp] : sg.b_lo[grp];
      __builtin_amdgcn_global_load_lds((const void*)((const char*)(base + kt * kBK) + off[j]),
                                       (__attribute__((address_space(3))) void*)(st + 16 * q * kBK), 16, 0, 0);
    };
    // fragments of half step ks (16 k) of stage kt into set f
    bf16x8 ah[2][TI], al[2][TI], bh[2][TJ], bl[2][TJ];
    auto read = [&](int f, int64_t kt, int ks) {
      const __bf16* st = lds + (kt & 1) * STAGE;
      const int c = ks * 2 + (lane >> 5);
#pragma unroll
      for (int i = 0; i < TI; ++i) {
        const int ar = r0 + i * 32 + (lane & 31);
        const int ao = ar * kBK + swz(ar, c) * 8;
        ah[f][i] = *(const bf16x8*)(st + ao);
        al[f][i] = *(const bf16x8*)(st + BM * kBK + ao);
      }
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const int br = c0 + j * 32 + (lane & 31);
        const int bo = br * kBK + swz(br, c) * 8;
        bh[f][j] = *(const bf16x8*)(st + 2 * BM * kBK + bo);
        bl[f][j] = *(const bf16x8*)(st + (2 * BM + BN) * kBK + bo);
      }
    };
    // the products of set f, the small ones first, a pass over the TI x TJ
    // tiles each (pass_alo / pass_blo: which planes a pass multiplies)
    auto mfma = [&](int f, int pass) {
      if (!on(pass)) return;
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pass_alo<PR>(pass) ? al[f][i] : ah[f][i],
                                                               pass_blo<PR>(pass) ? bl[f][j] : bh[f][j], acc[i][j],
                                                               0, 0, 0);
    };
    // Software pipeline, one barrier a step.  The fragments of one half step
    // are read during the other half step's MFMAs, after its first pass: the
    // compiler's wait for a half step's fragments (it waits for every LDS read
    // issued before it) then comes before the first pass, when only that half
    // step's reads, long issued, are outstanding; and the next reads reuse the
    // registers of the lo*hi pass's lo planes.  The loads of step kt + 2 are
    // issued once every wavefront has read step kt (the barrier in the middle
    // of step kt), a step ahead of their use, spread over the half step after
    // that barrier.
    issue(lo - seg0);
    if (lo + 1 < hi) {
      issue(lo + 1 - seg0);
      wait_vm<LPW>();  // this wavefront's part of the first step is in LDS
    } else {
      wait_vm<0>();
    }
    __builtin_amdgcn_s_barrier();
    read(0, lo - seg0, 0);
    // every step but the last (no branch around the reads)
    for (int64_t kv = lo; kv + 1 < hi; ++kv) {
      const int64_t kt = kv - seg0;
      mfma(0, 0);
      __builtin_amdgcn_sched_barrier(0);  // the reads stay between the passes
      read(1, kt, 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int pass = 1; pass < NP; ++pass) mfma(0, pass);
      __builtin_amdgcn_sched_barrier(0);
      // this wavefront's part of step kt + 1 is in LDS and its reads of step kt
      // are in registers; after the barrier, every wavefront's are
      wait_vm<0>();
      wait_lgkm0();
      __builtin_amdgcn_s_barrier();
      {
        // the second half step's MFMAs (its three passes) with the next half
        // step's fragment reads after the first pass and the loads of step
        // kt + 2 one after every second MFMA: a wavefront's direct-to-LDS loads
        // go out one at a time, and in a burst they held the younger wavefront
        // of each SIMD for ~2,700 cycles without an MFMA (the burst form took
        // 2 % longer a step)
        const bool ld = kv + 2 < hi;
#pragma unroll
        for (int t = 0; t < NP * TI * TJ; ++t) {
          const int pass = t / (TI * TJ), i = (t % (TI * TJ)) / TJ, j = t % TJ;
          if (on(pass))
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pass_alo<PR>(pass) ? al[1][i] : ah[1][i],
                                                               pass_blo<PR>(pass) ? bl[1][j] : bh[1][j], acc[i][j],
                                                               0, 0, 0);
          if (t == TI * TJ - 1) {
            __builtin_amdgcn_sched_barrier(0);
            read(0, kt + 1, 0);
            __builtin_amdgcn_sched_barrier(0);
          }
          if ((t + 1) % 2 == 0 && (t + 1) / 2 - 1 < LPW) {
            __builtin_amdgcn_sched_barrier(0);
            if (ld) issue_one(kt + 2, (t + 1) / 2 - 1);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
    }
    mfma(0, 0);
    read(1, hi - 1 - seg0, 1);
#pragma unroll
    for (int pass = 1; pass < NP; ++pass) mfma(0, pass);
#pragma unroll
    for (int pass = 0; pass < NP; ++pass) mfma(1, pass);
    __builtin_amdgcn_s_barrier();  // the ring is refilled by the next segment or tile
  };
  // segment by segment (the ring drains at a segment change)
  for (int s = 0; s < args.n_seg; ++s) {
    if constexpr (PR0 == PR1)
      seg_steps(s, PassSet<PR0, false>{}, 0u);
    else  // PR0 4, PR1 2: segment 1 runs passes 1 and 2 of the four (lo*hi, hi*lo)
      seg_steps(s, PassSet<4, true>{}, s ? 0x6u : 0xfu);
  }
  store_acc<BM, BN, TI, TJ>(p, w, acc, wave / WNW, wave % WNW, lane);
}

template <int BM, int BN, int WMW, int WNW, int PR>
__global__ __launch_bounds__(WMW * WNW * 64) void gemm_x3_kernel(const GemmArgs args) {
  extern __shared__ __attribute__((aligned(16))) __bf16 lds[];
  EG_GEMM_WALK(x3_tile<BM, BN, WMW, WNW, PR, PR>(args, w, lds))
}

// bf16x6 of one K segment in one launch: segment 0 is its hi and mid planes
// (the four products of pass set 4), segment 1 the same K over its hi and lo
// planes (lo*hi and hi*lo), both into the same accumulators.
template <int BM, int BN, int WMW, int WNW>
__global__ __launch_bounds__(WMW * WNW * 64) void gemm_x6_kernel(const GemmArgs args) {
  extern __shared__ __attribute__((aligned(16))) __bf16 lds[];
  EG_GEMM_WALK((x3_tile<BM, BN, WMW, WNW, 4, 2>(args, w, lds)))
}

// One MFMA takes one A and one B value per lane (lane l: row / column l % 32,
// k = l / 32), so each lane half works through its own 16 k of a step: lane
// half h reads k 16 h .. 16 h + 15 of its row as four 16-byte chunks and the
// 16 MFMAs of the step pair k = kk (half 0) with k = 16 + kk (half 1).  The
// 16-byte chunk c of tile row r sits in slot c ^ ((r >> 1) & 7): a fragment
// read (16 lanes at one chunk of 16 consecutive rows per LDS cycle) then
// touches 16 distinct 16-byte bank groups.  64 MFMAs of 64 cycles a step
// against 16 KB of LDS reads per wavefront: the matrix cores, not the LDS,
// bound it.  BM x BN tile, (BM / 64) x (BN / 64) wavefronts of 64 x 64; A and
// B tiles of BM and BN rows x 128 B a stage.
// One tile's (or piece's) K steps [w.kv0, w.kv1) and its store.
template <int BM, int BN>
__device__ inline void f32_tile(const F32Args& args, const Work& w, float* ldsf) {
  constexpr int WN = BN / 64, NW = (BM / 64) * WN;
  constexpr int STAGE = (BM + BN) * kBK;           // floats
  constexpr int LPW = (BM + BN) / 8 / NW;          // 8-row loads per wavefront per stage
  constexpr int LA = BM / 8 / NW;                  // of which on A
  static_assert((BM / 8) % NW == 0 && (BN / 8) % NW == 0, "loads per wavefront");
  const Plan& p = args.p;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int grp = w.grp;
  const int64_t n_grp = p.n[grp];

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // this wavefront's loads per stage: load q = wave + NW j covers rows 8 q' ..
  // 8 q' + 7 of A (j < LA, q' = q) or B (q' = q - BM / 8); lane i fills row
  // 8 q' + i / 8, slot i % 8.  Rows past m or n read row m-1 or n-1 (not stored).
  const int uwave = __builtin_amdgcn_readfirstlane(wave);

  for (int s = 0; s < args.n_seg; ++s) {
    const int64_t seg0 = s ? p.kt0 : 0, seg1 = s ? p.kt_total : p.kt0;
    const int64_t lo = w.kv0 > seg0 ? w.kv0 : seg0, hi = w.kv1 < seg1 ? w.kv1 : seg1;
    if (lo >= hi) continue;
    const F32Seg& sg = args.seg[s];
    // the load addresses, from an opaque copy of the lane: computed here for the
    // segment rather than once for the tile and held across the K loops (the
    // held form spilled 160 B a lane outside the loop and ran 2-4 % slower)
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const float* src[LPW];
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      const int q = uwave + NW * j, row = 8 * (j < LA ? q : q - BM / 8) + (ln >> 3);
      const int64_t gr = (j < LA ? w.m0 : w.n0) + row, lim = j < LA ? p.m : n_grp;
      src[j] = (j < LA ? sg.a : sg.b[grp]) + (gr < lim ? gr : lim - 1) * (j < LA ? sg.lda : sg.ldb[grp]) +
               swz8(row, ln & 7) * 4;
    }
    auto issue = [&](int64_t kt) {
      float* st = ldsf + (kt & 1) * STAGE;
#pragma unroll
      for (int j = 0; j < LPW; ++j) {
        const int q = uwave + NW * j;
        __builtin_amdgcn_global_load_lds((const void*)(src[j] + kt * kBK),
                                         (__attribute__((address_space(3))) void*)(st + 8 * q * kBK), 16, 0, 0);
      }
    };
    issue(lo - seg0);
    for (int64_t kv = lo; kv < hi; ++kv) {
      const int64_t kt = kv - seg0;
      wait_vm0();
      __builtin_amdgcn_s_barrier();
      const float* st = ldsf + (kt & 1) * STAGE;
      // two halves of the step's 16 k a lane half owns: 8 k (two chunks) of
      // each fragment in registers at a time.  The next step's loads go out
      // after the first half's fragment reads: the wait for them that the
      // compiler puts before the next LDS read (it cannot tell the stages
      // apart) then falls after the first half's MFMAs, not before them.
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        float4 fa[2][2], fb[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int ar = wm * 64 + i * 32 + (lane & 31);
          const int br = wn * 64 + i * 32 + (lane & 31);
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const int chunk = 4 * (lane >> 5) + 2 * half + c;
            fa[i][c] = *(const float4*)(st + ar * kBK + swz8(ar, chunk) * 4);
            fb[i][c] = *(const float4*)(st + BM * kBK + br * kBK + swz8(br, chunk) * 4);
          }
        }
        if (half == 0 && kv + 1 < hi) issue(kt + 1);
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              const float4& av = fa[i][kk >> 2];
              const float4& bv = fb[j][kk >> 2];
              const float x = (kk & 3) == 0 ? av.x : (kk & 3) == 1 ? av.y : (kk & 3) == 2 ? av.z : av.w;
              const float y = (kk & 3) == 0 ? bv.x : (kk & 3) == 1 ? bv.y : (kk & 3) == 2 ? bv.z : bv.w;
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(x, y, acc[i][j], 0, 0, 0);
            }
      }
    }
    __builtin_amdgcn_s_barrier();  // the ring is refilled by the next segment or tile
  }
  store_acc<BM, BN, 2, 2>(p, w, acc, wm, wn, lane);
}

// gemm_f32 over the walk.  The stores' lane addresses are recomputed for
// each part of a range (see store_acc): held across both K loops they spilled
// 62 VGPRs to scratch and cost 4 % on whole tiles.
template <int BM, int BN>
__global__ __launch_bounds__(BM * BN / 64) void gemm_f32_kernel(const F32Args args) {
  extern __shared__ __attribute__((aligned(16))) float ldsf[];
  EG_GEMM_WALK(f32_tile<BM, BN>(args, w, ldsf))
}

// C (+)= the sum of a last-round tile's pieces, in K order: BM BN / 1024
// blocks a tile, each thread four consecutive columns of one row.
template <int BM, int BN>
__global__ __launch_bounds__(256) void piece_sum_kernel(const Plan p) {
  constexpr int kBlocks = BM * BN / 1024;
  const int q = blockIdx.x / kBlocks;
  const int e = (blockIdx.x % kBlocks) * 256 + threadIdx.x;  // float4 of the BM x BN tile
  const int lr = e / (BN / 4), lc = (e % (BN / 4)) * 4;
  int tm, tn;
  grouped(p.dp_tiles + q, p.tiles_m, p.tiles_n, tm, tn);
  const int grp = tn < p.tiles_n0 ? 0 : 1;
  const int64_t row = (int64_t)tm * BM + lr;
  if (row >= p.m) return;
  const float4* ws = (const float4*)(p.ws + (int64_t)q * p.pieces * (BM * BN)) + e;
  float4 v = ws[0];
  for (int s = 1; s < p.pieces; ++s) {
    const float4 u = ws[(int64_t)s * (BM * BN / 4)];
    v.x += u.x;
    v.y += u.y;
    v.z += u.z;
    v.w += u.w;
  }
  const int64_t n_grp = p.n[grp], col0 = (int64_t)(grp ? tn - p.tiles_n0 : tn) * BN + lc;
  float* out = p.c[grp] + row * p.ldc[grp];
  const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int64_t col = col0 + t;
    if (col < n_grp) out[col] = p.accumulate ? out[col] + vv[t] : vv[t];
  }
}

// C (+)= the sum, in K order, of the parts of a last-round tile that the
// ranges of gemm_f32_kernel computed: the ranges meeting the tile, in
// increasing order (a tile one range covers whole was stored directly).
// BM BN / 1024 blocks a tile, four columns a thread.
template <int BM, int BN>
__global__ __launch_bounds__(256) void sk_sum_kernel(const Plan p) {
  constexpr int kBlocks = BM * BN / 1024;
  const int q = blockIdx.x / kBlocks;  // last-round tile
  const int e = (blockIdx.x % kBlocks) * 256 + threadIdx.x;
  const int lr = e / (BN / 4), lc = (e % (BN / 4)) * 4;
  const int64_t kt = p.kt_total, x0 = (int64_t)q * kt, x1 = x0 + kt;
  // the range holding unit x0: the last s with start(s) <= x0 (skips empty ranges)
  int64_t s = x0 * p.sk_groups / p.sk_units;
  while (s > 0 && sk_start(p, s) > x0) --s;
  while (s + 1 < p.sk_groups && sk_start(p, s + 1) <= x0) ++s;
  if (sk_start(p, s + 1) >= x1) return;  // one range covers the tile: stored directly
  int tm, tn;
  grouped(p.dp_tiles + q, p.tiles_m, p.tiles_n, tm, tn);
  const int grp = tn < p.tiles_n0 ? 0 : 1;
  const int64_t row = (int64_t)tm * BM + lr;
  if (row >= p.m) return;
  float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  bool first = true;
  for (; s < p.sk_groups; ++s) {
    const int64_t a = sk_start(p, s);
    if (a >= x1) break;
    if (a == sk_start(p, s + 1)) continue;  // empty range
    const int slot = 2 * (int)s + (int)(q - a / kt);
    const float4 u = *((const float4*)(p.ws + (int64_t)slot * (BM * BN)) + e);
    if (first) {
      v = u;
      first = false;
    } else {
      v.x += u.x;
      v.y += u.y;
      v.z += u.z;
      v.w += u.w;
    }
  }
  const int64_t n_grp = p.n[grp], col0 = (int64_t)(grp ? tn - p.tiles_n0 : tn) * BN + lc;
  float* out = p.c[grp] + row * p.ldc[grp];
  const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int64_t col = col0 + t;
    if (col < n_grp) out[col] = p.accumulate ? out[col] + vv[t] : vv[t];
  }
}

// ---------------------------------------------------------------------------
// Host side

struct PiecePlan {
  int dp;              // whole tiles
  int pieces;          // pieces per remaining tile
  int64_t kt_per_piece;
  int sk_groups;       // > 0: the remaining tiles' K steps in this many contiguous ranges instead of pieces
};

// A kernel's tile: BM x BN outputs of `threads` threads and `lds` bytes of
// LDS.  The plan counts `rounds_per_cu` tiles a CU as one round (one for
// both kernels' 256 x 256 tiles, whose LDS holds one workgroup a CU).
// `sum_cost` / (K steps) is the time of summing one round of pieces against
// the time of one round of tiles: 4 bytes read per output and piece at ~5
// TB/s against 192 (bf16 products, ~1 PFLOP/s reached) or 64 (fp32, ~130
// TFLOP/s) flops per output and K step.
// `ranges`: the kernel can take the last round as contiguous K ranges, one per
// workgroup of the round (gemm_f32_kernel), rather than as equal pieces of each
// tile.
struct Shape {
  int bm, bn, threads, rounds_per_cu;
  size_t lds;
  double sum_cost;
  bool ranges;
};

constexpr Shape kX3Shape{kX3BM, kX3BN, kX3WM * kX3WN * 64, 1, (size_t)kStages * 2 * (kX3BM + kX3BN) * kBK * 2, 4.2,
                         true};
constexpr int kF32BM = 256, kF32BN = 256;
constexpr Shape kF32Shape{kF32BM, kF32BN, kF32BM * kF32BN / 64, 1,
                          (size_t)kStages * (kF32BM + kF32BN) * kBK * 4, 1.6, true};

// k_slices >= 1: every tile in k_slices pieces (1: whole tiles).  0: the
// tiles of a partly filled last round (of `slots` tiles) in the piece count
// that minimises the time of that round in tile units, ceil(R s / slots) / s,
// plus the cost of summing the pieces, sum_cost / (K steps) per round of
// pieces.  At least 8 K steps a piece, and only for a gain of 10 % or more.
PiecePlan plan_pieces(int64_t tiles, int64_t kt_total, int k_slices, int slots, double sum_cost) {
  PiecePlan pp{(int)tiles, 1, kt_total > 0 ? kt_total : 1, 0};
  int s = 1;
  if (k_slices >= 1) {
    s = k_slices;
  } else {
    const int64_t r = tiles % slots;
    if (r == 0 || kt_total < 16) return pp;
    const double per_round = sum_cost / (double)kt_total;
    double best = 1.0;
    for (int c = 2; c <= 8 && kt_total / c >= 8; ++c) {
      const double t = (double)((r * c + slots - 1) / slots) / c + per_round * (double)(r * c) / slots;
      if (t < best) {
        best = t;
        s = c;
      }
    }
    if (best > 0.9) return pp;
  }
  if (kt_total < s) s = kt_total > 0 ? (int)kt_total : 1;
  if (s <= 1) return pp;
  pp.kt_per_piece = (kt_total + s - 1) / s;
  pp.pieces = (int)((kt_total + pp.kt_per_piece - 1) / pp.kt_per_piece);
  if (pp.pieces <= 1) {
    pp.pieces = 1;
    pp.kt_per_piece = kt_total;
    return pp;
  }
  pp.dp = k_slices >= 1 ? 0 : (int)(tiles - tiles % slots);
  return pp;
}

// CUs of the current device.
int device_cus(int* cus_out) {
  static std::mutex mu;
  static std::vector<std::pair<int, int>> known;  // (device, CU count)
  int dev = 0;
  EG_CHECK_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(mu);
  for (const auto& k : known)
    if (k.first == dev) {
      *cus_out = k.second;
      return EG_OK;
    }
  int cus = 0;
  EG_CHECK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  EG_CHECK_ARG(cus > 0, "device %d reports %d CUs", dev, cus);
  known.emplace_back(dev, cus);
  *cus_out = cus;
  return EG_OK;
}

int64_t tiles_of(const Shape& sh, int64_t m, int64_t n, int64_t n2) {
  return ((m + sh.bm - 1) / sh.bm) * ((n + sh.bn - 1) / sh.bn + (n2 + sh.bn - 1) / sh.bn);
}

int64_t piece_bytes(const Shape& sh, int64_t tiles, const PiecePlan& pp) {
  const int64_t tile = (int64_t)sh.bm * sh.bn * (int64_t)sizeof(float);
  if (pp.sk_groups > 0) return 2 * (int64_t)pp.sk_groups * tile;
  return pp.pieces > 1 ? (tiles - pp.dp) * pp.pieces * tile : 0;
}

int plan_for(const Shape& sh, int64_t m, int64_t n, int64_t n2, int64_t kt_total, int k_slices, int64_t* tiles,
             PiecePlan* pp) {
  int cus = 0;
  const int rc = device_cus(&cus);
  if (rc != EG_OK) return rc;
  *tiles = tiles_of(sh, m, n, n2);
  const int slots = sh.rounds_per_cu * cus;
  *pp = plan_pieces(*tiles, kt_total, k_slices, slots, sh.sum_cost);
  // a kernel that takes ranges: the last round that the plan cuts runs as one
  // contiguous range of its (tile, K step) units per workgroup slot, at least
  // 8 K steps a range (fewer pieces than equal cuts, and no tile cut more
  // often than the ranges meeting it)
  const int64_t r = *tiles - pp->dp;
  if (sh.ranges && k_slices == 0 && pp->pieces > 1 && r < slots && r * kt_total >= 8 * (int64_t)slots) {
    pp->pieces = 1;
    pp->kt_per_piece = kt_total;
    pp->sk_groups = slots;
  }
  return EG_OK;
}

int64_t workspace_size(const Shape& sh, int64_t m, int64_t n, int64_t n2, int64_t k, int32_t k_slices) {
  if (m <= 0 || n < 0 || n2 < 0 || n + n2 == 0 || k < 0 || k_slices < 0) return 0;
  int64_t tiles = 0;
  PiecePlan pp{};
  if (plan_for(sh, m, n, n2, k / 32, k_slices, &tiles, &pp) != EG_OK) return -1;
  return piece_bytes(sh, tiles, pp);
}

// The part of both entry points after their operands are checked: the plan,
// the LDS attribute, the launch and the pieces' sum.
template <int BM, int BN, typename Args>
int launch_gemm(const Shape& sh, void (*kernel)(const Args), const char* name, Args& g, int64_t m, int64_t n,
                int64_t n2, float* c, int64_t ldc, float* c2, int64_t ldc2, int32_t accumulate, int32_t k_slices,
                void* workspace, int64_t workspace_bytes, void* stream) {
  EG_CHECK_ARG(m >= 0 && n >= 0 && n2 >= 0 && k_slices >= 0, "m=%lld n=%lld n2=%lld k_slices=%d", (long long)m,
               (long long)n, (long long)n2, k_slices);
  EG_CHECK_ARG(n == 0 || (c != nullptr && ldc >= n), "c / ldc");
  EG_CHECK_ARG(n2 == 0 || (c2 != nullptr && ldc2 >= n2), "c2 / ldc2");
  if (m == 0 || n + n2 == 0) return 0;
  Plan& p = g.p;
  p.kt0 = g.n_seg > 0 ? g.seg[0].ktiles : 0;
  p.kt_total = p.kt0 + (g.n_seg > 1 ? g.seg[1].ktiles : 0);
  int64_t tiles = 0;
  PiecePlan pp{};
  int rc = plan_for(sh, m, n, n2, p.kt_total, k_slices, &tiles, &pp);
  if (rc != EG_OK) return rc;
  EG_CHECK_ARG(tiles < (1LL << 24), "too many tiles");
  const int64_t need = piece_bytes(sh, tiles, pp);
  if (need > 0) {
    EG_CHECK_ARG(workspace != nullptr && ((uintptr_t)workspace & 15) == 0 && workspace_bytes >= need,
                 "this call needs a 16-byte aligned workspace of %lld bytes (its _workspace_size function)",
                 (long long)need);
    p.ws = (float*)workspace;
  }
  p.dp_tiles = pp.dp;
  p.pieces = pp.pieces;
  p.kt_per_piece = pp.kt_per_piece;
  p.sk_groups = pp.sk_groups;
  p.sk_units = pp.sk_groups > 0 ? (tiles - pp.dp) * p.kt_total : 0;
  p.c[0] = c;
  p.c[1] = c2;
  p.ldc[0] = ldc;
  p.ldc[1] = ldc2;
  p.m = m;
  p.n[0] = n;
  p.n[1] = n2;
  p.tiles_m = (int)((m + BM - 1) / BM);
  p.tiles_n0 = (int)((n + BN - 1) / BN);
  p.tiles_n = p.tiles_n0 + (int)((n2 + BN - 1) / BN);
  p.accumulate = accumulate ? 1 : 0;
  const int64_t blocks = pp.dp + (pp.sk_groups > 0 ? (int64_t)pp.sk_groups : (tiles - pp.dp) * pp.pieces);
  EG_CHECK_ARG(blocks < (1LL << 31), "too many workgroups");
  hipStream_t st = (hipStream_t)stream;
  // the dynamic LDS attribute, once per device and kernel
  static std::mutex mu;
  static std::vector<std::pair<const void*, int>> done;
  int dev = 0;
  EG_CHECK_HIP(hipGetDevice(&dev));
  {
    std::lock_guard<std::mutex> lock(mu);
    const std::pair<const void*, int> key((const void*)kernel, dev);
    if (std::find(done.begin(), done.end(), key) == done.end()) {
      EG_CHECK_HIP(hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)sh.lds));
      done.push_back(key);
    }
  }
  hipLaunchKernelGGL(kernel, dim3((unsigned)blocks), dim3(sh.threads), sh.lds, st, g);
  rc = launch_status(name);
  if (rc != 0 || pp.dp == tiles) return rc;
  const dim3 sum_grid((unsigned)((tiles - pp.dp) * (BM * BN / 1024)));
  if (pp.sk_groups > 0) {
    hipLaunchKernelGGL((sk_sum_kernel<BM, BN>), sum_grid, dim3(256), 0, st, p);
    return launch_status("sk_sum_kernel");
  }
  hipLaunchKernelGGL((piece_sum_kernel<BM, BN>), sum_grid, dim3(256), 0, st, p);
  return launch_status("piece_sum_kernel");
}

}  // namespace
}  // namespace eg

extern "C" {

}  // extern "C"

namespace eg {
namespace {
// eg_split_bf16 (lo2 == nullptr) and eg_split_bf16x6.
int split_planes(const float* x, int64_t rows, int64_t cols, int64_t ld, void* hi, void* lo, void* lo2,
                 void* stream) {
  EG_CHECK_ARG(rows >= 0 && cols >= 0 && ld >= cols, "rows=%lld cols=%lld ld=%lld", (long long)rows, (long long)cols,
               (long long)ld);
  const int64_t kp = (cols + 31) / 32 * 32;
  if (rows == 0 || kp == 0) return 0;
  EG_CHECK_ARG(x != nullptr && hi != nullptr && lo != nullptr, "NULL argument");
  EG_CHECK_ARG(((uintptr_t)hi & 15) == 0 && ((uintptr_t)lo & 15) == 0 && ((uintptr_t)lo2 & 15) == 0,
               "the planes must be 16-byte aligned");
  const dim3 grid((unsigned)((kp / 4 + 255) / 256), (unsigned)(rows < 65535 ? rows : 65535));
  const bool vec = ld % 4 == 0 && ((uintptr_t)x & 15) == 0;
  hipStream_t st = (hipStream_t)stream;
  __bf16 *h = (__bf16*)hi, *l = (__bf16*)lo, *l2 = (__bf16*)lo2;
  if (lo2 != nullptr) {
    if (vec) hipLaunchKernelGGL((split_kernel<true, true>), grid, dim3(256), 0, st, x, rows, cols, ld, kp, h, l, l2);
    else hipLaunchKernelGGL((split_kernel<false, true>), grid, dim3(256), 0, st, x, rows, cols, ld, kp, h, l, l2);
  } else {
    if (vec) hipLaunchKernelGGL((split_kernel<true, false>), grid, dim3(256), 0, st, x, rows, cols, ld, kp, h, l, l2);
    else hipLaunchKernelGGL((split_kernel<false, false>), grid, dim3(256), 0, st, x, rows, cols, ld, kp, h, l, l2);
  }
  return launch_status("split_kernel");
}
}  // namespace
}  // namespace eg

extern "C" {

int eg_split_bf16(const float* x, int64_t rows, int64_t cols, int64_t ld, void* hi, void* lo, void* stream) {
  return eg::split_planes(x, rows, cols, ld, hi, lo, nullptr, stream);
}

int eg_split_bf16x6(const float* x, int64_t rows, int64_t cols, int64_t ld, void* hi, void* mid, void* lo,
                    void* stream) {
  EG_CHECK_ARG(lo != nullptr, "NULL argument");
  return eg::split_planes(x, rows, cols, ld, hi, mid, lo, stream);
}

int64_t eg_gemm_workspace_size(int64_t m, int64_t n, int64_t n2, int64_t k, int32_t k_slices) {
  return eg::workspace_size(eg::kX3Shape, m, n, n2, k, k_slices);
}

int64_t eg_gemm_f32_workspace_size(int64_t m, int64_t n, int64_t n2, int64_t k, int32_t k_slices) {
  return eg::workspace_size(eg::kF32Shape, m, n, n2, k, k_slices);
}

}  // extern "C"

namespace eg {
namespace {
// The kernel arguments of eg_gemm_bf16x3 / eg_gemm_bf16x6 operands (the planes checked).
int bf16_operands(const eg_gemm_operands* ops, int32_t n_seg, int64_t m, int64_t n, int64_t n2, GemmArgs& g) {
  EG_CHECK_ARG(ops != nullptr && n_seg >= 0 && n_seg <= 2, "n_seg=%d", n_seg);
  for (int s = 0; s < n_seg; ++s) {
    const eg_gemm_operands& o = ops[s];
    EG_CHECK_ARG(o.k >= 0 && o.k % 32 == 0, "segment %d: k must be a multiple of 32 (k=%lld)", s, (long long)o.k);
    if (o.k == 0) continue;
    const void* planes[6] = {o.a_hi, o.a_lo, o.b_hi, o.b_lo, o.b2_hi, o.b2_lo};
    for (int q = 0; q < 6; ++q) {
      if (q >= 4 && n2 == 0) break;
      EG_CHECK_ARG(planes[q] != nullptr && ((uintptr_t)planes[q] & 15) == 0,
                   "segment %d: plane %d is NULL or not 16-byte aligned", s, q);
    }
    EG_CHECK_ARG(o.lda % 8 == 0 && o.ldb % 8 == 0 && o.lda >= o.k && o.ldb >= o.k &&
                     (n2 == 0 || (o.ldb2 % 8 == 0 && o.ldb2 >= o.k)),
                 "segment %d: leading dimensions must be multiples of 8 and >= k", s);
    // the kernel addresses a row's 16-byte chunks by 32-bit byte offsets from the plane's start
    auto fits = [](int64_t rows, int64_t ld) { return rows <= 0 || ((rows - 1) * ld + 32) * 2 <= 0xffffffffLL; };
    EG_CHECK_ARG(fits(m, o.lda) && fits(n, o.ldb) && (n2 == 0 || fits(n2, o.ldb2)),
                 "segment %d: a bf16 plane spans 4 GiB or more", s);
    GemmSeg& sg = g.seg[g.n_seg];
    sg.a_hi = (const __bf16*)o.a_hi;
    sg.a_lo = (const __bf16*)o.a_lo;
    sg.b_hi[0] = (const __bf16*)o.b_hi;
    sg.b_lo[0] = (const __bf16*)o.b_lo;
    sg.b_hi[1] = (const __bf16*)(n2 ? o.b2_hi : o.b_hi);
    sg.b_lo[1] = (const __bf16*)(n2 ? o.b2_lo : o.b_lo);
    sg.lda = o.lda;
    sg.ldb[0] = o.ldb;
    sg.ldb[1] = n2 ? o.ldb2 : o.ldb;
    sg.ktiles = o.k / 32;
    ++g.n_seg;
  }
  return EG_OK;
}
}  // namespace
}  // namespace eg

extern "C" {

int eg_gemm_bf16x3(const eg_gemm_operands* ops, int32_t n_seg, int64_t m, int64_t n, int64_t n2, float* c,
                   int64_t ldc, float* c2, int64_t ldc2, int32_t accumulate, int32_t k_slices, void* workspace,
                   int64_t workspace_bytes, void* stream) {
  using namespace eg;
  GemmArgs g{};
  const int rc = bf16_operands(ops, n_seg, m, n, n2, g);
  if (rc != EG_OK) return rc;
  return launch_gemm<kX3BM, kX3BN>(kX3Shape, gemm_x3_kernel<kX3BM, kX3BN, kX3WM, kX3WN, 3>, "gemm_x3_kernel", g, m, n,
                                   n2, c, ldc, c2, ldc2, accumulate, k_slices, workspace, workspace_bytes,
                                   stream);
}

int eg_gemm_bf16x6(const eg_gemm_operands* hi_mid, const eg_gemm_operands* hi_lo, int32_t n_seg, int64_t m,
                   int64_t n, int64_t n2, float* c, int64_t ldc, float* c2, int64_t ldc2, int32_t accumulate,
                   int32_t k_slices, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace eg;
  GemmArgs g1{}, g2{};
  int rc = bf16_operands(hi_mid, n_seg, m, n, n2, g1);
  if (rc != EG_OK) return rc;
  rc = bf16_operands(hi_lo, n_seg, m, n, n2, g2);
  if (rc != EG_OK) return rc;
  bool same = g1.n_seg == g2.n_seg;
  for (int s = 0; same && s < g1.n_seg; ++s) same = g1.seg[s].ktiles == g2.seg[s].ktiles;
  EG_CHECK_ARG(same, "hi_mid and hi_lo must describe the same K segments");
  // One K segment: the six products in one launch, the hi / lo planes as a
  // second segment over the same K (one last round and one sum of its parts;
  // 12 % faster on the PLE key + value), when the workspace covers that
  // launch's plan.  Two K segments keep two launches: one launch's last round
  // of ranges, all of the backward's tiles, mixes steps of four and of two
  // products unevenly (4 % slower).
  if (g1.n_seg == 1) {
    GemmArgs g = g1;
    g.seg[1] = g2.seg[0];
    g.n_seg = 2;
    const int64_t need = workspace_size(kX3Shape, m, n, n2, 2 * 32 * g1.seg[0].ktiles, k_slices);
    if (need >= 0 && workspace_bytes >= need)
      return launch_gemm<kX3BM, kX3BN>(kX3Shape, gemm_x6_kernel<kX3BM, kX3BN, kX3WM, kX3WN>, "gemm_x6_kernel", g, m,
                                       n, n2, c, ldc, c2, ldc2, accumulate, k_slices, workspace, workspace_bytes,
                                       stream);
  }
  // lo*lo + lo*hi + hi*lo + hi*hi over the hi and mid planes, then lo*hi + hi*lo
  // over the hi and lo planes, added to it
  rc = launch_gemm<kX3BM, kX3BN>(kX3Shape, gemm_x3_kernel<kX3BM, kX3BN, kX3WM, kX3WN, 4>, "gemm_x3_kernel<4>", g1,
                                 m, n, n2, c, ldc, c2, ldc2, accumulate, k_slices, workspace, workspace_bytes,
                                 stream);
  if (rc != EG_OK) return rc;
  return launch_gemm<kX3BM, kX3BN>(kX3Shape, gemm_x3_kernel<kX3BM, kX3BN, kX3WM, kX3WN, 2>, "gemm_x3_kernel<2>", g2,
                                   m, n, n2, c, ldc, c2, ldc2, 1, k_slices, workspace, workspace_bytes, stream);
}

int eg_gemm_f32(const eg_gemm_f32_operands* ops, int32_t n_seg, int64_t m, int64_t n, int64_t n2, float* c,
                int64_t ldc, float* c2, int64_t ldc2, int32_t accumulate, int32_t k_slices, void* workspace,
                int64_t workspace_bytes, void* stream) {
  using namespace eg;
  EG_CHECK_ARG(ops != nullptr && n_seg >= 0 && n_seg <= 2, "n_seg=%d", n_seg);
  F32Args g{};
  for (int s = 0; s < n_seg; ++s) {
    const eg_gemm_f32_operands& o = ops[s];
    EG_CHECK_ARG(o.k >= 0 && o.k % 32 == 0, "segment %d: k must be a multiple of 32 (k=%lld)", s, (long long)o.k);
    if (o.k == 0) continue;
    const float* mats[3] = {o.a, o.b, o.b2};
    for (int q = 0; q < 3; ++q) {
      if (q == 2 && n2 == 0) break;
      EG_CHECK_ARG(mats[q] != nullptr && ((uintptr_t)mats[q] & 15) == 0,
                   "segment %d: operand %d is NULL or not 16-byte aligned", s, q);
    }
    EG_CHECK_ARG(o.lda % 4 == 0 && o.ldb % 4 == 0 && o.lda >= o.k && o.ldb >= o.k &&
                     (n2 == 0 || (o.ldb2 % 4 == 0 && o.ldb2 >= o.k)),
                 "segment %d: leading dimensions must be multiples of 4 and >= k", s);
    F32Seg& sg = g.seg[g.n_seg];
    sg.a = o.a;
    sg.b[0] = o.b;
    sg.b[1] = n2 ? o.b2 : o.b;
    sg.lda = o.lda;
    sg.ldb[0] = o.ldb;
    sg.ldb[1] = n2 ? o.ldb2 : o.ldb;
    sg.ktiles = o.k / 32;
    ++g.n_seg;
  }
  return launch_gemm<kF32BM, kF32BN>(kF32Shape, gemm_f32_kernel<kF32BM, kF32BN>, "gemm_f32_kernel", g, m, n, n2,
                                     c, ldc, c2, ldc2, accumulate, k_slices, workspace, workspace_bytes, stream);
}

}  // extern "C"
