// fp32 GEMM on the bf16 matrix cores, three products per operand pair:
//
//   C[M, N] (+)= A[M, K] B[N, K]^T  (+ A2[M, K2] B2[N, K2]^T)
//
// Each fp32 operand is split once (eg_split_bf16) into bf16 planes hi = rne(x)
// and lo = rne(x - hi) (x - hi is exact in fp32), and C accumulates
// hi*hi + hi*lo + lo*hi in fp32 on v_mfma_f32_32x32x16_bf16.  hi + lo keeps
// 16 of fp32's 24 mantissa bits, so each product carries a relative error up
// to ~3 x 2^-18 (fp32's own is 2^-24): about 1e-5 of the result on random
// data, at the bf16 rate.  This runs the PLE block's
// projections (engraft/replica/layers.py:594-606: key = emb w_key^T and
// value = emb w_value^T in one launch, as two column groups over the same A,
// and their backward d_emb = d_key w_key + d_value w_value as two K segments
// with the weights' transposes kept row-major).
//
// Tiling: 128 x 128 output tile per 256-thread workgroup (four wavefronts,
// 64 x 64 each as 2 x 2 MFMA tiles), K in steps of 32 through a two-stage LDS
// ring filled by direct-to-LDS loads (global_load_lds_dwordx4: lane i of a
// wavefront writes 16 bytes at the wavefront's LDS base + 16 i), so the next
// step's loads are in flight during the current step's MFMAs without passing
// through registers.  A plane tile is rows x 32 bf16 (64 B rows, no padding);
// the 16-byte chunk c of row r sits in slot c ^ ((r >> 1) & 3), which spreads
// the fragment reads (32 rows at one chunk) over the banks.  Two stages (64 KB)
// keep two workgroups on a CU.  Measured against it after a warm-up, launches
// interleaved: 128 x 256 and 256 x 128 tiles with eight wavefronts, 256 x 256
// with sixteen, three stages, and scheduling hints that interleave the LDS
// reads with the MFMAs ran 3-5 % slower; register-staged loads into a padded
// LDS tile ran 20 % slower.  With few
// output tiles (the backward's 16 x 20) the K range is cut into slices whose
// partial products go to a workspace and are summed in slice order by a
// second kernel, so the result does not depend on scheduling.
//
// Workgroups are dispatched round-robin over the 8 XCDs; the tile order is
// remapped so that each XCD takes a contiguous run of tiles, grouped 8 row
// tiles deep, whose A and B panels its own L2 shares.
#include "eg_common.h"

namespace eg {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kGroupM = 8;
constexpr int kXcds = 8;
constexpr int kBM = 128, kBN = 128, kBK = 32;
constexpr int kPlane = 128 * kBK;   // bf16 per plane tile
constexpr int kStage = 4 * kPlane;  // ah, al, bh, bl
constexpr int kStages = 2;
constexpr size_t kLds = (size_t)kStages * kStage * 2;  // 64 KB

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
  int64_t kt0;            // K tiles of segment 0
  int64_t kt_total;
  int64_t kt_per_slice;
  int slices;
  float* c[2];            // per column group (slices == 1)
  int64_t ldc[2];
  float* ws;              // slices > 1: [slices, m, n[0] + n[1]] partial products
  int64_t m, n[2];
  int tiles_m, tiles_n0, tiles_n;
  int accumulate;         // 1: C += result (slices == 1)
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
template <bool VEC>
__global__ __launch_bounds__(256) void split_kernel(const float* __restrict__ x, int64_t rows, int64_t cols,
                                                    int64_t ld, int64_t kp, __bf16* __restrict__ hi,
                                                    __bf16* __restrict__ lo) {
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
  }
}

// Workgroup b -> output tile: XCD-contiguous runs, then groups of kGroupM row tiles.
__device__ inline void tile_of(int b, int nb, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int x = b % kXcds, i = b / kXcds;
  const int per = nb / kXcds, extra = nb % kXcds;
  const int logical = x * per + (x < extra ? x : extra) + i;
  const int in_group = kGroupM * tiles_n;
  const int g = logical / in_group;
  const int first_m = g * kGroupM;
  const int gsize = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
  const int r = logical % in_group;
  tm = first_m + r % gsize;
  tn = r / gsize;
}

__device__ inline int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 3); }

// s_waitcnt vmcnt(0), leaving the other counters alone.
__device__ inline void wait_vm0() { __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); }

__global__ __launch_bounds__(256) void gemm_x3_kernel(const GemmArgs args) {
  extern __shared__ __attribute__((aligned(16))) __bf16 lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  int tm, tn;
  tile_of(blockIdx.x, gridDim.x, args.tiles_m, args.tiles_n, tm, tn);
  const int grp = tn < args.tiles_n0 ? 0 : 1;
  const int64_t m0 = (int64_t)tm * kBM, n0 = (int64_t)(grp ? tn - args.tiles_n0 : tn) * kBN;
  const int64_t n_grp = args.n[grp];

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // this wavefront's 8 loads per stage: load q = wave + 4 j covers plane q / 8
  // (ah, al, bh, bl), rows 16 (q % 8) .. +15; lane i fills row 16 (q % 8) + i / 4,
  // slot i % 4.  Rows past m or n read row m-1 or n-1: their products only reach
  // outputs that are not stored.
  const int uwave = __builtin_amdgcn_readfirstlane(wave);
  int64_t row_of[8];
  int col_of[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int q = uwave + 4 * j, plane = q >> 3, row = 16 * (q & 7) + (lane >> 2);
    const bool is_a = plane < 2;
    const int64_t gr = (is_a ? m0 : n0) + row, lim = is_a ? args.m : n_grp;
    row_of[j] = gr < lim ? gr : lim - 1;
    col_of[j] = swz(row, lane & 3) * 8;
  }

  // the slice's K steps, segment by segment (the ring drains at a segment change)
  const int64_t kv0 = (int64_t)blockIdx.y * args.kt_per_slice;
  const int64_t kv1 = kv0 + args.kt_per_slice < args.kt_total ? kv0 + args.kt_per_slice : args.kt_total;
  for (int s = 0; s < args.n_seg; ++s) {
    const int64_t seg0 = s ? args.kt0 : 0, seg1 = s ? args.kt_total : args.kt0;
    const int64_t lo = kv0 > seg0 ? kv0 : seg0, hi = kv1 < seg1 ? kv1 : seg1;
    if (lo >= hi) continue;
    const GemmSeg& sg = args.seg[s];
    const __bf16* src[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int plane = (uwave + 4 * j) >> 3;
      const __bf16* base = plane == 0 ? sg.a_hi : plane == 1 ? sg.a_lo : plane == 2 ? sg.b_hi[grp] : sg.b_lo[grp];
      const int64_t ld = plane < 2 ? sg.lda : sg.ldb[grp];
      src[j] = base + row_of[j] * ld + col_of[j];
    }
    auto issue = [&](int64_t kt) {  // K step kt of the segment
      __bf16* st = lds + (kt & 1) * kStage;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int q = uwave + 4 * j;
        __builtin_amdgcn_global_load_lds((const void*)(src[j] + kt * kBK),
                                         (__attribute__((address_space(3))) void*)(st + (q >> 3) * kPlane +
                                                                                   16 * (q & 7) * kBK),
                                         16, 0, 0);
      }
    };
    issue(lo - seg0);
    for (int64_t kv = lo; kv < hi; ++kv) {
      const int64_t kt = kv - seg0;
      wait_vm0();  // this wavefront's part of step kt is in LDS
      // every wavefront's part is in, and step kt-1 is no longer read.  A bare
      // s_barrier: no other memory operation needs ordering here.
      __builtin_amdgcn_s_barrier();
      if (kv + 1 < hi) issue(kt + 1);
      const __bf16* st = lds + (kt & 1) * kStage;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int c = ks * 2 + (lane >> 5);
        bf16x8 ah[2], al[2], bh[2], bl[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int ar = wm * 64 + i * 32 + (lane & 31);
          const int ao = ar * kBK + swz(ar, c) * 8;
          ah[i] = *(const bf16x8*)(st + ao);
          al[i] = *(const bf16x8*)(st + kPlane + ao);
          const int br = wn * 64 + i * 32 + (lane & 31);
          const int bo = br * kBK + swz(br, c) * 8;
          bh[i] = *(const bf16x8*)(st + 2 * kPlane + bo);
          bl[i] = *(const bf16x8*)(st + 3 * kPlane + bo);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[i], bh[j], acc[i][j], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bl[j], acc[i][j], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bh[j], acc[i][j], 0, 0, 0);
      }
    }
    __builtin_amdgcn_s_barrier();  // the ring is refilled by the next segment
  }

  // D of a 32 x 32 tile: lane l holds column l % 32 and rows 8 (r / 4) + 4 (l / 32) + r % 4
  const int64_t n_all = args.n[0] + args.n[1];
  float* out = args.slices > 1 ? args.ws + (int64_t)blockIdx.y * args.m * n_all + (grp ? args.n[0] : 0)
                               : args.c[grp];
  const int64_t ld_out = args.slices > 1 ? n_all : args.ldc[grp];
  const bool add = args.slices == 1 && args.accumulate;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = n0 + wn * 64 + j * 32 + (lane & 31);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < args.m && col < n_grp) {
          float* p = out + row * ld_out + col;
          *p = add ? *p + acc[i][j][r] : acc[i][j][r];
        }
      }
    }
}

// C (+)= the sum of the slices' partial products, in slice order.
__global__ __launch_bounds__(256) void slice_sum_kernel(const float* __restrict__ ws, int slices, int64_t m,
                                                        int64_t n0, int64_t n1, float* c0, int64_t ldc0, float* c1,
                                                        int64_t ldc1, int accumulate) {
  const int64_t n_all = n0 + n1, total = m * n_all;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t row = i / n_all, col = i % n_all;
    float v = ws[i];
    for (int s = 1; s < slices; ++s) v += ws[s * total + i];
    float* p = col < n0 ? c0 + row * ldc0 + col : c1 + row * ldc1 + (col - n0);
    *p = accumulate ? *p + v : v;
  }
}

}  // namespace
}  // namespace eg

extern "C" {

int eg_split_bf16(const float* x, int64_t rows, int64_t cols, int64_t ld, void* hi, void* lo, void* stream) {
  using namespace eg;
  EG_CHECK_ARG(rows >= 0 && cols >= 0 && ld >= cols, "rows=%lld cols=%lld ld=%lld", (long long)rows, (long long)cols,
               (long long)ld);
  const int64_t kp = (cols + 31) / 32 * 32;
  if (rows == 0 || kp == 0) return 0;
  EG_CHECK_ARG(x != nullptr && hi != nullptr && lo != nullptr, "NULL argument");
  EG_CHECK_ARG(((uintptr_t)hi & 15) == 0 && ((uintptr_t)lo & 15) == 0, "hi / lo must be 16-byte aligned");
  const dim3 grid((unsigned)((kp / 4 + 255) / 256), (unsigned)(rows < 65535 ? rows : 65535));
  const bool vec = ld % 4 == 0 && ((uintptr_t)x & 15) == 0;
  if (vec)
    hipLaunchKernelGGL(split_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream, x, rows, cols, ld, kp,
                       (__bf16*)hi, (__bf16*)lo);
  else
    hipLaunchKernelGGL(split_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream, x, rows, cols, ld, kp,
                       (__bf16*)hi, (__bf16*)lo);
  return launch_status("split_kernel");
}

int64_t eg_gemm_workspace_size(int64_t m, int64_t n, int64_t n2, int32_t k_slices) {
  return k_slices > 1 ? (int64_t)k_slices * m * (n + n2) * (int64_t)sizeof(float) : 0;
}

int eg_gemm_bf16x3(const eg_gemm_operands* ops, int32_t n_seg, int64_t m, int64_t n, int64_t n2, float* c,
                   int64_t ldc, float* c2, int64_t ldc2, int32_t accumulate, int32_t k_slices, void* workspace,
                   int64_t workspace_bytes, void* stream) {
  using namespace eg;
  EG_CHECK_ARG(ops != nullptr && n_seg >= 0 && n_seg <= 2, "n_seg=%d", n_seg);
  EG_CHECK_ARG(m >= 0 && n >= 0 && n2 >= 0 && k_slices >= 1, "m=%lld n=%lld n2=%lld k_slices=%d", (long long)m,
               (long long)n, (long long)n2, k_slices);
  EG_CHECK_ARG(n == 0 || (c != nullptr && ldc >= n), "c / ldc");
  EG_CHECK_ARG(n2 == 0 || (c2 != nullptr && ldc2 >= n2), "c2 / ldc2");
  if (m == 0 || n + n2 == 0) return 0;
  GemmArgs g{};
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
  g.kt0 = g.n_seg > 0 ? g.seg[0].ktiles : 0;
  g.kt_total = g.kt0 + (g.n_seg > 1 ? g.seg[1].ktiles : 0);
  int slices = k_slices;
  if (g.kt_total < slices) slices = g.kt_total > 0 ? (int)g.kt_total : 1;
  g.kt_per_slice = (g.kt_total + slices - 1) / slices;
  if (g.kt_total > 0) slices = (int)((g.kt_total + g.kt_per_slice - 1) / g.kt_per_slice);
  g.slices = slices;
  g.c[0] = c;
  g.c[1] = c2;
  g.ldc[0] = ldc;
  g.ldc[1] = ldc2;
  g.m = m;
  g.n[0] = n;
  g.n[1] = n2;
  g.accumulate = accumulate ? 1 : 0;
  if (slices > 1) {
    EG_CHECK_ARG(workspace != nullptr && ((uintptr_t)workspace & 15) == 0 &&
                     workspace_bytes >= eg_gemm_workspace_size(m, n, n2, slices),
                 "k_slices=%d needs a 16-byte aligned workspace of %lld bytes", slices,
                 (long long)eg_gemm_workspace_size(m, n, n2, slices));
    g.ws = (float*)workspace;
  }
  g.tiles_m = (int)((m + kBM - 1) / kBM);
  g.tiles_n0 = (int)((n + kBN - 1) / kBN);
  g.tiles_n = g.tiles_n0 + (int)((n2 + kBN - 1) / kBN);
  const int64_t blocks = (int64_t)g.tiles_m * g.tiles_n;
  EG_CHECK_ARG(blocks < (1LL << 31), "too many tiles");
  hipStream_t st = (hipStream_t)stream;
  static bool lds_set[64] = {};
  int dev = 0;
  EG_CHECK_HIP(hipGetDevice(&dev));
  if (dev < 64 && !lds_set[dev]) {
    EG_CHECK_HIP(hipFuncSetAttribute((const void*)gemm_x3_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLds));
    lds_set[dev] = true;
  }
  hipLaunchKernelGGL(gemm_x3_kernel, dim3((unsigned)blocks, (unsigned)slices), dim3(256), kLds, st, g);
  int rc = launch_status("gemm_x3_kernel");
  if (rc != 0 || slices == 1) return rc;
  const int64_t total = m * (n + n2);
  const int64_t sb = (total + 255) / 256 < 16384 ? (total + 255) / 256 : 16384;
  hipLaunchKernelGGL(slice_sum_kernel, dim3((unsigned)sb), dim3(256), 0, st, (const float*)g.ws, slices, m, n, n2, c,
                     ldc, c2, ldc2, g.accumulate);
  return launch_status("slice_sum_kernel");
}

}  // extern "C"
