// Backward half of the n-gram table path on gfx950: the deterministic sparse
// gradient scatter and the optimizer step on the touched overlay rows.
//
//   keys     slot s = p*heads + h  ->  (variable index of rows[s], s)
//   sort     stable LSD radix sort of the pairs by variable index (per-tile
//            digit histograms, one scan, a ballot-ranked stable scatter per
//            digit pass): equal variables keep ascending slot order
//   segment  one 32-lane group per sorted segment sums the slots' d_out
//            slices in that order (fp32), then runs Adam on the variable's
//            master row and requantises it
//   dense    rows no slot hit take their zero-gradient Adam step (dense mode)
//
// No floating-point atomics anywhere: the result is bitwise repeatable and is
// the sequential ascending-slot sum the CPU oracle computes.
#include <string.h>

#include "eg_common.h"

namespace eg {

constexpr int kSortThreads = 256;
constexpr int kSortIPT = 16;
constexpr int kSortTile = kSortThreads * kSortIPT;  // 4096 keys per tile
constexpr int kScanThreads = 1024;

__global__ __launch_bounds__(256) void keys_kernel(const int32_t* __restrict__ rows, int64_t n,
                                                   const int32_t* __restrict__ ids, int64_t n_var,
                                                   uint32_t* __restrict__ keys, uint32_t* __restrict__ vals) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t k = sorted_find(ids, n_var, rows[i]);
  keys[i] = k >= 0 ? (uint32_t)k : (uint32_t)n_var;  // frozen rows sort after every variable
  vals[i] = (uint32_t)i;
}

// Per-tile digit counts, digit-major: hist[d * n_tiles + tile].
__global__ __launch_bounds__(kSortThreads) void sort_hist(const uint32_t* __restrict__ keys, int64_t n, int shift,
                                                          int n_buckets, int n_tiles, uint32_t* __restrict__ hist) {
  __shared__ uint32_t h[256];
  for (int i = threadIdx.x; i < 256; i += kSortThreads) h[i] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kSortTile;
  const uint32_t mask = (uint32_t)n_buckets - 1u;
#pragma unroll 4
  for (int r = 0; r < kSortIPT; ++r) {
    const int64_t idx = base + r * kSortThreads + threadIdx.x;
    if (idx < n) atomicAdd(&h[(keys[idx] >> shift) & mask], 1u);
  }
  __syncthreads();
  for (int d = threadIdx.x; d < n_buckets; d += kSortThreads) hist[(int64_t)d * n_tiles + blockIdx.x] = h[d];
}

// In-place exclusive scan of a[0..len) by one workgroup.
__global__ __launch_bounds__(kScanThreads) void sort_scan(uint32_t* __restrict__ a, int64_t len) {
  __shared__ uint32_t tot[kScanThreads];
  const int tid = threadIdx.x;
  const int64_t per = (len + kScanThreads - 1) / kScanThreads;
  const int64_t lo = tid * per, hi = min(lo + per, len);
  uint32_t s = 0;
  for (int64_t i = lo; i < hi; ++i) s += a[i];
  tot[tid] = s;
  __syncthreads();
  for (int off = 1; off < kScanThreads; off <<= 1) {  // Hillis-Steele inclusive scan
    const uint32_t add = tid >= off ? tot[tid - off] : 0u;
    __syncthreads();
    tot[tid] += add;
    __syncthreads();
  }
  uint32_t run = tot[tid] - s;
  for (int64_t i = lo; i < hi; ++i) {
    const uint32_t v = a[i];
    a[i] = run;
    run += v;
  }
}

// Stable scatter of one digit pass.  Items are taken in index order (round r,
// then wave, then lane); within a wave the lanes holding the same digit are
// found with one ballot per digit bit, their rank is the popcount of the lower
// lanes, and per-digit LDS counters carry the running offset across waves and
// rounds.
__global__ __launch_bounds__(kSortThreads) void sort_scatter(const uint32_t* __restrict__ keys_in,
                                                             const uint32_t* __restrict__ vals_in,
                                                             uint32_t* __restrict__ keys_out,
                                                             uint32_t* __restrict__ vals_out, int64_t n, int shift,
                                                             int dbits, int n_tiles,
                                                             const uint32_t* __restrict__ offs) {
  constexpr int kWaves = kSortThreads / 64;
  __shared__ uint32_t run[256];
  __shared__ uint32_t wcnt[kWaves][256];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n_buckets = 1 << dbits;
  for (int d = tid; d < 256; d += kSortThreads) {
    run[d] = d < n_buckets ? offs[(int64_t)d * n_tiles + blockIdx.x] : 0u;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) wcnt[w][d] = 0;
  }
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kSortTile;
  const uint32_t mask = (uint32_t)n_buckets - 1u;
  const uint64_t lt = (1ull << lane) - 1ull;
  for (int r = 0; r < kSortIPT; ++r) {
    const int64_t idx = base + r * kSortThreads + tid;
    const bool valid = idx < n;
    uint32_t key = 0, val = 0, d = 0;
    if (valid) {
      key = keys_in[idx];
      val = vals_in[idx];
      d = (key >> shift) & mask;
    }
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < dbits; ++b) {
      const bool bit = (d >> b) & 1u;
      const uint64_t bal = __ballot(bit);
      peers &= bit ? bal : ~bal;
    }
    const uint32_t rank = (uint32_t)__popcll(peers & lt);
    if (valid && rank == 0) wcnt[wave][d] = (uint32_t)__popcll(peers);
    __syncthreads();
    if (valid) {
      uint32_t pos = run[d] + rank;
      for (int w = 0; w < wave; ++w) pos += wcnt[w][d];
      keys_out[pos] = key;
      vals_out[pos] = val;
    }
    __syncthreads();
    for (int dd = tid; dd < n_buckets; dd += kSortThreads) {
      uint32_t t = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        t += wcnt[w][dd];
        wcnt[w][dd] = 0;
      }
      run[dd] += t;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Segmented reduction + optimizer
// ---------------------------------------------------------------------------
struct SegArgs {
  const uint32_t* skeys;  // sorted variable index per slot (n_var = frozen)
  const uint32_t* svals;  // slot ids in the same order
  int64_t n;
  int64_t n_var;
  const void* d_out;
  int32_t d_out_f32;
  int32_t heads;
  int32_t dim;
  int64_t width;
  float* grad_out;        // gradient mode
  // optimizer mode
  const int32_t* ids;
  float* master;
  float* m;
  float* v;
  int32_t* stamp;
  TableDev quant;         // fmt 0: no requantised copy
  TableDev base;          // for the L2 pull term
  int64_t step;
  float w1, b2, w2, bc2s, eps, neg_step_size, l2c;
};

__device__ inline float grad_value(const SegArgs& a, int64_t idx) {
  if (a.d_out_f32) return ((const float*)a.d_out)[idx];
  return __uint_as_float((uint32_t)((const uint16_t*)a.d_out)[idx] << 16);
}

// Adam on variable k (lane `sub` owns columns sub + 32 t), torch's
// single-tensor order without contractions: m.lerp_(g, 1-b1);
// v.mul_(b2).addcmul_(g, g, 1-b2); p.addcdiv_(m, sqrt(v)/sqrt(bc2) + eps, -lr/bc1);
// then the requantised copy (block t is spread over the 32 lanes).
template <int NT>
__device__ void adam_row(const SegArgs& a, int64_t k, int sub, int nt, float g[NT]) {
#pragma clang fp contract(off)
  float pv[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if (t >= nt) break;
    const int col = sub + 32 * t;
    const int64_t idx = k * a.dim + col;
    float p = a.master[idx], m = a.m[idx], v = a.v[idx];
    float gt = g[t];
    if (a.l2c != 0.0f) {
      const int32_t row0 = a.ids[k];
      const float p0 = ((uint32_t)row0 < (uint64_t)a.base.n_rows) ? load_value_rt(a.base, row0, col)
                                                                  : __uint_as_float(0x7fc00000u);
      gt = gt + a.l2c * (2.0f * (p - p0));
    }
    m = m + a.w1 * (gt - m);
    v = v * a.b2 + (a.w2 * gt) * gt;
    const float denom = sqrtf(v) / a.bc2s + a.eps;
    p = p + a.neg_step_size * (m / denom);
    a.master[idx] = p;
    a.m[idx] = m;
    a.v[idx] = v;
    pv[t] = p;
  }
  if (a.quant.fmt == 0) return;
  const int nb = a.dim >> 5;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if (t >= nt) break;
    float amax = fabsf(pv[t]);
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 32));
    const int64_t qi = k * a.dim + sub + 32 * t;
    uint8_t* payload = (uint8_t*)a.quant.payload;
    if (a.quant.fmt == EG_FMT_Q8_0) {
      const uint16_t dh = f32_to_f16(amax / 127.0f);
      const float d = f16_to_f32(dh);
      float r = (d == 0.0f) ? 0.0f : rintf(pv[t] / d);
      r = fminf(fmaxf(r, -127.0f), 127.0f);
      payload[qi] = (uint8_t)(int32_t)r;
      if (sub == 0) ((uint16_t*)a.quant.scales)[k * nb + t] = dh;
    } else {  // EG_FMT_MXFP8
      const int ebits = (int)((__float_as_uint(amax) >> 23) & 0xffu);
      int e = (amax > 0.0f ? ebits - 127 : -127) - 8;
      e = min(max(e, -127), 127);
      if (amax * ldexpf(1.0f, -e) > 448.0f) e = min(e + 1, 127);
      const float s = fminf(fmaxf(pv[t] * ldexpf(1.0f, -e), -448.0f), 448.0f);
      payload[qi] = (uint8_t)f32_to_e4m3(s);
      if (sub == 0) ((uint8_t*)a.quant.scales)[k * nb + t] = (uint8_t)(e + 127);
    }
  }
}

// One 32-lane group per sorted position; the group at a segment's first
// position reduces the whole segment in slot order.
template <int NT, bool ADAM>
__global__ __launch_bounds__(256) void segment_kernel(const SegArgs a) {
  const int sub = threadIdx.x & 31;
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 5;
  if (i >= a.n) return;  // uniform per group
  const uint32_t key = a.skeys[i];
  if ((int64_t)key >= a.n_var) return;                 // frozen rows: no variable
  if (i > 0 && a.skeys[i - 1] == key) return;          // not the segment's first slot
  const int nt = a.dim >> 5;
  float g[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) g[t] = 0.0f;
  // Walk the segment four slots at a time: the loads of four slots are issued
  // together, the additions stay in slot order.
  for (int64_t j = i;; j += 4) {
    uint32_t kk[4], vv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      kk[u] = (j + u < a.n) ? a.skeys[j + u] : 0xffffffffu;
      vv[u] = (j + u < a.n) ? a.svals[j + u] : 0u;
    }
    float x[4][NT];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (kk[u] == key) {
        const int64_t p = vv[u] / (uint32_t)a.heads;
        const int h = (int)(vv[u] - p * a.heads);
        const int64_t base = p * a.width + (int64_t)h * a.dim + sub;
#pragma unroll
        for (int t = 0; t < NT; ++t)
          if (t < nt) x[u][t] = grad_value(a, base + 32 * t);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (kk[u] == key) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
          if (t < nt) g[t] = g[t] + x[u][t];
      }
    if (kk[3] != key) break;
  }
  if constexpr (ADAM) {
    adam_row<NT>(a, key, sub, nt, g);
    if (sub == 0) a.stamp[key] = (int32_t)a.step;
  } else {
#pragma unroll
    for (int t = 0; t < NT; ++t)
      if (t < nt) {
        float* dst = a.grad_out + (int64_t)key * a.dim + sub + 32 * t;
        *dst = *dst + g[t];
      }
  }
}

// Dense mode: the variables no slot hit this step take a zero-gradient step.
template <int NT>
__global__ __launch_bounds__(256) void dense_kernel(const SegArgs a) {
  const int sub = threadIdx.x & 31;
  const int64_t k = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 5;
  if (k >= a.n_var) return;
  if (a.stamp[k] == (int32_t)a.step) return;
  float g[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) g[t] = 0.0f;
  adam_row<NT>(a, k, sub, a.dim >> 5, g);
}

struct Workspace {
  uint32_t* keys[2];
  uint32_t* vals[2];
  uint32_t* hist;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static size_t workspace_bytes(int64_t n) {
  const int64_t tiles = (n + kSortTile - 1) / kSortTile;
  return 4 * align256((size_t)n * 4) + align256((size_t)tiles * 256 * 4);
}

static Workspace carve(void* ws, int64_t n) {
  Workspace w;
  char* p = (char*)ws;
  const size_t kb = align256((size_t)n * 4);
  w.keys[0] = (uint32_t*)p;
  w.vals[0] = (uint32_t*)(p + kb);
  w.keys[1] = (uint32_t*)(p + 2 * kb);
  w.vals[1] = (uint32_t*)(p + 3 * kb);
  w.hist = (uint32_t*)(p + 4 * kb);
  return w;
}

// keys + stable radix sort; returns the index (0/1) of the sorted buffers.
static int sort_slots(const int32_t* rows, int64_t n, const int32_t* ids, int64_t n_var, const Workspace& w,
                      hipStream_t st, int* sorted) {
  hipLaunchKernelGGL(keys_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, rows, n, ids, n_var,
                     w.keys[0], w.vals[0]);
  int rc = launch_status("keys_kernel");
  if (rc != EG_OK) return rc;
  int bits = 0;
  while (bits < 32 && ((uint64_t)n_var >> bits) != 0) ++bits;  // keys lie in [0, n_var]
  int cur = 0;
  if (bits > 0) {
    const int passes = (bits + 7) / 8;
    const int dbits = (bits + passes - 1) / passes;
    const int n_tiles = (int)((n + kSortTile - 1) / kSortTile);
    for (int pass = 0; pass < passes; ++pass) {
      const int shift = pass * dbits;
      hipLaunchKernelGGL(sort_hist, dim3(n_tiles), dim3(kSortThreads), 0, st, w.keys[cur], n, shift, 1 << dbits,
                         n_tiles, w.hist);
      hipLaunchKernelGGL(sort_scan, dim3(1), dim3(kScanThreads), 0, st, w.hist, (int64_t)n_tiles << dbits);
      hipLaunchKernelGGL(sort_scatter, dim3(n_tiles), dim3(kSortThreads), 0, st, w.keys[cur], w.vals[cur],
                         w.keys[cur ^ 1], w.vals[cur ^ 1], n, shift, dbits, n_tiles, w.hist);
      rc = launch_status("radix sort pass");
      if (rc != EG_OK) return rc;
      cur ^= 1;
    }
  }
  *sorted = cur;
  return EG_OK;
}

template <bool ADAM>
static void launch_segments(const SegArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)((a.n * 32 + 255) / 256));
  const int nt = a.dim >> 5;
  if (nt == 4) hipLaunchKernelGGL((segment_kernel<4, ADAM>), grid, dim3(256), 0, st, a);
  else if (nt == 5) hipLaunchKernelGGL((segment_kernel<5, ADAM>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((segment_kernel<16, ADAM>), grid, dim3(256), 0, st, a);
}

static int check_common(const void* d_out, const int32_t* rows, int64_t n_pos, int32_t heads, int32_t dim,
                        const int32_t* ids, int64_t n_var, void* ws, size_t ws_bytes) {
  EG_CHECK_ARG(n_pos >= 0 && heads >= 1 && heads <= EG_MAX_HEADS, "n_pos=%lld heads=%d", (long long)n_pos, heads);
  EG_CHECK_ARG(dim > 0 && dim % 32 == 0 && dim <= 512, "dim=%d must be a multiple of 32 in [32, 512]", dim);
  EG_CHECK_ARG(n_var >= 0 && n_var < (1LL << 31), "n_var=%lld", (long long)n_var);
  const int64_t n = n_pos * heads;
  EG_CHECK_ARG(n < (1LL << 31), "n_pos*heads=%lld slots exceed 2^31", (long long)n);
  EG_CHECK_ARG(n == 0 || (d_out != nullptr && rows != nullptr), "d_out/rows is NULL");
  EG_CHECK_ARG(n_var == 0 || ids != nullptr, "ids is NULL");
  if (ws_bytes < workspace_bytes(n))
    return set_error(EG_ERR_WORKSPACE, "workspace of %zu bytes < %zu needed", ws_bytes, workspace_bytes(n));
  EG_CHECK_ARG(n == 0 || ws != nullptr, "workspace is NULL");
  return EG_OK;
}

}  // namespace eg

using namespace eg;

extern "C" {

size_t eg_backward_workspace_size(int64_t n_slots) { return workspace_bytes(n_slots < 0 ? 0 : n_slots); }

int eg_scatter_grad(const void* d_out, int32_t d_out_f32, const int32_t* rows, int64_t n_pos, int32_t heads,
                    int32_t dim, const int32_t* ids, int64_t n_var, float* grad_out, void* workspace,
                    size_t workspace_bytes_, void* stream) {
  int rc = check_common(d_out, rows, n_pos, heads, dim, ids, n_var, workspace, workspace_bytes_);
  if (rc != EG_OK) return rc;
  EG_CHECK_ARG(n_var == 0 || grad_out != nullptr, "grad_out is NULL");
  const int64_t n = n_pos * heads;
  if (n == 0 || n_var == 0) return EG_OK;
  hipStream_t st = (hipStream_t)stream;
  const Workspace w = carve(workspace, n);
  int cur = 0;
  rc = sort_slots(rows, n, ids, n_var, w, st, &cur);
  if (rc != EG_OK) return rc;
  SegArgs a;
  memset(&a, 0, sizeof(a));
  a.skeys = w.keys[cur];
  a.svals = w.vals[cur];
  a.n = n;
  a.n_var = n_var;
  a.d_out = d_out;
  a.d_out_f32 = d_out_f32;
  a.heads = heads;
  a.dim = dim;
  a.width = (int64_t)heads * dim;
  a.grad_out = grad_out;
  launch_segments<false>(a, st);
  return launch_status("segment_kernel");
}

int eg_descent_step(const void* d_out, int32_t d_out_f32, const int32_t* rows, int64_t n_pos, int32_t heads,
                    const eg_descent_state* state, const eg_adam* opt, const eg_table* base, void* workspace,
                    size_t workspace_bytes_, void* stream) {
  EG_CHECK_ARG(state != nullptr && opt != nullptr, "state/opt is NULL");
  int rc = check_common(d_out, rows, n_pos, heads, state->dim, state->ids, state->n, workspace, workspace_bytes_);
  if (rc != EG_OK) return rc;
  EG_CHECK_ARG(state->n == 0 || (state->master && state->m && state->v && state->stamp),
               "state master/m/v/stamp is NULL");
  EG_CHECK_ARG(opt->step >= 1 && opt->step < (1LL << 31), "step=%lld", (long long)opt->step);
  EG_CHECK_ARG(opt->lr >= 0.0 && opt->beta1 >= 0.0 && opt->beta1 < 1.0 && opt->beta2 >= 0.0 &&
                   opt->beta2 < 1.0 && opt->eps >= 0.0,
               "invalid Adam hyper-parameters");
  SegArgs a;
  memset(&a, 0, sizeof(a));
  if (state->quant.payload != nullptr) {
    rc = make_table(&state->quant, &a.quant, "requantised rows");
    if (rc != EG_OK) return rc;
    EG_CHECK_ARG(state->quant.fmt == EG_FMT_Q8_0 || state->quant.fmt == EG_FMT_MXFP8,
                 "requantised rows must be Q8_0 or MXFP8");
    EG_CHECK_ARG(state->quant.dim == state->dim && state->quant.n_rows >= state->n, "requantised rows shape");
  }
  if (opt->l2_coef != 0.0f) {
    rc = make_table(base, &a.base, "base table");
    if (rc != EG_OK) return rc;
    EG_CHECK_ARG(base->dim == state->dim, "base table dim %d != state dim %d", base->dim, state->dim);
  }
  const int64_t n = n_pos * heads;
  if (state->n == 0) return EG_OK;
  hipStream_t st = (hipStream_t)stream;
  const Workspace w = carve(workspace, n);
  int cur = 0;
  if (n > 0) {
    rc = sort_slots(rows, n, state->ids, state->n, w, st, &cur);
    if (rc != EG_OK) return rc;
  }
  a.skeys = w.keys[cur];
  a.svals = w.vals[cur];
  a.n = n;
  a.n_var = state->n;
  a.d_out = d_out;
  a.d_out_f32 = d_out_f32;
  a.heads = heads;
  a.dim = state->dim;
  a.width = (int64_t)heads * state->dim;
  a.ids = state->ids;
  a.master = state->master;
  a.m = state->m;
  a.v = state->v;
  a.stamp = state->stamp;
  a.step = opt->step;
  const double b1 = opt->beta1, b2 = opt->beta2;
  const double bc1 = 1.0 - pow(b1, (double)opt->step);
  const double bc2 = 1.0 - pow(b2, (double)opt->step);
  a.w1 = (float)(1.0 - b1);
  a.b2 = (float)b2;
  a.w2 = (float)(1.0 - b2);
  a.bc2s = (float)sqrt(bc2);
  a.eps = (float)opt->eps;
  a.neg_step_size = -(float)(opt->lr / bc1);
  a.l2c = opt->l2_coef;
  if (n > 0) {
    launch_segments<true>(a, st);
    rc = launch_status("segment_kernel");
    if (rc != EG_OK) return rc;
  }
  if (opt->dense) {
    const dim3 grid((unsigned)((state->n * 32 + 255) / 256));
    const int nt = state->dim >> 5;
    if (nt == 4) hipLaunchKernelGGL(dense_kernel<4>, grid, dim3(256), 0, st, a);
    else if (nt == 5) hipLaunchKernelGGL(dense_kernel<5>, grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(dense_kernel<16>, grid, dim3(256), 0, st, a);
    rc = launch_status("dense_kernel");
  }
  return rc;
}

}  // extern "C"
