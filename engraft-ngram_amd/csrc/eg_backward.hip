// Backward half of the n-gram table path on gfx950: the deterministic sparse
// gradient scatter and the optimizer step on the touched overlay rows.
//
//   keys     slot s = p*heads + h -> (variable index of rows[s], s); the
//            variable is found through an LDS splitter table of the sorted
//            ids; the first digit's per-tile histogram is built on the way
//   sort     stable LSD radix sort of the pairs by variable index, digits of
//            up to 9 bits: one scan and one ballot-ranked stable scatter per
//            pass (the scatter also counts the next pass's digits), so equal
//            variables keep ascending slot order
//   segment  one 32-lane group per segment of at most 32 slots sums the
//            slots' d_out slices in slot order (fp32) and runs Adam +
//            requantisation on the variable; a longer segment is reduced by
//            a whole workgroup of the same launch: pieces of 32 slots summed
//            in order, piece sums accumulated per group (pieces j = g mod 8),
//            the eight group sums added in group order
//   dense    variables no slot hit take their zero-gradient step (dense mode)
//
// No floating-point atomics: the association of every sum is fixed by the
// sorted order alone, so results are bitwise repeatable, and the CPU oracle
// reproduces them exactly.
#include <string.h>

#include "eg_common.h"

namespace eg {

constexpr int kTileThreads = 256;
constexpr int kTileIPT = 4;
constexpr int kTile = kTileThreads * kTileIPT;  // 1024 keys per tile
constexpr int kMaxDigitBits = 9;
constexpr int kMaxBuckets = 1 << kMaxDigitBits;
constexpr int kScanThreads = 1024;
constexpr int kSplitMax = 2048;  // splitters staged in LDS (8 KB)
constexpr int kPiece = 32;       // slots per piece of a long segment
constexpr int kLongGroups = 8;   // 32-lane groups per long-segment workgroup

// ---------------------------------------------------------------------------
// Row index: open addressing over a power-of-two table of (row << 32 | k)
// entries, Fibonacci hashing, linear probing.  Lookups are deterministic
// whatever order the entries were inserted in.
// ---------------------------------------------------------------------------
constexpr unsigned long long kIndexEmpty = ~0ull;

__device__ inline uint64_t index_slot(int32_t row, int bits) {
  return (uint64_t)(((uint32_t)row * 0x9E3779B1u) >> (32 - bits));
}

__global__ __launch_bounds__(256) void index_fill_kernel(unsigned long long* __restrict__ tab, int64_t cap) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < cap; i += (int64_t)gridDim.x * 256)
    tab[i] = kIndexEmpty;
}

__global__ __launch_bounds__(256) void index_build_kernel(const int32_t* __restrict__ ids, int64_t n,
                                                          unsigned long long* __restrict__ tab, int bits) {
  const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (k >= n) return;
  const int32_t row = ids[k];
  const uint64_t mask = (1ull << bits) - 1ull;
  const unsigned long long packed = ((unsigned long long)(uint32_t)row << 32) | (uint32_t)k;
  uint64_t h = index_slot(row, bits);
  for (uint64_t probe = 0; probe <= mask; ++probe) {  // the table is at most half full
    if (atomicCAS(&tab[h], kIndexEmpty, packed) == kIndexEmpty) return;
    h = (h + 1) & mask;
  }
}

// ---------------------------------------------------------------------------
// Keys + first histogram
// ---------------------------------------------------------------------------
// MODE 0: search the sorted ids; 1: probe the row index; 2: rows already hold
// variable indices (< 0 or >= n_var: no variable).
template <int MODE>
__global__ __launch_bounds__(kTileThreads) void keys_hist_kernel(
    const int32_t* __restrict__ rows, int64_t n, const int32_t* __restrict__ ids, int64_t n_var, int split_shift,
    const unsigned long long* __restrict__ index, int index_bits, uint32_t* __restrict__ keys,
    uint32_t* __restrict__ vals, int dbits, int n_tiles, uint32_t* __restrict__ hist) {
  __shared__ int32_t spl[kSplitMax];
  __shared__ uint32_t h[kMaxBuckets];
  const int tid = threadIdx.x;
  const int ns = MODE == 0 ? (int)((n_var + (1LL << split_shift) - 1) >> split_shift) : 0;
  for (int i = tid; i < ns; i += kTileThreads) spl[i] = ids[(int64_t)i << split_shift];
  for (int i = tid; i < kMaxBuckets; i += kTileThreads) h[i] = 0;
  __syncthreads();
  const uint32_t mask = (1u << dbits) - 1u;
  // The kTileIPT lookups of a thread run in lockstep (fixed-length branchless
  // searches), so their memory latencies overlap.
  int32_t row[kTileIPT];
  bool ok[kTileIPT];
#pragma unroll
  for (int r = 0; r < kTileIPT; ++r) {
    const int64_t idx = (int64_t)blockIdx.x * kTile + r * kTileThreads + tid;
    ok[r] = idx < n;
    row[r] = ok[r] ? rows[idx] : 0;
  }
  uint32_t key[kTileIPT];
  if constexpr (MODE == 2) {
#pragma unroll
    for (int r = 0; r < kTileIPT; ++r)
      key[r] = (row[r] >= 0 && (int64_t)row[r] < n_var) ? (uint32_t)row[r] : (uint32_t)n_var;
  } else if constexpr (MODE == 1) {
    // probe the row index; the items' probes advance in lockstep
    const uint64_t imask = (1ull << index_bits) - 1ull;
    uint64_t hslot[kTileIPT];
    bool done[kTileIPT];
#pragma unroll
    for (int r = 0; r < kTileIPT; ++r) {
      hslot[r] = index_slot(row[r], index_bits);
      done[r] = !ok[r];
      key[r] = (uint32_t)n_var;
    }
    for (uint64_t probe = 0; probe <= imask; ++probe) {
      bool any = false;
#pragma unroll
      for (int r = 0; r < kTileIPT; ++r) {
        if (done[r]) continue;
        const unsigned long long e = index[hslot[r]];
        if (e == kIndexEmpty) {
          done[r] = true;
        } else if ((uint32_t)(e >> 32) == (uint32_t)row[r]) {
          key[r] = (uint32_t)e;
          done[r] = true;
        } else {
          hslot[r] = (hslot[r] + 1) & imask;
          any = true;
        }
      }
      if (!any) break;
    }
  } else {
    // level 1 (LDS): lo = number of splitters <= row
    int lo[kTileIPT];
#pragma unroll
    for (int r = 0; r < kTileIPT; ++r) lo[r] = 0;
    for (int step = kSplitMax; step >= 1; step >>= 1) {
#pragma unroll
      for (int r = 0; r < kTileIPT; ++r)
        if (lo[r] + step <= ns && spl[lo[r] + step - 1] <= row[r]) lo[r] += step;
    }
    // level 2 (global): the last id <= row inside that splitter's window
    const int64_t win = 1LL << split_shift;
    int64_t pos[kTileIPT], end[kTileIPT];
#pragma unroll
    for (int r = 0; r < kTileIPT; ++r) {
      pos[r] = lo[r] > 0 ? ((int64_t)(lo[r] - 1) << split_shift) : 0;
      end[r] = lo[r] > 0 ? min(pos[r] + win, n_var) : 0;
    }
    for (int64_t step = win >> 1; step >= 1; step >>= 1) {
#pragma unroll
      for (int r = 0; r < kTileIPT; ++r)
        if (pos[r] + step < end[r] && ids[pos[r] + step] <= row[r]) pos[r] += step;
    }
#pragma unroll
    for (int r = 0; r < kTileIPT; ++r) {
      key[r] = (ok[r] && lo[r] > 0 && ids[pos[r]] == row[r]) ? (uint32_t)pos[r] : (uint32_t)n_var;
    }
  }
#pragma unroll
  for (int r = 0; r < kTileIPT; ++r) {
    if (!ok[r]) continue;
    const int64_t idx = (int64_t)blockIdx.x * kTile + r * kTileThreads + tid;
    keys[idx] = key[r];
    vals[idx] = (uint32_t)idx;
    atomicAdd(&h[key[r] & mask], 1u);
  }
  __syncthreads();
  for (int d = tid; d < (1 << dbits); d += kTileThreads) hist[(int64_t)d * n_tiles + blockIdx.x] = h[d];
}

// ---------------------------------------------------------------------------
// Exclusive scan (one workgroup, coalesced strips) + clearing of the next
// pass's histogram
// ---------------------------------------------------------------------------
__device__ inline uint32_t wave_inclusive_scan(uint32_t x, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  return x;
}

// Block-wide exclusive scan of one value per thread (1024 threads).
__device__ inline uint32_t block_exclusive_scan(uint32_t t, uint32_t* wsum, uint32_t* total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t incl = wave_inclusive_scan(t, lane);
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kScanThreads / 64; ++w) {
    const uint32_t x = wsum[w];
    if (w < wave) before += x;
    all += x;
  }
  *total = all;
  return before + incl - t;
}

constexpr int kScanChunk = 4 * kScanThreads;  // entries per scan workgroup
constexpr int kMaxChunksLds = 2048;            // scan chunks a scatter can count in LDS

// Pass 1 of the exclusive scan: the total of every chunk; also clears the next
// pass's histogram.
__global__ __launch_bounds__(kScanThreads) void scan_partials(const uint32_t* __restrict__ a, int64_t len,
                                                              uint32_t* __restrict__ partial,
                                                              uint32_t* __restrict__ clear, int64_t clear_len) {
  __shared__ uint32_t wsum[kScanThreads / 64];
  const int tid = threadIdx.x;
  for (int64_t i = (int64_t)blockIdx.x * kScanThreads + tid; i < clear_len; i += (int64_t)gridDim.x * kScanThreads)
    clear[i] = 0;
  const int64_t i0 = (int64_t)blockIdx.x * kScanChunk + 4 * tid;
  uint32_t t = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) t += (i0 + u < len) ? a[i0 + u] : 0u;
  uint32_t total;
  block_exclusive_scan(t, wsum, &total);
  if (tid == 0) partial[blockIdx.x] = total;
}

// Pass 2: exclusive scan of every chunk, offset by the totals of the chunks
// before it.
__global__ __launch_bounds__(kScanThreads) void scan_apply(uint32_t* __restrict__ a, int64_t len,
                                                           const uint32_t* __restrict__ partial,
                                                           uint32_t* __restrict__ clear, int64_t clear_len) {
  __shared__ uint32_t wsum[kScanThreads / 64];
  __shared__ uint32_t wsum2[kScanThreads / 64];
  const int tid = threadIdx.x;
  for (int64_t i = (int64_t)blockIdx.x * kScanThreads + tid; i < clear_len; i += (int64_t)gridDim.x * kScanThreads)
    clear[i] = 0;
  uint32_t pre = 0;
  for (int g = tid; g < (int)blockIdx.x; g += kScanThreads) pre += partial[g];
  const int64_t i0 = (int64_t)blockIdx.x * kScanChunk + 4 * tid;
  uint32_t v[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) v[u] = (i0 + u < len) ? a[i0 + u] : 0u;
  uint32_t base;
  block_exclusive_scan(pre, wsum2, &base);  // base = sum of every thread's share of the earlier chunks
  __syncthreads();
  uint32_t total;
  uint32_t run = base + block_exclusive_scan(v[0] + v[1] + v[2] + v[3], wsum, &total);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    if (i0 + u < len) a[i0 + u] = run;
    run += v[u];
  }
}

// ---------------------------------------------------------------------------
// Stable scatter of one digit pass.  Items are taken in index order (round,
// then wave, then lane); lanes holding the same digit are found with one
// ballot per digit bit, their rank is the popcount of the lower lanes, and
// per-digit LDS counters carry the running offset across waves and rounds.
// The next pass's per-tile histogram is counted at the destination.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kTileThreads) void scatter_kernel(
    const uint32_t* __restrict__ keys_in, const uint32_t* __restrict__ vals_in, uint32_t* __restrict__ keys_out,
    uint32_t* __restrict__ vals_out, int64_t n, int shift, int dbits, int n_tiles, const uint32_t* __restrict__ offs,
    uint32_t* __restrict__ hist_next, uint32_t* __restrict__ partial_next, int next_shift, int next_dbits) {
  constexpr int kWaves = kTileThreads / 64;
  __shared__ uint32_t run[kMaxBuckets];
  __shared__ uint32_t wcnt[kWaves][kMaxBuckets];
  __shared__ uint32_t chunk_cnt[kMaxChunksLds];  // the next scan's chunk totals, this tile's share
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n_buckets = 1 << dbits;
  for (int d = tid; d < n_buckets; d += kTileThreads) {
    run[d] = offs[(int64_t)d * n_tiles + blockIdx.x];
#pragma unroll
    for (int w = 0; w < kWaves; ++w) wcnt[w][d] = 0;
  }
  __syncthreads();
  const int64_t next_chunks =
      partial_next ? (((int64_t)n_tiles << next_dbits) + kScanChunk - 1) / kScanChunk : 0;  // <= kMaxChunksLds
  for (int c = tid; c < next_chunks; c += kTileThreads) chunk_cnt[c] = 0;
  __syncthreads();
  const uint32_t mask = (uint32_t)n_buckets - 1u;
  const uint32_t next_mask = (1u << next_dbits) - 1u;
  const uint64_t lt = (1ull << lane) - 1ull;
  for (int r = 0; r < kTileIPT; ++r) {
    const int64_t idx = (int64_t)blockIdx.x * kTile + r * kTileThreads + tid;
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
      if (hist_next != nullptr) {
        const int64_t hi = (int64_t)((key >> next_shift) & next_mask) * n_tiles + pos / kTile;
        atomicAdd(&hist_next[hi], 1u);
        if (partial_next != nullptr) atomicAdd(&chunk_cnt[hi / kScanChunk], 1u);
      }
    }
    __syncthreads();
    for (int dd = tid; dd < n_buckets; dd += kTileThreads) {
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
  for (int c = tid; c < next_chunks; c += kTileThreads)
    if (chunk_cnt[c] != 0) atomicAdd(&partial_next[c], chunk_cnt[c]);
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
  TableDev base;          // for the pull term
  int64_t step;
  int32_t dense;          // stamp the rows hit (the dense pass skips them)
  float w1, b2, w2, bc2s, eps, neg_step_size, l2c;
};

// A lane owns VPL columns of a row: consecutive (sub*VPL + t) when VPL divides
// 32 (vector loads, a 32-value block spans 32/VPL lanes), else strided
// (sub + 32 t: block t spans the 32 lanes).
template <int VPL, bool CONSEC>
__device__ inline int col_of(int sub, int t) {
  return CONSEC ? sub * VPL + t : sub + 32 * t;
}

// (The state rows and d_out slices are touched once per step: streaming,
// non-temporal accesses keep them from evicting the sorted keys from L2.)
template <int VPL, bool CONSEC>
__device__ inline void load_f32(const float* __restrict__ row, int sub, float x[VPL]) {
  if constexpr (CONSEC && VPL == 4) {
    const u32x4 q = __builtin_nontemporal_load((const u32x4*)(row + sub * 4));
#pragma unroll
    for (int t = 0; t < 4; ++t) x[t] = __uint_as_float(q[t]);
  } else {
#pragma unroll
    for (int t = 0; t < VPL; ++t) x[t] = row[col_of<VPL, CONSEC>(sub, t)];
  }
}

template <int VPL, bool CONSEC>
__device__ inline void store_f32(float* __restrict__ row, int sub, const float x[VPL]) {
  if constexpr (CONSEC && VPL == 4) {
    __builtin_nontemporal_store(u32x4{__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]),
                                      __float_as_uint(x[3])},
                                (u32x4*)(row + sub * 4));
  } else {
#pragma unroll
    for (int t = 0; t < VPL; ++t) row[col_of<VPL, CONSEC>(sub, t)] = x[t];
  }
}

// d_out slice of one slot (bf16 or f32), VPL values of this lane.
template <int VPL, bool CONSEC>
__device__ inline void load_grad(const SegArgs& a, uint32_t slot, int sub, float x[VPL]) {
  const int64_t p = slot / (uint32_t)a.heads;
  const int h = (int)(slot - p * a.heads);
  const int64_t base = p * a.width + (int64_t)h * a.dim;
  if (a.d_out_f32) {
    load_f32<VPL, CONSEC>((const float*)a.d_out + base, sub, x);
  } else {
    const uint16_t* src = (const uint16_t*)a.d_out + base;
    if constexpr (CONSEC && VPL == 4) {
      const u32x2 q = __builtin_nontemporal_load((const u32x2*)(src + sub * 4));
      x[0] = __uint_as_float(q.x << 16);
      x[1] = __uint_as_float(q.x & 0xffff0000u);
      x[2] = __uint_as_float(q.y << 16);
      x[3] = __uint_as_float(q.y & 0xffff0000u);
    } else {
#pragma unroll
      for (int t = 0; t < VPL; ++t) x[t] = __uint_as_float((uint32_t)src[col_of<VPL, CONSEC>(sub, t)] << 16);
    }
  }
}

// Sums the d_out slices of `cnt` (<= 32) consecutive sorted slots whose slot
// ids sit in lane (gbase + e) of `vl`, in order, onto g.  Loads go out kBatch
// slots at a time; the additions stay in slot order.
template <int VPL, bool CONSEC, int kBatch>
__device__ inline void sum_piece(const SegArgs& a, uint32_t vl, int gbase, int cnt, int sub, float g[VPL]) {
  for (int e0 = 0; e0 < cnt; e0 += kBatch) {
    float x[kBatch][VPL];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const uint32_t s = (uint32_t)__shfl((int)vl, gbase + ((e0 + u) & 31));
      if (e0 + u < cnt) load_grad<VPL, CONSEC>(a, s, sub, x[u]);
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (e0 + u < cnt) {
#pragma unroll
        for (int t = 0; t < VPL; ++t) g[t] = g[t] + x[u][t];
      }
  }
}

// Adam on variable k (torch's single-tensor order, no contractions):
// m.lerp_(g, 1-b1); v.mul_(b2).addcmul_(g, g, 1-b2);
// p.addcdiv_(m, sqrt(v)/sqrt(bc2) + eps, -lr/bc1); then the requantised copy.
template <int VPL, bool CONSEC>
__device__ void adam_apply(const SegArgs& a, int64_t k, int sub, const float g[VPL], float p[VPL], float m[VPL],
                           float v[VPL]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int t = 0; t < VPL; ++t) {
    float gt = g[t];
    if (a.l2c != 0.0f) {
      const int32_t row0 = a.ids[k];
      const float p0 = ((uint32_t)row0 < (uint64_t)a.base.n_rows)
                           ? load_value_rt(a.base, row0, col_of<VPL, CONSEC>(sub, t))
                           : __uint_as_float(0x7fc00000u);
      gt = gt + a.l2c * (2.0f * (p[t] - p0));
    }
    m[t] = m[t] + a.w1 * (gt - m[t]);
    v[t] = v[t] * a.b2 + (a.w2 * gt) * gt;
    const float denom = sqrtf(v[t]) / a.bc2s + a.eps;
    p[t] = p[t] + a.neg_step_size * (m[t] / denom);
  }
  const int64_t off = k * a.dim;
  store_f32<VPL, CONSEC>(a.master + off, sub, p);
  store_f32<VPL, CONSEC>(a.m + off, sub, m);
  store_f32<VPL, CONSEC>(a.v + off, sub, v);
  if (a.quant.fmt == 0) return;
  const int nb = a.dim >> 5;
  uint8_t* payload = (uint8_t*)a.quant.payload;
  if constexpr (CONSEC) {
    // this lane's values all lie in block sub / (32 / VPL)
    constexpr int kLanesPerBlock = 32 / VPL;
    float amax = 0.0f;
#pragma unroll
    for (int t = 0; t < VPL; ++t) amax = fmaxf(amax, fabsf(p[t]));
#pragma unroll
    for (int o = kLanesPerBlock / 2; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 32));
    const int blk = sub / kLanesPerBlock;
    uint32_t packed = 0;
    if (a.quant.fmt == EG_FMT_Q8_0) {
      const uint16_t dh = f32_to_f16(amax / 127.0f);
      const float d = f16_to_f32(dh);
#pragma unroll
      for (int t = 0; t < VPL; ++t) {
        float r = (d == 0.0f) ? 0.0f : rintf(p[t] / d);
        r = fminf(fmaxf(r, -127.0f), 127.0f);
        const uint32_t b = (uint32_t)(int32_t)r & 0xffu;
        if constexpr (VPL == 4) packed |= b << (8 * t);
        else payload[off + col_of<VPL, CONSEC>(sub, t)] = (uint8_t)b;
      }
      if (sub % kLanesPerBlock == 0) ((uint16_t*)a.quant.scales)[k * nb + blk] = dh;
    } else {  // EG_FMT_MXFP8
      const int ebits = (int)((__float_as_uint(amax) >> 23) & 0xffu);
      int e = (amax > 0.0f ? ebits - 127 : -127) - 8;
      e = min(max(e, -127), 127);
      if (amax * ldexpf(1.0f, -e) > 448.0f) e = min(e + 1, 127);
      const float inv = ldexpf(1.0f, -e);
#pragma unroll
      for (int t = 0; t < VPL; ++t) {
        const uint32_t b = f32_to_e4m3(fminf(fmaxf(p[t] * inv, -448.0f), 448.0f));
        if constexpr (VPL == 4) packed |= b << (8 * t);
        else payload[off + col_of<VPL, CONSEC>(sub, t)] = (uint8_t)b;
      }
      if (sub % kLanesPerBlock == 0) ((uint8_t*)a.quant.scales)[k * nb + blk] = (uint8_t)(e + 127);
    }
    if constexpr (VPL == 4) *(uint32_t*)(payload + off + sub * 4) = packed;
  } else {
#pragma unroll
    for (int t = 0; t < VPL; ++t) {
      float amax = fabsf(p[t]);
#pragma unroll
      for (int o = 16; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 32));
      const int64_t qi = off + sub + 32 * t;
      if (a.quant.fmt == EG_FMT_Q8_0) {
        const uint16_t dh = f32_to_f16(amax / 127.0f);
        const float d = f16_to_f32(dh);
        float r = (d == 0.0f) ? 0.0f : rintf(p[t] / d);
        r = fminf(fmaxf(r, -127.0f), 127.0f);
        payload[qi] = (uint8_t)(int32_t)r;
        if (sub == 0) ((uint16_t*)a.quant.scales)[k * nb + t] = dh;
      } else {
        const int ebits = (int)((__float_as_uint(amax) >> 23) & 0xffu);
        int e = (amax > 0.0f ? ebits - 127 : -127) - 8;
        e = min(max(e, -127), 127);
        if (amax * ldexpf(1.0f, -e) > 448.0f) e = min(e + 1, 127);
        payload[qi] = (uint8_t)f32_to_e4m3(fminf(fmaxf(p[t] * ldexpf(1.0f, -e), -448.0f), 448.0f));
        if (sub == 0) ((uint8_t*)a.quant.scales)[k * nb + t] = (uint8_t)(e + 127);
      }
    }
  }
}

// The sum g of variable k is final: optimizer step, or accumulation into grad_out.
template <int VPL, bool CONSEC, bool ADAM>
__device__ inline void finish(const SegArgs& a, int64_t k, int sub, const float g[VPL], float p[VPL], float m[VPL],
                              float v[VPL]) {
  if constexpr (ADAM) {
    adam_apply<VPL, CONSEC>(a, k, sub, g, p, m, v);
    if (a.dense && sub == 0) a.stamp[k] = (int32_t)a.step;
  } else {
    float* dst = a.grad_out + k * a.dim;
    float cur[VPL];
    load_f32<VPL, CONSEC>(dst, sub, cur);
#pragma unroll
    for (int t = 0; t < VPL; ++t) cur[t] = cur[t] + g[t];
    store_f32<VPL, CONSEC>(dst, sub, cur);
  }
}

// One launch for every segment.  A segment longer than kPiece slots is taken
// by one of the first n_long_blocks workgroups: block b owns the sorted
// positions [(kPiece+1) b, (kPiece+1)(b+1)), which hold at most one long
// segment's first slot (two such firsts are more than kPiece apart).  It sums
// pieces of kPiece slots in order, adds piece j to group j mod kLongGroups and
// the group sums in group order.  These blocks are dispatched first, so their
// longer chains overlap the rest.
// Every other workgroup holds eight 32-lane groups, one per sorted position:
// the group at the first slot of a segment of at most kPiece slots reduces it.
template <int VPL, bool CONSEC, bool ADAM>
__global__ __launch_bounds__(256) void reduce_kernel(const SegArgs a, int64_t n_long_blocks) {
  __shared__ float part[kLongGroups][512];
  const int lane = threadIdx.x & 63, sub = lane & 31, gbase = lane & 32;
  if ((int64_t)blockIdx.x < n_long_blocks) {
    __shared__ int64_t found;
    if (threadIdx.x == 0) found = -1;
    __syncthreads();
    if (threadIdx.x <= kPiece) {
      const int64_t c = (int64_t)blockIdx.x * (kPiece + 1) + threadIdx.x;
      if (c + kPiece < a.n) {
        const uint32_t kc = a.skeys[c];
        if ((int64_t)kc < a.n_var && a.skeys[c + kPiece] == kc && (c == 0 || a.skeys[c - 1] != kc)) found = c;
      }
    }
    __syncthreads();
    if (found < 0) return;  // uniform per workgroup
    const int grp = threadIdx.x >> 5;
    const int64_t i0 = found;
    const uint32_t key = a.skeys[i0];
    float p[VPL], m[VPL], v[VPL];
    if (ADAM && grp == 0) {  // independent of the gradient: fetched first
      const int64_t off = (int64_t)key * a.dim;
      load_f32<VPL, CONSEC>(a.master + off, sub, p);
      load_f32<VPL, CONSEC>(a.m + off, sub, m);
      load_f32<VPL, CONSEC>(a.v + off, sub, v);
    }
    float G[VPL];
#pragma unroll
    for (int t = 0; t < VPL; ++t) G[t] = 0.0f;
    for (int64_t j = grp;; j += kLongGroups) {
      const int64_t start = i0 + j * kPiece;
      if (start >= a.n) break;
      const uint32_t kl = (start + sub < a.n) ? a.skeys[start + sub] : 0xffffffffu;
      const uint32_t vl = (start + sub < a.n) ? a.svals[start + sub] : 0u;
      const int cnt = __popc((uint32_t)(__ballot(kl == key) >> gbase));
      if (cnt == 0) break;
      float P[VPL];
#pragma unroll
      for (int t = 0; t < VPL; ++t) P[t] = 0.0f;
      sum_piece<VPL, CONSEC, 4>(a, vl, gbase, cnt, sub, P);
#pragma unroll
      for (int t = 0; t < VPL; ++t) G[t] = G[t] + P[t];
      if (cnt < kPiece) break;
    }
#pragma unroll
    for (int t = 0; t < VPL; ++t) part[grp][col_of<VPL, CONSEC>(sub, t)] = G[t];
    __syncthreads();
    if (grp == 0) {
      float g[VPL];
#pragma unroll
      for (int t = 0; t < VPL; ++t) {
        const int c = col_of<VPL, CONSEC>(sub, t);
        g[t] = part[0][c];
        for (int q = 1; q < kLongGroups; ++q) g[t] = g[t] + part[q][c];
      }
      finish<VPL, CONSEC, ADAM>(a, key, sub, g, p, m, v);
    }
    return;
  }
  const int64_t i = (((int64_t)blockIdx.x - n_long_blocks) * 256 + threadIdx.x) >> 5;
  if (i >= a.n) return;  // uniform per group
  // The window [i, i+32), its neighbours i-1 and i+32: one round of loads.
  const uint32_t kl = (i + sub < a.n) ? a.skeys[i + sub] : 0xffffffffu;
  const uint32_t vl = (i + sub < a.n) ? a.svals[i + sub] : 0u;
  const uint32_t prev = (i > 0) ? a.skeys[i - 1] : 0xffffffffu;
  const uint32_t next = (i + kPiece < a.n) ? a.skeys[i + kPiece] : 0xffffffffu;
  const uint32_t key = (uint32_t)__shfl((int)kl, gbase);
  if ((int64_t)key >= a.n_var) return;  // frozen rows: no variable
  if (prev == key) return;              // not the segment's first slot
  if (next == key) return;              // a long segment: its own workgroup takes it
  float p[VPL], m[VPL], v[VPL];
  if constexpr (ADAM) {  // the state rows do not depend on the gradient: fetch them first
    const int64_t off = (int64_t)key * a.dim;
    load_f32<VPL, CONSEC>(a.master + off, sub, p);
    load_f32<VPL, CONSEC>(a.m + off, sub, m);
    load_f32<VPL, CONSEC>(a.v + off, sub, v);
  }
  const int cnt = __popc((uint32_t)(__ballot(kl == key) >> gbase));
  float g[VPL];
#pragma unroll
  for (int t = 0; t < VPL; ++t) g[t] = 0.0f;
  sum_piece<VPL, CONSEC, 4>(a, vl, gbase, cnt, sub, g);
  finish<VPL, CONSEC, ADAM>(a, key, sub, g, p, m, v);
}

// Dense mode: the variables no slot hit this step take a zero-gradient step.
template <int VPL, bool CONSEC>
__global__ __launch_bounds__(256) void dense_kernel(const SegArgs a) {
  const int sub = threadIdx.x & 31;
  const int64_t k = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 5;
  if (k >= a.n_var) return;
  if (a.stamp[k] == (int32_t)a.step) return;
  float g[VPL], p[VPL], m[VPL], v[VPL];
#pragma unroll
  for (int t = 0; t < VPL; ++t) g[t] = 0.0f;
  const int64_t off = k * a.dim;
  load_f32<VPL, CONSEC>(a.master + off, sub, p);
  load_f32<VPL, CONSEC>(a.m + off, sub, m);
  load_f32<VPL, CONSEC>(a.v + off, sub, v);
  adam_apply<VPL, CONSEC>(a, k, sub, g, p, m, v);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
struct Workspace {
  uint32_t* keys[2];
  uint32_t* vals[2];
  uint32_t* hist[2];
  uint32_t* partial[2];  // per scan chunk, one buffer per pass parity
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static int64_t n_tiles_of(int64_t n) { return (n + kTile - 1) / kTile; }

static size_t partial_bytes(int64_t n) {
  return align256((size_t)((n_tiles_of(n) * kMaxBuckets + kScanChunk - 1) / kScanChunk + 1) * 4);
}

static size_t workspace_bytes(int64_t n) {
  const size_t kb = align256((size_t)n * 4);
  const size_t hb = align256((size_t)n_tiles_of(n) * kMaxBuckets * 4);
  return 4 * kb + 2 * hb + 2 * partial_bytes(n);
}

static Workspace carve(void* ws, int64_t n) {
  Workspace w;
  char* p = (char*)ws;
  const size_t kb = align256((size_t)n * 4);
  const size_t hb = align256((size_t)n_tiles_of(n) * kMaxBuckets * 4);
  w.keys[0] = (uint32_t*)p;
  w.vals[0] = (uint32_t*)(p + kb);
  w.keys[1] = (uint32_t*)(p + 2 * kb);
  w.vals[1] = (uint32_t*)(p + 3 * kb);
  w.hist[0] = (uint32_t*)(p + 4 * kb);
  w.hist[1] = (uint32_t*)(p + 4 * kb + hb);
  w.partial[0] = (uint32_t*)(p + 4 * kb + 2 * hb);
  w.partial[1] = (uint32_t*)(p + 4 * kb + 2 * hb + partial_bytes(n));
  return w;
}

// keys + stable radix sort; *sorted = index (0/1) of the sorted buffers.
static int sort_slots(const int32_t* rows, int64_t n, const int32_t* ids, int64_t n_var, const int64_t* index,
                      int64_t index_capacity, bool direct, const Workspace& w, hipStream_t st, int* sorted) {
  int bits = 0;
  while (bits < 32 && ((uint64_t)n_var >> bits) != 0) ++bits;  // keys lie in [0, n_var]
  const int passes = bits == 0 ? 0 : (bits + kMaxDigitBits - 1) / kMaxDigitBits;
  const int dbits = passes == 0 ? 1 : (bits + passes - 1) / passes;
  int split_shift = 0;
  while (((n_var + (1LL << split_shift) - 1) >> split_shift) > kSplitMax) ++split_shift;
  const int n_tiles = (int)n_tiles_of(n);
  if (direct) {
    hipLaunchKernelGGL(keys_hist_kernel<2>, dim3(n_tiles), dim3(kTileThreads), 0, st, rows, n, ids, n_var, 0,
                       (const unsigned long long*)nullptr, 0, w.keys[0], w.vals[0], dbits, n_tiles, w.hist[0]);
  } else if (index != nullptr) {
    int ib = 0;
    while ((1LL << ib) < index_capacity) ++ib;
    hipLaunchKernelGGL(keys_hist_kernel<1>, dim3(n_tiles), dim3(kTileThreads), 0, st, rows, n, ids, n_var, 0,
                       (const unsigned long long*)index, ib, w.keys[0], w.vals[0], dbits, n_tiles, w.hist[0]);
  } else {
    hipLaunchKernelGGL(keys_hist_kernel<0>, dim3(n_tiles), dim3(kTileThreads), 0, st, rows, n, ids, n_var,
                       split_shift, (const unsigned long long*)nullptr, 0, w.keys[0], w.vals[0], dbits, n_tiles,
                       w.hist[0]);
  }
  int rc = launch_status("keys_hist_kernel");
  if (rc != EG_OK) return rc;
  int cur = 0;
  for (int pass = 0; pass < passes; ++pass) {
    const bool last = pass + 1 == passes;
    uint32_t* h = w.hist[pass & 1];
    uint32_t* h_next = last ? nullptr : w.hist[(pass + 1) & 1];
    const int64_t len = (int64_t)n_tiles << dbits;
    const unsigned chunks = (unsigned)((len + kScanChunk - 1) / kScanChunk);
    // Pass 0 sums its scan chunks here; a later pass's chunk totals are counted
    // by the scatter before it when they fit its LDS (fused), else summed here.
    // What the next scatter accumulates into is cleared before it runs.
    const bool fused = chunks <= (unsigned)kMaxChunksLds;
    uint32_t* part = w.partial[pass & 1];
    uint32_t* part_next = (last || !fused) ? nullptr : w.partial[(pass + 1) & 1];
    if (pass == 0 || !fused)
      hipLaunchKernelGGL(scan_partials, dim3(chunks), dim3(kScanThreads), 0, st, h, len, part, h_next,
                         last ? (int64_t)0 : len);
    else if (!last)
      hipLaunchKernelGGL(scan_partials, dim3(1), dim3(kScanThreads), 0, st, h, (int64_t)0, part_next, h_next, len);
    hipLaunchKernelGGL(scan_apply, dim3(chunks), dim3(kScanThreads), 0, st, h, len, part, part_next,
                       part_next ? (int64_t)chunks + 1 : (int64_t)0);
    hipLaunchKernelGGL(scatter_kernel, dim3(n_tiles), dim3(kTileThreads), 0, st, w.keys[cur], w.vals[cur],
                       w.keys[cur ^ 1], w.vals[cur ^ 1], n, pass * dbits, dbits, n_tiles, h, h_next, part_next,
                       (pass + 1) * dbits, dbits);
    rc = launch_status("radix sort pass");
    if (rc != EG_OK) return rc;
    cur ^= 1;
  }
  *sorted = cur;
  return EG_OK;
}

template <bool ADAM, int VPL, bool CONSEC>
static void launch_reduce_t(const SegArgs& a, hipStream_t st) {
  const int64_t n_long_blocks = (a.n + kPiece) / (kPiece + 1);
  const dim3 grid((unsigned)(n_long_blocks + (a.n * 32 + 255) / 256));
  hipLaunchKernelGGL((reduce_kernel<VPL, CONSEC, ADAM>), grid, dim3(256), 0, st, a, n_long_blocks);
}

template <bool ADAM>
static int launch_reduce(const SegArgs& a, hipStream_t st) {
  switch (a.dim) {
    case 128: launch_reduce_t<ADAM, 4, true>(a, st); break;
    case 64: launch_reduce_t<ADAM, 2, true>(a, st); break;
    case 256: launch_reduce_t<ADAM, 8, true>(a, st); break;
    case 160: launch_reduce_t<ADAM, 5, false>(a, st); break;
    default: return set_error(EG_ERR_UNSUPPORTED, "backward for dim %d (built: 64, 128, 160, 256)", a.dim);
  }
  return launch_status("reduce_kernel");
}

static int launch_dense(const SegArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)((a.n_var * 32 + 255) / 256));
  switch (a.dim) {
    case 128: hipLaunchKernelGGL((dense_kernel<4, true>), grid, dim3(256), 0, st, a); break;
    case 64: hipLaunchKernelGGL((dense_kernel<2, true>), grid, dim3(256), 0, st, a); break;
    case 256: hipLaunchKernelGGL((dense_kernel<8, true>), grid, dim3(256), 0, st, a); break;
    case 160: hipLaunchKernelGGL((dense_kernel<5, false>), grid, dim3(256), 0, st, a); break;
    default: return set_error(EG_ERR_UNSUPPORTED, "backward for dim %d", a.dim);
  }
  return launch_status("dense_kernel");
}

static int check_common(const void* d_out, const int32_t* rows, int64_t n_pos, int32_t heads, int32_t dim,
                        const int32_t* ids, int64_t n_var, void* ws, size_t ws_bytes) {
  EG_CHECK_ARG(n_pos >= 0 && heads >= 1 && heads <= EG_MAX_HEADS, "n_pos=%lld heads=%d", (long long)n_pos, heads);
  EG_CHECK_ARG(dim == 64 || dim == 128 || dim == 160 || dim == 256, "backward dim=%d (built: 64, 128, 160, 256)",
               dim);
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

int eg_build_row_index(const int32_t* ids, int64_t n, int64_t* table, int64_t capacity, void* stream) {
  EG_CHECK_ARG(n >= 0 && n < (1LL << 31), "n=%lld", (long long)n);
  EG_CHECK_ARG(capacity >= 2 && capacity >= 2 * n && (capacity & (capacity - 1)) == 0 && capacity <= (1LL << 32),
               "capacity=%lld must be a power of two >= 2*n", (long long)capacity);
  EG_CHECK_ARG(table != nullptr && (n == 0 || ids != nullptr), "ids/table is NULL");
  int bits = 0;
  while ((1LL << bits) < capacity) ++bits;
  hipStream_t st = (hipStream_t)stream;
  const int64_t fill_blocks = (capacity + 255) / 256;
  hipLaunchKernelGGL(index_fill_kernel, dim3((unsigned)(fill_blocks < 4096 ? fill_blocks : 4096)), dim3(256), 0, st,
                     (unsigned long long*)table, capacity);
  if (n > 0)
    hipLaunchKernelGGL(index_build_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, ids, n,
                       (unsigned long long*)table, bits);
  return launch_status("row index kernels");
}

static int scatter_grad_impl(const void* d_out, int32_t d_out_f32, const int32_t* rows, int64_t n_pos,
                             int32_t heads, int32_t dim, const int32_t* ids, int64_t n_var, bool direct,
                             float* grad_out, void* workspace, size_t workspace_bytes_, void* stream) {
  int rc = check_common(d_out, rows, n_pos, heads, dim, direct ? (const int32_t*)rows : ids, n_var, workspace,
                        workspace_bytes_);
  if (rc != EG_OK) return rc;
  EG_CHECK_ARG(n_var == 0 || grad_out != nullptr, "grad_out is NULL");
  const int64_t n = n_pos * heads;
  if (n == 0 || n_var == 0) return EG_OK;
  hipStream_t st = (hipStream_t)stream;
  const Workspace w = carve(workspace, n);
  int cur = 0;
  rc = sort_slots(rows, n, ids, n_var, nullptr, 0, direct, w, st, &cur);
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
  return launch_reduce<false>(a, st);
}

int eg_scatter_grad(const void* d_out, int32_t d_out_f32, const int32_t* rows, int64_t n_pos, int32_t heads,
                    int32_t dim, const int32_t* ids, int64_t n_var, float* grad_out, void* workspace,
                    size_t workspace_bytes_, void* stream) {
  return scatter_grad_impl(d_out, d_out_f32, rows, n_pos, heads, dim, ids, n_var, false, grad_out, workspace,
                           workspace_bytes_, stream);
}

int eg_scatter_grad_slots(const void* d_out, int32_t d_out_f32, const int32_t* slot_var, int64_t n_pos,
                          int32_t heads, int32_t dim, int64_t n_var, float* grad_out, void* workspace,
                          size_t workspace_bytes_, void* stream) {
  return scatter_grad_impl(d_out, d_out_f32, slot_var, n_pos, heads, dim, nullptr, n_var, true, grad_out, workspace,
                           workspace_bytes_, stream);
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
  EG_CHECK_ARG(opt->lr >= 0.0 && opt->beta1 >= 0.0 && opt->beta1 < 1.0 && opt->beta2 >= 0.0 && opt->beta2 < 1.0 &&
                   opt->eps >= 0.0,
               "invalid Adam hyper-parameters");
  if (state->index != nullptr)
    EG_CHECK_ARG(state->index_capacity >= 2 * state->n && state->index_capacity >= 2 &&
                     (state->index_capacity & (state->index_capacity - 1)) == 0 && state->index_capacity <= (1LL << 32),
                 "index_capacity=%lld must be a power of two >= 2*n", (long long)state->index_capacity);
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
    rc = sort_slots(rows, n, state->ids, state->n, state->index, state->index_capacity, false, w, st, &cur);
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
  a.dense = opt->dense != 0;
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
    rc = launch_reduce<true>(a, st);
    if (rc != EG_OK) return rc;
  }
  if (opt->dense) rc = launch_dense(a, st);
  return rc;
}

}  // extern "C"
