// Backward half of the n-gram table path on gfx950: the deterministic sparse
// gradient scatter and the optimizer step on the touched overlay rows.
//
//   keys     slot s = p*heads + h -> variable index k of rows[s] (an LDS
//            splitter search of the sorted ids, a probe of the row index, or
//            given directly); every variable's slot count is accumulated
//   offsets  exclusive scan of the counts; variables hit by more than 32
//            slots are listed
//   fill     every slot id is written at its variable's range start plus the
//            rank its counting atomic returned (CSR, no atomics); the order
//            inside a range is whatever the counting atomics gave
//   order    each range is put in ascending slot order inside the reduction:
//            ranges of at most 32 slots by a 32-lane bitonic network on
//            registers, longer ones by their workgroup (LDS bitonic network,
//            or the same network on global memory beyond the LDS capacity)
//   segment  one 32-lane group per variable hit by at most 32 slots sums the
//            slots' d_out slices in ascending slot order (fp32) and runs
//            Adam + requantisation; a longer range is reduced by a whole
//            workgroup: pieces of 32 slots summed in order, piece j added to
//            group j mod 8's sum, the eight group sums added in group order
//   dense    variables no slot hit take their zero-gradient step (dense mode)
//
// No floating-point atomics: the association of every sum is fixed by the
// ascending slot order alone, so results are bitwise repeatable, and the CPU
// oracle reproduces them exactly.
#include <string.h>

#include <mutex>

#include "eg_common.h"

namespace eg {

constexpr int kTileThreads = 256;
constexpr int kTileIPT = 2;                       // lockstep lookups per thread in the keys kernel
constexpr int kTile = kTileThreads * kTileIPT;    // slots per keys workgroup
constexpr int kScanThreads = 1024;
constexpr int kSplitMax = 2048;  // splitters staged in LDS (8 KB)
constexpr int kPiece = 32;       // slots per piece of a long segment
constexpr int kLongGroups = 8;   // 32-lane groups per long-segment workgroup

// ---------------------------------------------------------------------------
// Row index: open addressing over a power-of-two table of (row << 32 | k)
// entries (at least 8), Fibonacci hashing, linear probing from the start of the
// aligned group of 8 entries (64 bytes) that holds the hash slot: a lookup reads
// whole groups, and at most a quarter full a row's group holds it (or an empty
// entry) for all but ~1e-4 of the lookups.  Lookups are deterministic whatever
// order the entries were inserted in.
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
  uint64_t h = index_slot(row, bits) & ~7ull;
  for (uint64_t probe = 0; probe <= mask; ++probe) {  // the table is at most half full
    if (atomicCAS(&tab[h], kIndexEmpty, packed) == kIndexEmpty) return;
    h = (h + 1) & mask;
  }
}

// ---------------------------------------------------------------------------
// Keys + per-variable counts
// ---------------------------------------------------------------------------
// Variable index (key) of IPT slots per thread, the slots of thread tid of a
// block of NT threads at base + r*NT + tid.  MODE 0: search the sorted ids
// (level 1 in the LDS splitters spl[0, ns)); 1: probe the row index; 2: rows
// already hold variable indices.  key = n_var: no variable (or idx >= n).
// The IPT lookups of a thread run in lockstep and every load is issued
// unconditionally (indices clamped in range, results masked): a load inside a
// lane-divergent branch would be waited for inside it, which would serialise
// the lookups.
template <int MODE, int IPT, int NT>
__device__ inline void slot_keys(const int32_t* __restrict__ rows, int64_t n, int64_t base, int tid,
                                 const int32_t* __restrict__ ids, int64_t n_var, int split_shift, const int32_t* spl,
                                 int ns, const unsigned long long* __restrict__ index, int index_bits,
                                 uint32_t key[IPT], bool ok[IPT]) {
  int32_t row[IPT];
#pragma unroll
  for (int r = 0; r < IPT; ++r) {
    const int64_t idx = base + r * NT + tid;
    ok[r] = idx < n;
    row[r] = rows[ok[r] ? idx : n - 1];
  }
  if constexpr (MODE == 2) {
#pragma unroll
    for (int r = 0; r < IPT; ++r)
      key[r] = (ok[r] && row[r] >= 0 && (int64_t)row[r] < n_var) ? (uint32_t)row[r] : (uint32_t)n_var;
  } else if constexpr (MODE == 1) {
    // probe the row index a group of 8 entries at a time, the row's group
    // first (the linear probe's order): one round of loads settles a
    // wavefront's lookups but for ~1 % of the wavefronts.  The items' probes
    // advance in lockstep.
    const uint64_t imask = (1ull << index_bits) - 1ull;
    uint64_t grp[IPT];
    bool done[IPT];
#pragma unroll
    for (int r = 0; r < IPT; ++r) {
      grp[r] = index_slot(row[r], index_bits) & ~7ull;
      done[r] = !ok[r];
      key[r] = (uint32_t)n_var;
    }
    for (uint64_t probe = 0; probe <= (imask >> 3); ++probe) {  // every group once
      bool any = false;
      ulonglong2 e[IPT][4];
#pragma unroll
      for (int r = 0; r < IPT; ++r)
#pragma unroll
        for (int q = 0; q < 4; ++q) e[r][q] = ((const ulonglong2*)(index + grp[r]))[q];
#pragma unroll
      for (int r = 0; r < IPT; ++r) {
        if (done[r]) continue;
        bool fin = false;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const unsigned long long ent = (j & 1) ? e[r][j >> 1].y : e[r][j >> 1].x;
          if (!fin) {
            if (ent == kIndexEmpty) {
              fin = true;
            } else if ((uint32_t)(ent >> 32) == (uint32_t)row[r]) {
              key[r] = (uint32_t)ent;
              fin = true;
            }
          }
        }
        if (fin) {
          done[r] = true;
        } else {
          grp[r] = (grp[r] + 8) & imask;
          any = true;
        }
      }
      if (!any) break;
    }
  } else {
    // level 1 (LDS): lo = number of splitters <= row
    int lo[IPT];
#pragma unroll
    for (int r = 0; r < IPT; ++r) lo[r] = 0;
    for (int step = kSplitMax; step >= 1; step >>= 1) {
#pragma unroll
      for (int r = 0; r < IPT; ++r)
        if (lo[r] + step <= ns && spl[lo[r] + step - 1] <= row[r]) lo[r] += step;
    }
    // level 2 (global): the last id <= row inside that splitter's window
    const int64_t win = 1LL << split_shift;
    int64_t pos[IPT], end[IPT];
#pragma unroll
    for (int r = 0; r < IPT; ++r) {
      pos[r] = lo[r] > 0 ? ((int64_t)(lo[r] - 1) << split_shift) : 0;
      end[r] = lo[r] > 0 ? min(pos[r] + win, n_var) : 0;
    }
    for (int64_t step = win >> 1; step >= 1; step >>= 1) {
      int32_t probe[IPT];
#pragma unroll
      for (int r = 0; r < IPT; ++r) probe[r] = ids[min(pos[r] + step, n_var - 1)];
#pragma unroll
      for (int r = 0; r < IPT; ++r)
        if (pos[r] + step < end[r] && probe[r] <= row[r]) pos[r] += step;
    }
#pragma unroll
    for (int r = 0; r < IPT; ++r) {
      const int32_t at = ids[pos[r]];
      key[r] = (ok[r] && lo[r] > 0 && at == row[r]) ? (uint32_t)pos[r] : (uint32_t)n_var;
    }
  }
}

// Splitters of the sorted ids for slot_keys<0>: every 2^split_shift-th id.
__device__ inline int load_splitters(const int32_t* __restrict__ ids, int64_t n_var, int split_shift, int32_t* spl,
                                     int tid, int nt) {
  const int ns = (int)((n_var + (1LL << split_shift) - 1) >> split_shift);
  for (int i = tid; i < ns; i += nt) spl[i] = ids[(int64_t)i << split_shift];
  return ns;
}

// Keys + per-variable counts (the grouping for more than kBucketsMax buckets).
// cnt[k] += the slots of k; ranks[s] = the count of k before slot s was
// counted (its place in k's range).
template <int MODE>
__global__ __launch_bounds__(kTileThreads) void keys_count_kernel(
    const int32_t* __restrict__ rows, int64_t n, const int32_t* __restrict__ ids, int64_t n_var, int split_shift,
    const unsigned long long* __restrict__ index, int index_bits, uint32_t* __restrict__ keys,
    uint32_t* __restrict__ ranks, uint32_t* __restrict__ cnt) {
  __shared__ int32_t spl[kSplitMax];
  const int tid = threadIdx.x;
  int ns = 0;
  if constexpr (MODE == 0) {
    ns = load_splitters(ids, n_var, split_shift, spl, tid, kTileThreads);
    __syncthreads();
  }
  uint32_t key[kTileIPT];
  bool ok[kTileIPT];
  slot_keys<MODE, kTileIPT, kTileThreads>(rows, n, (int64_t)blockIdx.x * kTile, tid, ids, n_var, split_shift, spl, ns,
                                          index, index_bits, key, ok);
#pragma unroll
  for (int r = 0; r < kTileIPT; ++r) {
    if (!ok[r]) continue;
    const int64_t idx = (int64_t)blockIdx.x * kTile + r * kTileThreads + tid;
    keys[idx] = key[r];
    if ((int64_t)key[r] < n_var) ranks[idx] = atomicAdd(&cnt[key[r]], 1u);
  }
}

// ---------------------------------------------------------------------------
// Bucketed grouping: two launches, no global atomics, no waits between workgroups
// ---------------------------------------------------------------------------
// Bucket b holds the variables [b << bs, (b + 1) << bs).
// tile_sort_kernel: tile t (kGroupTile slots) computes its slots' keys and
//   counting-sorts its (key, slot) pairs by bucket in LDS into its own region
//   pairs[t * kGroupTile, ...), writing per bucket the segment
//   seg[b][t] = count << 16 | offset, the offset being the slots of t in
//   the buckets before b (bucket-major: a bucket reads its segments of every
//   tile as one contiguous run).
// bucket_ranges_kernel: bucket b gathers its pairs from every tile, counts
//   its keys in LDS and writes every variable's range [start, end) and its
//   slot ids (in no particular order inside a range: the reduction orders
//   them).  Its region of the slots array starts at the slots of every tile
//   in the earlier buckets, which is the sum over t of its own segments'
//   offsets: each bucket finds it alone.  Its variables of more than kPiece
//   slots are appended to the long list (one atomic a bucket on its length,
//   which the tile sort zeroes): the list is dense, in no particular order.
// A tile of 1,024 slots, one a thread: the row-index probe is a chain of
// dependent loads, and 16 wavefronts a CU hide it better than 8 of two slots
// each (config 2's step 148.5 against 150.1 us, the same result bit for bit).
constexpr int kGroupThreads = 1024;
constexpr int kGroupIPT = 1;
constexpr int kGroupTile = kGroupThreads * kGroupIPT;  // slots per tile
constexpr int kBucketsMax = 1024;
constexpr uint32_t kNoVar = 0xffffffffu;                // an unused entry of the long list
constexpr int kBucketKeysLog2Max = 11;                 // at most 2048 variables per bucket
// 512 threads a bucket: one of its 512 variables a thread in the count, scan and
// range writes (148.0 against 149.1 us a config-2 step with 256, bitwise the same)
constexpr int kRangeThreads = 512;
constexpr int kRangeTilesMax = 1024;                // tiles bucket_ranges_kernel reads (at most 2 a thread)

// Exclusive scan of x[0, len) in LDS by a block of NT threads (len <= PER * NT).
template <int NT, int PER>
__device__ inline void lds_exclusive_scan(uint32_t* x, int len, uint32_t* wsum) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t v[PER];
  uint32_t t = 0;
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int i = tid * PER + u;
    v[u] = i < len ? x[i] : 0u;
    t += v[u];
  }
  uint32_t incl = t;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  uint32_t before = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w)
    if (w < wave) before += wsum[w];
  uint32_t run = before + incl - t;
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int i = tid * PER + u;
    if (i < len) x[i] = run;
    run += v[u];
  }
  __syncthreads();
}

template <int MODE>
__global__ __launch_bounds__(kGroupThreads) void tile_sort_kernel(
    const int32_t* __restrict__ rows, int64_t n, const int32_t* __restrict__ ids, int64_t n_var, int split_shift,
    const unsigned long long* __restrict__ index, int index_bits, int bs, int nb, int64_t n_tiles,
    unsigned long long* __restrict__ pairs, uint32_t* __restrict__ seg, uint32_t* __restrict__ n_long) {
  __shared__ int32_t spl[MODE == 0 ? kSplitMax : 1];
  __shared__ uint32_t bh[kBucketsMax];
  __shared__ uint32_t wsum[kGroupThreads / 64];
  const int tid = threadIdx.x;
  const int64_t t = blockIdx.x;
  if (t == 0 && tid == 0) *n_long = 0u;  // the long list's length, counted by the next launch
  for (int i = tid; i < nb; i += kGroupThreads) bh[i] = 0u;
  int ns = 0;
  if constexpr (MODE == 0) ns = load_splitters(ids, n_var, split_shift, spl, tid, kGroupThreads);
  __syncthreads();
  uint32_t key[kGroupIPT];
  bool ok[kGroupIPT];
  slot_keys<MODE, kGroupIPT, kGroupThreads>(rows, n, t * kGroupTile, tid, ids, n_var, split_shift, spl, ns, index,
                                            index_bits, key, ok);
  uint32_t rank[kGroupIPT];
#pragma unroll
  for (int r = 0; r < kGroupIPT; ++r) {
    rank[r] = 0u;
    if (ok[r] && (int64_t)key[r] < n_var) rank[r] = atomicAdd(&bh[key[r] >> bs], 1u);
  }
  __syncthreads();
  uint32_t cnt_b[kBucketsMax / kGroupThreads];
#pragma unroll
  for (int u = 0; u < kBucketsMax / kGroupThreads; ++u) {
    const int b = tid + u * kGroupThreads;
    cnt_b[u] = b < nb ? bh[b] : 0u;
  }
  __syncthreads();
  lds_exclusive_scan<kGroupThreads, kBucketsMax / kGroupThreads>(bh, nb, wsum);
#pragma unroll
  for (int u = 0; u < kBucketsMax / kGroupThreads; ++u) {
    const int b = tid + u * kGroupThreads;
    if (b < nb) seg[(int64_t)b * n_tiles + t] = cnt_b[u] << 16 | bh[b];  // both <= kGroupTile
  }
#pragma unroll
  for (int r = 0; r < kGroupIPT; ++r) {
    if (ok[r] && (int64_t)key[r] < n_var) {
      const int64_t s = t * kGroupTile + r * kGroupThreads + tid;
      pairs[t * kGroupTile + bh[key[r] >> bs] + rank[r]] = ((unsigned long long)key[r] << 32) | (uint32_t)s;
    }
  }
}

template <int TPT>
__global__ __launch_bounds__(kRangeThreads) void bucket_ranges_kernel(
    const unsigned long long* __restrict__ pairs, const uint32_t* __restrict__ seg, int64_t n_tiles, int nb, int bs,
    int64_t n_var, uint32_t* __restrict__ start, uint32_t* __restrict__ end,
    uint32_t* __restrict__ slots, uint32_t* __restrict__ long_list, uint32_t* __restrict__ n_long) {
  constexpr int kKeys = 1 << kBucketKeysLog2Max;
  constexpr int kKeep = 4;                         // pairs of one tile a thread holds in registers
  __shared__ uint32_t cnt[kKeys];                  // pairs held in registers, per variable
  __shared__ uint32_t over[kKeys];                 // pairs beyond kKeep of a tile, per variable
  __shared__ uint32_t lst[kKeys];
  __shared__ uint32_t lng[kKeys];                  // the bucket's variables of more than kPiece slots
  __shared__ uint32_t wsum[2][kRangeThreads / 64];
  __shared__ uint32_t n_long_b, long_at;
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.x;
  const int64_t key0 = b << bs;
  const int nkeys = (int)min((int64_t)1 << bs, n_var - key0);
  for (int i = tid; i < nkeys; i += kRangeThreads) {
    cnt[i] = 0u;
    over[i] = 0u;
  }
  if (tid == 0) n_long_b = 0u;
  // this thread's tiles: (count, offset) of the bucket's segment in each; the
  // offsets add up to the bucket's place in the slots array
  constexpr int kTilesPerThread = TPT;  // n_tiles <= TPT * kRangeThreads (the host picks TPT)
  u32x2 sg[kTilesPerThread];
  uint32_t tot = 0, pre = 0;
#pragma unroll
  for (int j = 0; j < kTilesPerThread; ++j) {
    const int64_t t = tid + (int64_t)j * kRangeThreads;
    const uint32_t e = t < n_tiles ? seg[b * n_tiles + t] : 0u;
    sg[j] = u32x2{e >> 16, e & 0xffffu};
    tot += sg[j].x;
    pre += sg[j].y;
  }
  // the first kKeep pairs of each tile segment: loaded together, counted, and
  // given their rank among the variable's register-held pairs
  unsigned long long pr[kTilesPerThread][kKeep];
  uint32_t rk[kTilesPerThread][kKeep];
#pragma unroll
  for (int j = 0; j < kTilesPerThread; ++j) {
    const int64_t t = tid + (int64_t)j * kRangeThreads;
    // an empty segment's offset may equal the tile's size: read the tile's first pair instead (unused)
    const unsigned long long* src = pairs + (t < n_tiles ? t : 0) * kGroupTile + (sg[j].x ? sg[j].y : 0u);
#pragma unroll
    for (int e = 0; e < kKeep; ++e) pr[j][e] = src[(uint32_t)e < sg[j].x ? e : 0];
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    tot += __shfl_xor(tot, o);
    pre += __shfl_xor(pre, o);
  }
  if ((tid & 63) == 0) {
    wsum[0][tid >> 6] = tot;
    wsum[1][tid >> 6] = pre;
  }
  __syncthreads();  // (also closes the zeroing of the counts)
#pragma unroll
  for (int j = 0; j < kTilesPerThread; ++j)
#pragma unroll
    for (int e = 0; e < kKeep; ++e)
      rk[j][e] = ((uint32_t)e < sg[j].x) ? atomicAdd(&cnt[(uint32_t)(pr[j][e] >> 32) - (uint32_t)key0], 1u) : 0u;
  // the rest of a long segment (a variable hit many times in one tile): counted apart
#pragma unroll
  for (int j = 0; j < kTilesPerThread; ++j) {
    if (sg[j].x <= (uint32_t)kKeep) continue;
    const unsigned long long* src = pairs + (tid + (int64_t)j * kRangeThreads) * kGroupTile + sg[j].y;
    for (uint32_t e = kKeep; e < sg[j].x; ++e) atomicAdd(&over[(uint32_t)(src[e] >> 32) - (uint32_t)key0], 1u);
  }
  uint32_t total = 0, base = 0;
#pragma unroll
  for (int w = 0; w < kRangeThreads / 64; ++w) {
    total += wsum[0][w];
    base += wsum[1][w];
  }
  __syncthreads();
  for (int i = tid; i < nkeys; i += kRangeThreads) lst[i] = cnt[i] + over[i];
  __syncthreads();
  lds_exclusive_scan<kRangeThreads, kKeys / kRangeThreads>(lst, nkeys, wsum[0]);
  for (int i = tid; i < nkeys; i += kRangeThreads) {
    const uint32_t c = cnt[i] + over[i];
    start[key0 + i] = base + lst[i];
    end[key0 + i] = base + lst[i] + c;
    if (c > (uint32_t)kPiece) lng[atomicAdd(&n_long_b, 1u)] = (uint32_t)(key0 + i);
    over[i] = lst[i] + cnt[i];  // where the variable's overflow pairs go
  }
  __syncthreads();
  // the bucket's long variables, appended to the list (its order is free: each
  // long variable is reduced by one workgroup, whichever entry holds it)
  if (tid == 0) long_at = n_long_b ? atomicAdd(n_long, n_long_b) : 0u;
  __syncthreads();
  for (uint32_t j = tid; j < n_long_b; j += kRangeThreads) long_list[long_at + j] = lng[j];
  // every slot id at its variable's place (the order inside a range is free)
#pragma unroll
  for (int j = 0; j < kTilesPerThread; ++j)
#pragma unroll
    for (int e = 0; e < kKeep; ++e)
      if ((uint32_t)e < sg[j].x) {
        const uint32_t i = (uint32_t)(pr[j][e] >> 32) - (uint32_t)key0;
        slots[base + lst[i] + rk[j][e]] = (uint32_t)pr[j][e];
      }
#pragma unroll
  for (int j = 0; j < kTilesPerThread; ++j) {
    if (sg[j].x <= (uint32_t)kKeep) continue;
    const unsigned long long* src = pairs + (tid + (int64_t)j * kRangeThreads) * kGroupTile + sg[j].y;
    for (uint32_t e = kKeep; e < sg[j].x; ++e) {
      const unsigned long long q = src[e];
      const uint32_t i = (uint32_t)(q >> 32) - (uint32_t)key0;
      slots[base + atomicAdd(&over[i], 1u)] = (uint32_t)q;
    }
  }
}

// a[0, len) = 0 and l[0, l_len) = kNoVar.
__global__ __launch_bounds__(256) void clear_kernel(uint32_t* __restrict__ a, int64_t len, uint32_t* __restrict__ l,
                                                    int64_t l_len) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < len; i += (int64_t)gridDim.x * 256) a[i] = 0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < l_len; i += (int64_t)gridDim.x * 256) l[i] = kNoVar;
}

// ---------------------------------------------------------------------------
// Exclusive scan (two kernels over 4096-entry chunks), in place
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

// Pass 1: the total of every chunk.
__global__ __launch_bounds__(kScanThreads) void scan_partials(const uint32_t* __restrict__ a, int64_t len,
                                                              uint32_t* __restrict__ partial) {
  __shared__ uint32_t wsum[kScanThreads / 64];
  const int tid = threadIdx.x;
  const int64_t i0 = (int64_t)blockIdx.x * kScanChunk + 4 * tid;
  uint32_t t = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) t += (i0 + u < len) ? a[i0 + u] : 0u;
  uint32_t total;
  block_exclusive_scan(t, wsum, &total);
  if (tid == 0) partial[blockIdx.x] = total;
}

// Pass 2: exclusive scan of every chunk, offset by the totals of the chunks
// before it.  Entries whose count exceeds kPiece are appended to long_list.
__global__ __launch_bounds__(kScanThreads) void scan_apply(uint32_t* __restrict__ a, int64_t len,
                                                           const uint32_t* __restrict__ partial,
                                                           uint32_t* __restrict__ long_list,
                                                           uint32_t* __restrict__ n_long) {
  __shared__ uint32_t wsum[kScanThreads / 64];
  __shared__ uint32_t wsum2[kScanThreads / 64];
  const int tid = threadIdx.x;
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
    if (i0 + u < len) {
      a[i0 + u] = run;
      if (v[u] > (uint32_t)kPiece) long_list[atomicAdd(n_long, 1u)] = (uint32_t)(i0 + u);
    }
    run += v[u];
  }
}

// ---------------------------------------------------------------------------
// CSR fill and the ordering of long ranges
// ---------------------------------------------------------------------------
// off[k] enters as variable k's first position and leaves as its end.
__global__ __launch_bounds__(256) void fill_kernel(const uint32_t* __restrict__ keys,
                                                   const uint32_t* __restrict__ ranks, int64_t n, int64_t n_var,
                                                   const uint32_t* __restrict__ start, uint32_t* __restrict__ slots) {
  const int64_t s = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (s >= n) return;
  const uint32_t k = keys[s];
  if ((int64_t)k < n_var) slots[start[k] + ranks[s]] = (uint32_t)s;
}

// Ascending order of x[0, len) with the bitonic network in its one-direction
// form: for each block size k, compare i with i ^ (k-1), then i with i ^ j for
// j = k/4 .. 1, the smaller value to the lower index.  Entries at len and
// beyond count as +infinity, so comparisons that reach them are skipped.
template <typename Ptr>
__device__ void bitonic_sort(Ptr x, int64_t len) {
  int64_t P = 1;
  while (P < len) P <<= 1;
  for (int64_t k = 2; k <= P; k <<= 1) {
    for (int64_t j = k >> 1; j > 0; j >>= 1) {
      for (int64_t i = threadIdx.x; i < (P >> 1); i += blockDim.x) {
        const int64_t lo = ((i & ~(j - 1)) << 1) | (i & (j - 1));  // i with a zero bit inserted at j
        const int64_t hi = (j == (k >> 1)) ? (lo ^ (k - 1)) : (lo + j);
        if (hi < len) {
          const uint32_t u = x[lo], w = x[hi];
          if (w < u) {
            x[lo] = w;
            x[hi] = u;
          }
        }
      }
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------------------
// Segmented reduction + optimizer
// ---------------------------------------------------------------------------
struct SegArgs {
  const uint32_t* start;      // [n_var] start of each variable's range in slots
  const uint32_t* end;        // [n_var] its end
  const uint32_t* slots;      // slot ids grouped by variable (CSR)
  const uint32_t* long_list;  // variables with more than kPiece slots, the first *long_count entries
  const uint32_t* long_count;
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
  int64_t stride;         // floats from one variable's master / m / v row to the next
  int32_t* stamp;
  TableDev quant;         // fmt 0: no requantised copy
  TableDev base;          // for the pull term (rows0 at the variables' ids)
  const float* anchor;    // or rows0 per variable [n_var, dim]
  int64_t step;
  int32_t dense;          // stamp the rows hit (the dense pass skips them)
  float w1, b2, w2, bc2s, eps, neg_step_size, l2c;
  int32_t overwrite;      // gradient mode: grad_out = the sum (0 for a variable no slot hits), not +=
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

// d_out slice of one slot (F32: f32, else bf16), VPL values of this lane.
template <int VPL, bool CONSEC, bool F32>
__device__ inline void load_grad(const SegArgs& a, uint32_t slot, int sub, float x[VPL]) {
  const int64_t p = slot / (uint32_t)a.heads;
  const int h = (int)(slot - p * a.heads);
  const int64_t base = p * a.width + (int64_t)h * a.dim;
  if constexpr (F32) {
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

// Sums the d_out slices of `cnt` (1..32) consecutive sorted slots whose slot
// ids sit in lane (gbase + e) of `vl`, in order, onto g.  Loads go out kBatch
// slots at a time, all of them issued (a slot past cnt re-reads the first one,
// unused): a load inside a lane-divergent branch would be waited for there.
// The additions stay in slot order.
template <int VPL, bool CONSEC, int kBatch, bool F32>
__device__ inline void sum_piece(const SegArgs& a, uint32_t vl, int gbase, int cnt, int sub, float g[VPL]) {
  const uint32_t s0 = (uint32_t)__shfl((int)vl, gbase);
  for (int e0 = 0; e0 < cnt; e0 += kBatch) {
    float x[kBatch][VPL];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const uint32_t s = (uint32_t)__shfl((int)vl, gbase + ((e0 + u) & 31));
      load_grad<VPL, CONSEC, F32>(a, e0 + u < cnt ? s : s0, sub, x[u]);
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (e0 + u < cnt) {
#pragma unroll
        for (int t = 0; t < VPL; ++t) g[t] = g[t] + x[u][t];
      }
  }
}

// Row k of the Q8_0 / MXFP8 store q from the fp32 values p this lane owns
// (the 32 lanes of a row together): Q8_0 d = fp16(amax/127), q = rint(x/d)
// clamped to +-127; MXFP8 the smallest shared exponent e with amax*2^-e <= 448.
template <int VPL, bool CONSEC>
__device__ void requant_row(const TableDev& q, int64_t k, int dim, int sub, const float p[VPL]) {
  const int64_t off = k * dim;
  const int nb = dim >> 5;
  uint8_t* payload = (uint8_t*)q.payload;
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
    if (q.fmt == EG_FMT_Q8_0) {
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
      if (sub % kLanesPerBlock == 0) ((uint16_t*)q.scales)[k * nb + blk] = dh;
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
      if (sub % kLanesPerBlock == 0) ((uint8_t*)q.scales)[k * nb + blk] = (uint8_t)(e + 127);
    }
    if constexpr (VPL == 4) *(uint32_t*)(payload + off + sub * 4) = packed;
  } else {
#pragma unroll
    for (int t = 0; t < VPL; ++t) {
      float amax = fabsf(p[t]);
#pragma unroll
      for (int o = 16; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 32));
      const int64_t qi = off + sub + 32 * t;
      if (q.fmt == EG_FMT_Q8_0) {
        const uint16_t dh = f32_to_f16(amax / 127.0f);
        const float d = f16_to_f32(dh);
        float r = (d == 0.0f) ? 0.0f : rintf(p[t] / d);
        r = fminf(fmaxf(r, -127.0f), 127.0f);
        payload[qi] = (uint8_t)(int32_t)r;
        if (sub == 0) ((uint16_t*)q.scales)[k * nb + t] = dh;
      } else {
        const int ebits = (int)((__float_as_uint(amax) >> 23) & 0xffu);
        int e = (amax > 0.0f ? ebits - 127 : -127) - 8;
        e = min(max(e, -127), 127);
        if (amax * ldexpf(1.0f, -e) > 448.0f) e = min(e + 1, 127);
        payload[qi] = (uint8_t)f32_to_e4m3(fminf(fmaxf(p[t] * ldexpf(1.0f, -e), -448.0f), 448.0f));
        if (sub == 0) ((uint8_t*)q.scales)[k * nb + t] = (uint8_t)(e + 127);
      }
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
      const float p0 = a.anchor != nullptr ? a.anchor[k * a.dim + col_of<VPL, CONSEC>(sub, t)]
                       : ((uint32_t)row0 < (uint64_t)a.base.n_rows)
                           ? load_value_rt(a.base, row0, col_of<VPL, CONSEC>(sub, t))
                           : __uint_as_float(0x7fc00000u);
      gt = gt + a.l2c * (2.0f * (p[t] - p0));
    }
    m[t] = m[t] + a.w1 * (gt - m[t]);
    v[t] = v[t] * a.b2 + (a.w2 * gt) * gt;
    const float denom = sqrtf(v[t]) / a.bc2s + a.eps;
    p[t] = p[t] + a.neg_step_size * (m[t] / denom);
  }
  const int64_t off = k * a.stride;
  store_f32<VPL, CONSEC>(a.master + off, sub, p);
  store_f32<VPL, CONSEC>(a.m + off, sub, m);
  store_f32<VPL, CONSEC>(a.v + off, sub, v);
  if (a.quant.fmt != 0) requant_row<VPL, CONSEC>(a.quant, k, a.dim, sub, p);
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
    if (a.overwrite) {
      // the sum starts from +0, so it is never -0: storing it is bit-identical
      // to adding it to a zeroed buffer
      store_f32<VPL, CONSEC>(dst, sub, g);
    } else {
      float cur[VPL];
      load_f32<VPL, CONSEC>(dst, sub, cur);
#pragma unroll
      for (int t = 0; t < VPL; ++t) cur[t] = cur[t] + g[t];
      store_f32<VPL, CONSEC>(dst, sub, cur);
    }
  }
}

// Ascending sort of one value per lane over the first `span` lanes of each
// 32-lane group (bitonic, one-direction form; span a wavefront-uniform power
// of two in [1, 32]; the lanes from span on already hold the largest values
// and stay in place).
__device__ inline uint32_t sort32(uint32_t v, int sub, int span = 32) {
  for (int k = 2; k <= span; k <<= 1) {
    {
      const uint32_t o = (uint32_t)__shfl_xor((int)v, k - 1, 32);
      v = (sub < (sub ^ (k - 1))) ? min(v, o) : max(v, o);
    }
    for (int j = k >> 2; j > 0; j >>= 1) {
      const uint32_t o = (uint32_t)__shfl_xor((int)v, j, 32);
      v = ((sub & j) == 0) ? min(v, o) : max(v, o);
    }
  }
  return v;
}

// One launch for every variable hit.  The workgroups of the long list (the
// first n_long_head of the grid and every one after the n_short_blocks that
// follow them) take the listed variables of more than kPiece slots: the
// workgroup puts the variable's slot ids in ascending order (in LDS up to
// kLongLds ids, else in place on global memory), sums pieces of kPiece slots
// in order, adds piece j to group j mod kLongGroups and the group sums in
// group order.  The head is dispatched first, so the longer chains overlap the
// rest.  Every short workgroup holds eight 32-lane groups, one per variable: a
// variable of 1..kPiece slots loads its slot ids, sorts them on the lanes and
// reduces them in order.
constexpr int kLongLds = kLongGroups * 512;  // slot ids a long range orders in LDS (the partial-sum buffer)

template <int VPL, bool CONSEC, bool ADAM, bool F32>
__global__ __launch_bounds__(256) void reduce_kernel(const SegArgs a, int64_t n_long_head, int64_t n_short_blocks) {
  __shared__ uint32_t lds[kLongLds];
  float* part = (float*)lds;  // [kLongGroups][512] once the slot ids are no longer needed
  const int lane = threadIdx.x & 63, sub = lane & 31, gbase = lane & 32;
  const int64_t bid = blockIdx.x;
  if (bid < n_long_head || bid >= n_long_head + n_short_blocks) {
    // long-list entry e: the first entries' workgroups open the grid, the
    // rest (most of which find no entry) close it
    const int64_t e = bid < n_long_head ? bid : bid - n_short_blocks;
    if (e >= (int64_t)*a.long_count) return;  // uniform per workgroup
    const uint32_t key = a.long_list[e];
    const int grp = threadIdx.x >> 5;
    const int64_t lo = a.start[key];
    const int64_t hi = a.end[key];
    const int64_t len = hi - lo;
    float p[VPL], m[VPL], v[VPL];
    if (ADAM && grp == 0) {  // independent of the gradient: fetched first
      const int64_t off = (int64_t)key * a.stride;
      load_f32<VPL, CONSEC>(a.master + off, sub, p);
      load_f32<VPL, CONSEC>(a.m + off, sub, m);
      load_f32<VPL, CONSEC>(a.v + off, sub, v);
    }
    const bool in_lds = len <= kLongLds;
    uint32_t* gseg = (uint32_t*)a.slots + lo;
    if (in_lds) {
      for (int64_t i = threadIdx.x; i < len; i += 256) lds[i] = gseg[i];
      __syncthreads();
      bitonic_sort(lds, len);
    } else {
      bitonic_sort(gseg, len);  // global memory; the workgroup barrier orders its accesses
    }
    float G[VPL];
#pragma unroll
    for (int t = 0; t < VPL; ++t) G[t] = 0.0f;
    for (int64_t start = (int64_t)grp * kPiece; start < len; start += (int64_t)kLongGroups * kPiece) {
      const int cnt = (int)min((int64_t)kPiece, len - start);
      const uint32_t vl = (sub < cnt) ? (in_lds ? lds[start + sub] : gseg[start + sub]) : 0u;
      float P[VPL];
#pragma unroll
      for (int t = 0; t < VPL; ++t) P[t] = 0.0f;
      // eight slots' loads in flight at a time (four with both the optimizer's
      // state and f32 gradients held: eight would cost occupancy there)
      sum_piece<VPL, CONSEC, (ADAM && F32) ? 4 : 8, F32>(a, vl, gbase, cnt, sub, P);
#pragma unroll
      for (int t = 0; t < VPL; ++t) G[t] = G[t] + P[t];
    }
    __syncthreads();  // every slot id has been read: the buffer takes the group sums
#pragma unroll
    for (int t = 0; t < VPL; ++t) part[grp * 512 + col_of<VPL, CONSEC>(sub, t)] = G[t];
    __syncthreads();
    if (grp == 0) {
      float g[VPL];
#pragma unroll
      for (int t = 0; t < VPL; ++t) {
        const int c = col_of<VPL, CONSEC>(sub, t);
        g[t] = part[c];
        for (int q = 1; q < kLongGroups; ++q) g[t] = g[t] + part[q * 512 + c];
      }
      finish<VPL, CONSEC, ADAM>(a, key, sub, g, p, m, v);
    }
    return;
  }
  const int64_t k = ((bid - n_long_head) * 256 + threadIdx.x) >> 5;
  if (k >= a.n_var) return;  // uniform per group
  const int64_t lo = a.start[k];
  const int64_t len = (int64_t)a.end[k] - lo;
  if (!ADAM && len == 0 && a.overwrite) {  // a variable no slot hits: its gradient is zero
    float z[VPL];
#pragma unroll
    for (int t = 0; t < VPL; ++t) z[t] = 0.0f;
    store_f32<VPL, CONSEC>(a.grad_out + k * a.dim, sub, z);
    return;
  }
  if (len == 0 || len > kPiece) return;  // not hit, or a long range (its own workgroup)
  float p[VPL], m[VPL], v[VPL];
  if constexpr (ADAM) {  // the state rows do not depend on the gradient: fetch them first
    const int64_t off = k * a.stride;
    load_f32<VPL, CONSEC>(a.master + off, sub, p);
    load_f32<VPL, CONSEC>(a.m + off, sub, m);
    load_f32<VPL, CONSEC>(a.v + off, sub, v);
  }
  const int cnt = (int)len;
  const uint32_t sl = a.slots[lo + min(sub, cnt - 1)];  // every lane loads (no divergent load)
  // the network only as wide as the longest of the wavefront's two ranges needs
  // (most ranges hold one or two slots); lanes past a range hold 0xffffffff
  // (the other group's count is read from its lanes; a group that has already
  // returned leaves an arbitrary value there, which only widens the network)
  const int other = __shfl_xor(cnt, 32);
  const int cmax = max(cnt, (other >= 1 && other <= kPiece) ? other : 1);
  const int span = cmax <= 1 ? 1 : 1 << (32 - __clz(cmax - 1));
  const uint32_t vl = sort32(sub < cnt ? sl : 0xffffffffu, sub, __builtin_amdgcn_readfirstlane(span));
  float g[VPL];
#pragma unroll
  for (int t = 0; t < VPL; ++t) g[t] = 0.0f;
  // loads go out as many slots at a time as the wavefront's longer range has,
  // up to four (a batch re-reads its first slot past the range's end)
  const int cw = __builtin_amdgcn_readfirstlane(cmax);
  if (cw == 1) sum_piece<VPL, CONSEC, 1, F32>(a, vl, gbase, cnt, sub, g);
  else if (cw == 2) sum_piece<VPL, CONSEC, 2, F32>(a, vl, gbase, cnt, sub, g);
  else sum_piece<VPL, CONSEC, 4, F32>(a, vl, gbase, cnt, sub, g);
  finish<VPL, CONSEC, ADAM>(a, k, sub, g, p, m, v);
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
  const int64_t off = k * a.stride;
  load_f32<VPL, CONSEC>(a.master + off, sub, p);
  load_f32<VPL, CONSEC>(a.m + off, sub, m);
  load_f32<VPL, CONSEC>(a.v + off, sub, v);
  adam_apply<VPL, CONSEC>(a, k, sub, g, p, m, v);
}

// Requantisation on its own: src row i -> row dst_rows[i] (i when NULL) of q,
// one 32-lane group per row; a destination outside q is skipped.
template <int VPL, bool CONSEC>
__global__ __launch_bounds__(256) void quantize_kernel(const float* __restrict__ src, int64_t n, int dim,
                                                       const int32_t* __restrict__ dst_rows, const TableDev q) {
  const int sub = threadIdx.x & 31;
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 5;
  if (i >= n) return;
  const int64_t k = dst_rows ? (int64_t)dst_rows[i] : i;
  if (k < 0 || k >= q.n_rows) return;
  float p[VPL];
  load_f32<VPL, CONSEC>(src + i * dim, sub, p);
  requant_row<VPL, CONSEC>(q, k, dim, sub, p);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
// How a call groups its slots: the bucketed path (two launches) whenever the
// variables fit kBucketsMax buckets of at most 2^kBucketKeysLog2Max, the
// counting path (counts by global atomics, scan, fill) otherwise.
struct GroupPlan {
  bool bucketed;
  int bs;           // bucket b holds the variables [b << bs, (b + 1) << bs)
  int nb;           // buckets
  int64_t n_tiles;  // tiles of kGroupTile slots
};


static GroupPlan plan_for(int64_t n, int64_t n_var) {
  GroupPlan g{false, 0, 0, 0};
  if (n_var < 1 || n_var > ((int64_t)kBucketsMax << kBucketKeysLog2Max)) return g;
  if ((n + kGroupTile - 1) / kGroupTile > kRangeTilesMax) return g;
  // at most 512 buckets where the bucket width allows: on config 2 (226k
  // variables) 442 buckets of 512 took the step to 147.2 us, against 149.3
  // with 884 of 256 (twice the segments a tile writes and a bucket reads) and
  // 151.3 with 221 of 1,024
  int bs = 0;
  while (((n_var + (1LL << bs) - 1) >> bs) > kBucketsMax / 2 && bs < kBucketKeysLog2Max) ++bs;
  while (((n_var + (1LL << bs) - 1) >> bs) > kBucketsMax) ++bs;
  g.bucketed = true;
  g.bs = bs;
  g.nb = (int)((n_var + (1LL << bs) - 1) >> bs);
  g.n_tiles = (n + kGroupTile - 1) / kGroupTile;
  return g;
}

struct Workspace {
  // both paths
  uint32_t* slots;      // [n] slot ids grouped by variable
  uint32_t* start;      // [n_var] range start of every variable
  uint32_t* end;        // [n_var] range end (the counting path: start + 1)
  uint32_t* long_list;  // [n / (kPiece + 1) + 1] variables of more than kPiece slots, first n_long entries
  uint32_t* n_long;     // the long list's length
  // the counting path
  uint32_t* keys;       // [n] variable of every slot (n_var: none)
  uint32_t* ranks;      // [n] place of every slot in its variable's range
  uint32_t* off;        // [n_var + 2] counts -> range starts ([n_var]: the total); [n_var + 1]: long-list length
  uint32_t* partial;    // scan chunk totals
  // the bucketed path
  unsigned long long* pairs;  // [n_tiles * kGroupTile] (key << 32 | slot), bucket-sorted per tile
  uint32_t* seg;              // [nb, n_tiles] slots of bucket b in tile t << 16 | the slots of t before b
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static int64_t n_long_max(int64_t n) { return n / (kPiece + 1) + 1; }

static int64_t scan_chunks(int64_t n_var) { return (n_var + kScanChunk - 1) / kScanChunk; }

// Lays the workspace out (ws == nullptr: only measures it); returns its size.
static size_t carve(void* ws, int64_t n, int64_t n_var, Workspace* out) {
  const GroupPlan g = plan_for(n, n_var);
  Workspace w;
  memset(&w, 0, sizeof(w));
  char* base = (char*)ws;
  size_t at = 0;
  auto take = [&](size_t bytes) {
    void* p = base ? (void*)(base + at) : nullptr;
    at += align256(bytes);
    return p;
  };
  w.slots = (uint32_t*)take((size_t)n * 4);
  w.long_list = (uint32_t*)take((size_t)(n_long_max(n) + 1) * 4);
  w.n_long = w.long_list ? w.long_list + n_long_max(n) : nullptr;
  if (g.bucketed) {
    w.start = (uint32_t*)take((size_t)n_var * 4);
    w.end = (uint32_t*)take((size_t)n_var * 4);
    w.pairs = (unsigned long long*)take((size_t)g.n_tiles * kGroupTile * 8);
    w.seg = (uint32_t*)take((size_t)g.n_tiles * g.nb * 4);
  } else {
    w.keys = (uint32_t*)take((size_t)n * 4);
    w.ranks = (uint32_t*)take((size_t)n * 4);
    w.off = (uint32_t*)take((size_t)(n_var + 2) * 4);
    w.partial = (uint32_t*)take((size_t)(scan_chunks(n_var + 1) + 1) * 4);
    w.start = w.off;
    w.end = w.off ? w.off + 1 : nullptr;
  }
  if (out) *out = w;
  return at;
}

static size_t workspace_bytes(int64_t n, int64_t n_var) { return carve(nullptr, n, n_var, nullptr); }

static unsigned grid_for(int64_t items, int64_t per_block, int64_t cap) {
  const int64_t b = (items + per_block - 1) / per_block;
  return (unsigned)(b < 1 ? 1 : (b > cap ? cap : b));
}

// Every variable's range [start, end) of slot ids, and the long list.
static int group_slots(const int32_t* rows, int64_t n, const int32_t* ids, int64_t n_var, const int64_t* index,
                       int64_t index_capacity, bool direct, const Workspace& w, hipStream_t st) {
  int split_shift = 0;
  while (((n_var + (1LL << split_shift) - 1) >> split_shift) > kSplitMax) ++split_shift;
  int ib = 0;
  while ((1LL << ib) < index_capacity) ++ib;
  const int mode = direct ? 2 : (index != nullptr ? 1 : 0);
  const unsigned long long* idx = (const unsigned long long*)index;
  const GroupPlan g = plan_for(n, n_var);
  if (g.bucketed) {
    const dim3 tgrid((unsigned)g.n_tiles);
#define EG_TILE_SORT(M)                                                                                            \
  hipLaunchKernelGGL(tile_sort_kernel<M>, tgrid, dim3(kGroupThreads), 0, st, rows, n, ids, n_var, split_shift, idx, \
                     ib, g.bs, g.nb, g.n_tiles, w.pairs, w.seg, w.n_long)
    if (mode == 2) EG_TILE_SORT(2);
    else if (mode == 1) EG_TILE_SORT(1);
    else EG_TILE_SORT(0);
#undef EG_TILE_SORT
    // as few tiles a thread as the tile count allows (the loads of a thread's
    // tiles past the last are wasted issue slots in the kernel's dependent round)
#define EG_BUCKET_RANGES(TPT)                                                                                     \
  hipLaunchKernelGGL(bucket_ranges_kernel<TPT>, dim3((unsigned)g.nb), dim3(kRangeThreads), 0, st, w.pairs, w.seg, \
                     g.n_tiles, g.nb, g.bs, n_var, w.start, w.end, w.slots, w.long_list, w.n_long)
    static_assert(kRangeTilesMax <= 2 * kRangeThreads, "at most two tiles a thread");
    if (g.n_tiles <= kRangeThreads) EG_BUCKET_RANGES(1);
    else EG_BUCKET_RANGES(2);
#undef EG_BUCKET_RANGES
    return launch_status("slot grouping kernels");
  }
  hipLaunchKernelGGL(clear_kernel, dim3(grid_for(n_var + 2, 256, 1024)), dim3(256), 0, st, w.off, n_var + 2,
                     w.long_list, n_long_max(n));
  const dim3 kgrid((unsigned)((n + kTile - 1) / kTile));
  if (mode == 2) {
    hipLaunchKernelGGL(keys_count_kernel<2>, kgrid, dim3(kTileThreads), 0, st, rows, n, ids, n_var, 0,
                       (const unsigned long long*)nullptr, 0, w.keys, w.ranks, w.off);
  } else if (mode == 1) {
    hipLaunchKernelGGL(keys_count_kernel<1>, kgrid, dim3(kTileThreads), 0, st, rows, n, ids, n_var, 0, idx, ib,
                       w.keys, w.ranks, w.off);
  } else {
    hipLaunchKernelGGL(keys_count_kernel<0>, kgrid, dim3(kTileThreads), 0, st, rows, n, ids, n_var, split_shift,
                       (const unsigned long long*)nullptr, 0, w.keys, w.ranks, w.off);
  }
  // the scan runs over n_var + 1 entries (the last count is zero), so off[n_var] is the total
  const unsigned chunks = (unsigned)scan_chunks(n_var + 1);
  hipLaunchKernelGGL(scan_partials, dim3(chunks), dim3(kScanThreads), 0, st, w.off, n_var + 1, w.partial);
  hipLaunchKernelGGL(scan_apply, dim3(chunks), dim3(kScanThreads), 0, st, w.off, n_var + 1, w.partial, w.long_list,
                     w.off + n_var + 1);
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, w.keys, w.ranks, n, n_var,
                     w.off, w.slots);
  return launch_status("slot grouping kernels");
}

static void fill_seg(SegArgs* a, const Workspace& w, int64_t n, int64_t n_var) {
  a->start = w.start;
  a->end = w.end;
  a->slots = w.slots;
  a->long_list = w.long_list;
  // the counting grouping counts its long variables in off[n_var + 1]
  a->long_count = plan_for(n, n_var).bucketed ? w.n_long : w.off + n_var + 1;
  a->n = n;
  a->n_var = n_var;
}

// One workgroup per long-list entry (the list's length is known on the device
// only): the first kLongHead at the start of the grid, so that the long
// chains overlap the rest, the others at its end, where the workgroups that
// find no entry exit within the short ranges' tail.
constexpr int64_t kLongHead = 256;

template <bool ADAM, int VPL, bool CONSEC>
static void launch_reduce_t(const SegArgs& a, hipStream_t st) {
  const int64_t n_long = n_long_max(a.n);
  const int64_t head = n_long < kLongHead ? n_long : kLongHead;
  const int64_t n_short = (a.n_var * 32 + 255) / 256;
  const dim3 grid((unsigned)(n_long + n_short));
  if (a.d_out_f32)
    hipLaunchKernelGGL((reduce_kernel<VPL, CONSEC, ADAM, true>), grid, dim3(256), 0, st, a, head, n_short);
  else
    hipLaunchKernelGGL((reduce_kernel<VPL, CONSEC, ADAM, false>), grid, dim3(256), 0, st, a, head, n_short);
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

// d_out and rows as the call uses them: a plan has no d_out, an apply no rows.
static int check_common(const void* d_out, bool use_dout, const int32_t* rows, bool use_rows, int64_t n_pos,
                        int32_t heads, int32_t dim, const int32_t* ids, int64_t n_var, const void* ws,
                        size_t ws_bytes) {
  EG_CHECK_ARG(n_pos >= 0 && heads >= 1 && heads <= EG_MAX_HEADS, "n_pos=%lld heads=%d", (long long)n_pos, heads);
  EG_CHECK_ARG(dim == 64 || dim == 128 || dim == 160 || dim == 256, "backward dim=%d (built: 64, 128, 160, 256)",
               dim);
  EG_CHECK_ARG(n_var >= 0 && n_var < (1LL << 31), "n_var=%lld", (long long)n_var);
  const int64_t n = n_pos * heads;
  EG_CHECK_ARG(n < (1LL << 31), "n_pos*heads=%lld slots exceed 2^31", (long long)n);
  EG_CHECK_ARG(n == 0 || !use_dout || d_out != nullptr, "d_out is NULL");
  EG_CHECK_ARG(n == 0 || !use_rows || rows != nullptr, "rows is NULL");
  EG_CHECK_ARG(n_var == 0 || ids != nullptr, "ids is NULL");
  if (ws_bytes < workspace_bytes(n, n_var))
    return set_error(EG_ERR_WORKSPACE, "workspace of %zu bytes < %zu needed", ws_bytes, workspace_bytes(n, n_var));
  EG_CHECK_ARG(n == 0 || ws != nullptr, "workspace is NULL");
  return EG_OK;
}

// ---------------------------------------------------------------------------
// Static scratch of eg_descent_step_noalloc: the grouping workspace in a
// file-scope device array, so that callers that may not allocate (code under
// stream capture, serving loops) still get a descent step.  Every GPU holds its
// own copy of the array at its own address, for the life of the process.
// ---------------------------------------------------------------------------
constexpr size_t kStaticScratchBytes = (size_t)16 << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

// The device address of `scratch` on the current device, looked up once per
// device.  The array's name is only a host-side stand-in: kernels must get
// this address, never the name.
static int static_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(EG_ERR_HIP, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return set_error(EG_ERR_UNSUPPORTED, "device %d >= %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return set_error(EG_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return EG_OK;
}

}  // namespace eg

using namespace eg;

extern "C" {

size_t eg_backward_workspace_size(int64_t n_slots, int64_t n_var) {
  return workspace_bytes(n_slots < 0 ? 0 : n_slots, n_var < 0 ? 0 : n_var);
}

int eg_build_row_index(const int32_t* ids, int64_t n, int64_t* table, int64_t capacity, void* stream) {
  EG_CHECK_ARG(n >= 0 && n < (1LL << 31), "n=%lld", (long long)n);
  EG_CHECK_ARG(capacity >= 8 && capacity >= 2 * n && (capacity & (capacity - 1)) == 0 && capacity <= (1LL << 32),
               "capacity=%lld must be a power of two >= max(8, 2*n)", (long long)capacity);
  EG_CHECK_ARG(table != nullptr && (n == 0 || ids != nullptr), "ids/table is NULL");
  EG_CHECK_ARG(((uintptr_t)table & 15) == 0, "table must be 16-byte aligned");
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
  int rc = check_common(d_out, true, rows, true, n_pos, heads, dim, direct ? (const int32_t*)rows : ids, n_var,
                        workspace, workspace_bytes_);
  if (rc != EG_OK) return rc;
  EG_CHECK_ARG(n_var == 0 || grad_out != nullptr, "grad_out is NULL");
  const int64_t n = n_pos * heads;
  if (n == 0 || n_var == 0) return EG_OK;
  hipStream_t st = (hipStream_t)stream;
  Workspace w;
  carve(workspace, n, n_var, &w);
  rc = group_slots(rows, n, ids, n_var, nullptr, 0, direct, w, st);
  if (rc != EG_OK) return rc;
  SegArgs a;
  memset(&a, 0, sizeof(a));
  fill_seg(&a, w, n, n_var);
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

int eg_scatter_grad_plan_slots(const int32_t* slot_var, int64_t n_pos, int32_t heads, int64_t n_var,
                               void* workspace, size_t workspace_bytes_, void* stream) {
  int rc = check_common(nullptr, false, slot_var, true, n_pos, heads, 128, slot_var, n_var, workspace,
                        workspace_bytes_);
  if (rc != EG_OK) return rc;
  const int64_t n = n_pos * heads;
  if (n == 0 || n_var == 0) return EG_OK;
  Workspace w;
  carve(workspace, n, n_var, &w);
  return group_slots(slot_var, n, nullptr, n_var, nullptr, 0, true, w, (hipStream_t)stream);
}

int eg_scatter_grad_apply(const void* d_out, int32_t d_out_f32, int64_t n_pos, int32_t heads, int32_t dim,
                          int64_t n_var, float* grad_out, int32_t overwrite, void* workspace, size_t workspace_bytes_,
                          void* stream) {
  EG_CHECK_ARG(n_pos >= 0 && heads >= 1 && heads <= EG_MAX_HEADS, "n_pos=%lld heads=%d", (long long)n_pos, heads);
  EG_CHECK_ARG(n_var >= 0 && n_var < (1LL << 31), "n_var=%lld", (long long)n_var);
  EG_CHECK_ARG(dim == 64 || dim == 128 || dim == 160 || dim == 256, "backward dim=%d (built: 64, 128, 160, 256)", dim);
  EG_CHECK_ARG(n_var == 0 || grad_out != nullptr, "grad_out is NULL");
  const int64_t n = n_pos * heads;
  hipStream_t st = (hipStream_t)stream;
  if (n_var == 0) return EG_OK;
  if (n == 0) {  // no slot: a zero gradient (a fill kernel, so the call can sit in a captured graph)
    if (overwrite) {
      const int64_t words = n_var * dim;
      hipLaunchKernelGGL(clear_kernel, dim3(grid_for(words, 256, 4096)), dim3(256), 0, st, (uint32_t*)grad_out, words,
                         (uint32_t*)nullptr, (int64_t)0);
      return launch_status("clear_kernel");
    }
    return EG_OK;
  }
  int rc = check_common(d_out, true, nullptr, false, n_pos, heads, dim, (const int32_t*)workspace, n_var, workspace,
                        workspace_bytes_);
  if (rc != EG_OK) return rc;
  Workspace w;
  carve(workspace, n, n_var, &w);
  SegArgs a;
  memset(&a, 0, sizeof(a));
  fill_seg(&a, w, n, n_var);
  a.d_out = d_out;
  a.d_out_f32 = d_out_f32;
  a.heads = heads;
  a.dim = dim;
  a.width = (int64_t)heads * dim;
  a.grad_out = grad_out;
  a.overwrite = overwrite != 0;
  return launch_reduce<false>(a, st);
}

// The descent state's own checks (every entry point of the step).
static int check_state(const eg_descent_state* state) {
  EG_CHECK_ARG(state != nullptr, "state is NULL");
  EG_CHECK_ARG(state->n == 0 || (state->master && state->m && state->v && state->stamp),
               "state master/m/v/stamp is NULL");
  EG_CHECK_ARG(state->row_stride == 0 || state->row_stride >= state->dim, "row_stride=%lld below dim=%d",
               (long long)state->row_stride, state->dim);
  if (state->index != nullptr)
    EG_CHECK_ARG(state->index_capacity >= 2 * state->n && state->index_capacity >= 8 &&
                     (state->index_capacity & (state->index_capacity - 1)) == 0 &&
                     state->index_capacity <= (1LL << 32) && ((uintptr_t)state->index & 15) == 0,
                 "index_capacity=%lld must be a power of two >= max(8, 2*n), the index 16-byte aligned",
                 (long long)state->index_capacity);
  return EG_OK;
}

int eg_descent_plan(const int32_t* rows, int64_t n_pos, int32_t heads, const eg_descent_state* state,
                    void* workspace, size_t workspace_bytes_, void* stream) {
  int rc = check_state(state);
  if (rc != EG_OK) return rc;
  rc = check_common(nullptr, false, rows, true, n_pos, heads, state->dim, state->ids, state->n, workspace,
                    workspace_bytes_);
  if (rc != EG_OK) return rc;
  const int64_t n = n_pos * heads;
  if (state->n == 0 || n == 0) return EG_OK;
  Workspace w;
  carve(workspace, n, state->n, &w);
  return group_slots(rows, n, state->ids, state->n, state->index, state->index_capacity, false, w,
                     (hipStream_t)stream);
}

int eg_descent_plan_slots(const int32_t* slot_var, int64_t n_pos, int32_t heads, const eg_descent_state* state,
                          void* workspace, size_t workspace_bytes_, void* stream) {
  int rc = check_state(state);
  if (rc != EG_OK) return rc;
  rc = check_common(nullptr, false, slot_var, true, n_pos, heads, state->dim, state->ids, state->n, workspace,
                    workspace_bytes_);
  if (rc != EG_OK) return rc;
  const int64_t n = n_pos * heads;
  if (state->n == 0 || n == 0) return EG_OK;
  Workspace w;
  carve(workspace, n, state->n, &w);
  // the slots' variables are given: no row lookup (values outside [0, n) hit no variable)
  return group_slots(slot_var, n, state->ids, state->n, nullptr, 0, true, w, (hipStream_t)stream);
}

int eg_descent_apply(const void* d_out, int32_t d_out_f32, int64_t n_pos, int32_t heads,
                     const eg_descent_state* state, const eg_adam* opt, const eg_table* base, void* workspace,
                     size_t workspace_bytes_, void* stream) {
  int rc = check_state(state);
  if (rc != EG_OK) return rc;
  EG_CHECK_ARG(opt != nullptr, "opt is NULL");
  rc = check_common(d_out, true, nullptr, false, n_pos, heads, state->dim, state->ids, state->n, workspace,
                    workspace_bytes_);
  if (rc != EG_OK) return rc;
  EG_CHECK_ARG(opt->step >= 1 && opt->step < (1LL << 31), "step=%lld", (long long)opt->step);
  EG_CHECK_ARG(opt->lr >= 0.0 && opt->beta1 >= 0.0 && opt->beta1 < 1.0 && opt->beta2 >= 0.0 && opt->beta2 < 1.0 &&
                   opt->eps >= 0.0,
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
  if (opt->l2_coef != 0.0f && opt->anchor == nullptr) {
    rc = make_table(base, &a.base, "base table");
    if (rc != EG_OK) return rc;
    EG_CHECK_ARG(base->dim == state->dim, "base table dim %d != state dim %d", base->dim, state->dim);
  }
  a.anchor = opt->l2_coef != 0.0f ? opt->anchor : nullptr;
  const int64_t n = n_pos * heads;
  if (state->n == 0) return EG_OK;
  hipStream_t st = (hipStream_t)stream;
  Workspace w;
  carve(workspace, n, state->n, &w);
  fill_seg(&a, w, n, state->n);
  a.d_out = d_out;
  a.d_out_f32 = d_out_f32;
  a.heads = heads;
  a.dim = state->dim;
  a.width = (int64_t)heads * state->dim;
  a.ids = state->ids;
  a.master = state->master;
  a.m = state->m;
  a.v = state->v;
  a.stride = state->row_stride > 0 ? state->row_stride : state->dim;
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

int eg_descent_step(const void* d_out, int32_t d_out_f32, const int32_t* rows, int64_t n_pos, int32_t heads,
                    const eg_descent_state* state, const eg_adam* opt, const eg_table* base, void* workspace,
                    size_t workspace_bytes_, void* stream) {
  int rc = check_state(state);
  if (rc != EG_OK) return rc;
  EG_CHECK_ARG(opt != nullptr, "opt is NULL");
  // both halves' argument checks before either launches anything
  rc = check_common(d_out, true, rows, true, n_pos, heads, state->dim, state->ids, state->n, workspace,
                    workspace_bytes_);
  if (rc != EG_OK) return rc;
  EG_CHECK_ARG(opt->step >= 1 && opt->step < (1LL << 31), "step=%lld", (long long)opt->step);
  EG_CHECK_ARG(opt->lr >= 0.0 && opt->beta1 >= 0.0 && opt->beta1 < 1.0 && opt->beta2 >= 0.0 && opt->beta2 < 1.0 &&
                   opt->eps >= 0.0,
               "invalid Adam hyper-parameters");
  rc = eg_descent_plan(rows, n_pos, heads, state, workspace, workspace_bytes_, stream);
  if (rc != EG_OK) return rc;
  return eg_descent_apply(d_out, d_out_f32, n_pos, heads, state, opt, base, workspace, workspace_bytes_, stream);
}

size_t eg_descent_step_noalloc_max_bytes(void) { return kStaticScratchBytes; }

int eg_descent_step_noalloc(const void* d_out, int32_t d_out_f32, const int32_t* rows, int64_t n_pos, int32_t heads,
                            const eg_descent_state* state, const eg_adam* opt, const eg_table* base, void* stream) {
  EG_CHECK_ARG(state != nullptr && opt != nullptr, "state/opt is NULL");
  EG_CHECK_ARG(n_pos >= 0 && heads >= 1 && heads <= EG_MAX_HEADS, "n_pos=%lld heads=%d", (long long)n_pos, heads);
  EG_CHECK_ARG(state->n >= 0 && state->n < (1LL << 31), "n_var=%lld", (long long)state->n);
  const int64_t n = n_pos * heads;
  EG_CHECK_ARG(n < (1LL << 31), "n_pos*heads=%lld slots exceed 2^31", (long long)n);
  const size_t need = workspace_bytes(n, state->n);
  if (need > kStaticScratchBytes)
    return set_error(EG_ERR_WORKSPACE,
                     "eg_descent_step_noalloc: %lld slots and %lld variables need %zu bytes of scratch, more than "
                     "its static %zu; use eg_descent_step with a workspace",
                     (long long)n, (long long)state->n, need, kStaticScratchBytes);
  void* ws = nullptr;
  const int rc = static_scratch(&ws);
  if (rc != EG_OK) return rc;
  // every kernel that reads a part of the scratch first writes or clears it in
  // this same call (counts by a fill kernel, never hipMemsetAsync)
  return eg_descent_step(d_out, d_out_f32, rows, n_pos, heads, state, opt, base, ws, kStaticScratchBytes, stream);
}

int eg_quantize_rows(const float* src, int64_t n, int32_t dim, const int32_t* dst_rows, const eg_table* dst,
                     void* stream) {
  EG_CHECK_ARG(dst != nullptr, "dst is NULL");
  EG_CHECK_ARG(dst->fmt == EG_FMT_Q8_0 || dst->fmt == EG_FMT_MXFP8, "dst must be Q8_0 or MXFP8 (fmt %d)", dst->fmt);
  EG_CHECK_ARG(dim == dst->dim, "dim %d != dst dim %d", dim, dst->dim);
  EG_CHECK_ARG(n >= 0 && n < (1LL << 31), "n=%lld", (long long)n);
  EG_CHECK_ARG(dst_rows != nullptr || n <= dst->n_rows, "n=%lld > dst rows %lld", (long long)n,
               (long long)dst->n_rows);
  EG_CHECK_ARG(n == 0 || src != nullptr, "src is NULL");
  TableDev q;
  int rc = make_table(dst, &q, "dst");
  if (rc != EG_OK) return rc;
  if (n == 0) return EG_OK;
  const dim3 grid((unsigned)((n * 32 + 255) / 256));
  hipStream_t st = (hipStream_t)stream;
  switch (dim) {
    case 128: hipLaunchKernelGGL((quantize_kernel<4, true>), grid, dim3(256), 0, st, src, n, dim, dst_rows, q); break;
    case 64: hipLaunchKernelGGL((quantize_kernel<2, true>), grid, dim3(256), 0, st, src, n, dim, dst_rows, q); break;
    case 256: hipLaunchKernelGGL((quantize_kernel<8, true>), grid, dim3(256), 0, st, src, n, dim, dst_rows, q); break;
    case 160: hipLaunchKernelGGL((quantize_kernel<5, false>), grid, dim3(256), 0, st, src, n, dim, dst_rows, q); break;
    default: return set_error(EG_ERR_UNSUPPORTED, "requantisation for dim %d (built: 64, 128, 160, 256)", dim);
  }
  return launch_status("quantize_kernel");
}

}  // extern "C"
