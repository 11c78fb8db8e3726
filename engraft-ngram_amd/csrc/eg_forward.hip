// Forward half of the n-gram table path on gfx950: the row hash, the fused
// hash -> gather -> dequant -> (overlay) -> residual-add kernel, and the gather
// by explicit row ids.  All of it is HBM-bound integer/byte work: one
// wavefront per position, 8 values per lane per 16-byte chunk, coalesced
// row-segment reads, streaming (non-temporal) residual traffic so the L2 and
// the Infinity Cache keep the Zipf-hot table rows.
#include <string.h>

#include <hip/hip_ext.h>

#include "eg_common.h"

namespace eg {

// ---------------------------------------------------------------------------
// Error reporting and argument translation
// ---------------------------------------------------------------------------
static thread_local char g_err[512];

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int make_layer_hash(const eg_hash_spec* s, LayerHash* L) {
  EG_CHECK_ARG(s != nullptr, "hash spec is NULL");
  EG_CHECK_ARG(s->ngram_size >= 2 && s->ngram_size <= EG_MAX_NGRAM,
               "ngram_size=%d outside [2, %d]", s->ngram_size, EG_MAX_NGRAM);
  EG_CHECK_ARG(s->heads_per_ngram >= 1, "heads_per_ngram=%d < 1", s->heads_per_ngram);
  const int n_heads = (s->ngram_size - 1) * s->heads_per_ngram;
  EG_CHECK_ARG(n_heads <= EG_MAX_HEADS, "n_heads=%d > %d", n_heads, EG_MAX_HEADS);
  memset(L, 0, sizeof(*L));
  L->eos = s->eos_token_id;
  L->ngram_size = s->ngram_size;
  L->heads_per_ngram = s->heads_per_ngram;
  L->n_heads = n_heads;
  for (int j = 0; j < EG_MAX_NGRAM; ++j) L->mult[j] = s->layer_multipliers[j];
  L->head_mult = s->head_multipliers;
  for (int h = 0; h < n_heads; ++h) {
    const uint64_t p = s->head_vocab_sizes[h];
    EG_CHECK_ARG(p >= 1 && p < (1ull << 32), "head_vocab_sizes[%d]=%llu outside [1, 2^32)", h,
                 (unsigned long long)p);
    const int64_t off = s->head_offsets[h];
    EG_CHECK_ARG(off >= 0 && off + (int64_t)p <= 2147483647LL,
                 "head %d: offset %lld + vocab %llu exceeds int32 global ids", h, (long long)off,
                 (unsigned long long)p);
    L->vocab[h] = (uint32_t)p;
    L->magic[h] = UINT64_MAX / p;
    L->offset[h] = (int32_t)off;
  }
  return EG_OK;
}

int make_table(const eg_table* t, TableDev* out, const char* what) {
  EG_CHECK_ARG(t != nullptr, "%s: table is NULL", what);
  EG_CHECK_ARG(t->dim > 0 && t->dim % 32 == 0 && t->dim <= 512, "%s: dim=%d must be a multiple of 32 in [32, 512]",
               what, t->dim);
  EG_CHECK_ARG(t->fmt >= EG_FMT_BF16 && t->fmt <= EG_FMT_F32, "%s: unknown row format %d", what, t->fmt);
  EG_CHECK_ARG(t->payload != nullptr || t->n_rows == 0, "%s: payload is NULL", what);
  const bool scaled = t->fmt == EG_FMT_Q8_0 || t->fmt == EG_FMT_MXFP8;
  EG_CHECK_ARG(!scaled || t->scales != nullptr || t->n_rows == 0, "%s: format %d needs scales", what, t->fmt);
  EG_CHECK_ARG(t->n_rows >= 0, "%s: n_rows < 0", what);
  out->payload = (const uint8_t*)t->payload;
  out->scales = (const uint8_t*)t->scales;
  out->n_rows = t->n_rows;
  out->fmt = t->fmt;
  out->dim = t->dim;
  const int64_t own = t->fmt == EG_FMT_IQ4_NL ? (int64_t)(t->dim / 32) * 18 : 0;
  if (t->fmt == EG_FMT_IQ4_NL) {
    EG_CHECK_ARG(t->row_stride == 0 || (t->row_stride >= own && t->row_stride % 2 == 0),
                 "%s: row_stride=%lld (IQ4_NL: 0, or an even count >= %lld)", what, (long long)t->row_stride,
                 (long long)own);
  } else {
    EG_CHECK_ARG(t->row_stride == 0, "%s: row_stride=%lld (format %d takes 0)", what, (long long)t->row_stride,
                 t->fmt);
  }
  out->stride = t->row_stride ? t->row_stride : own;
  return EG_OK;
}

// ---------------------------------------------------------------------------
// Hash: one thread per (position, head)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void hash_kernel(const LayerHash L, const int64_t* __restrict__ tokens,
                                                   int64_t n_pos, int64_t seq_len,
                                                   const int32_t* __restrict__ seg_start, int32_t global_ids,
                                                   int32_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n_pos * L.n_heads) return;
  const int64_t p = i / L.n_heads;
  const int h = (int)(i - p * L.n_heads);
  uint64_t ctx[EG_MAX_NGRAM];
  build_ctx(L, tokens, p, seg_start_of(p, seq_len, seg_start), ctx);
  out[i] = head_row(L, h, ctx, global_ids != 0);
}

// ---------------------------------------------------------------------------
// Damage scan: one group of G lanes per kScanPP positions (G = 16 or 32 >= n_heads)
// ---------------------------------------------------------------------------
#ifndef EG_SCAN_PP
#define EG_SCAN_PP 4
#endif
constexpr int kScanPP = EG_SCAN_PP;
// Position p of the block (p >= start) hashes its n_heads rows (the block as
// one sequence), looks each up in the sorted overlay ids and reduces over its
// heads: the number of rows found, the max and the sum of their dnorm (a fixed
// pairwise tree over the heads); every row found adds one to its read count.
// Nothing per slot is written to memory.  A group of G lanes (one head a lane)
// takes PP positions at once, every load of one stage issued for all of them
// before any is waited for: the scan is a chain of dependent loads (tokens ->
// filter -> pair -> dnorm), and PP chains in flight per lane keep more of the
// memory system busy.
// With the rank bitmap of the overlay ids (eg_build_id_bitmap: its filter
// blocks, 1/2048 of the rows' count in bytes, stay in each XCD's L2 and settle
// almost every miss), a lookup is one filter probe and, rarely, one pair probe:
// overlay index = the pair's rank + popcount of its bits below the row -- in
// place of the ~19 dependent loads of the binary search.
template <int G, typename TOK, int PP>
__global__ __launch_bounds__(256) void scan_kernel(const LayerHash L, const TOK* __restrict__ tokens, int64_t n,
                                                   int64_t start, const int32_t* __restrict__ ids, int64_t n_ids,
                                                   const uint32_t* __restrict__ bitmap, int64_t n_bits,
                                                   const float* __restrict__ dnorm, int32_t* __restrict__ n_hit,
                                                   float* __restrict__ dmax, float* __restrict__ dsum,
                                                   unsigned long long* __restrict__ counts) {
  // positions start + t0 + j, j < PP, of this group (uniform per group)
  const int64_t t0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) / G * PP;
  const int h = (int)(threadIdx.x % G);
  if (start + t0 >= n) return;
  const int hh = min(h, L.n_heads - 1);
  uint64_t mult[EG_MAX_NGRAM];
  load_head_mult(L, hh, mult);
  const HeadConst hc = load_head_const(L, hh);
  // 1. every position's tokens, then every row id
  uint64_t raw[PP][EG_MAX_NGRAM];
#pragma unroll
  for (int j = 0; j < PP; ++j) load_ctx_tokens(tokens, min(start + t0 + j, n - 1), L.ngram_size, raw[j]);
  int32_t row[PP];
#pragma unroll
  for (int j = 0; j < PP; ++j) {
    uint64_t ctx[EG_MAX_NGRAM];
    ctx_from(L, raw[j], min(start + t0 + j, n - 1), 0, ctx);
    row[j] = row_of(L, hh, ctx, mult, hc, true);
  }
  // 2. every lookup.  With the bitmap: all filter blocks, then all pairs (a
  //    row the filter rejects reads pair 0 in place of its own: every lane
  //    issues every load, and the rejected ones hit one cached line), then
  //    every hit's dnorm (a miss reads dnorm[0]).
  int64_t k[PP];
  if (bitmap != nullptr) {
    const int64_t nw = bitmap_words(n_bits);
    const uint32_t n_fb = (uint32_t)bitmap_filter_blocks(n_bits);
    const uint64_t* filt = (const uint64_t*)(bitmap + 2 * nw);
    uint64_t fb[PP], mask[PP];
#pragma unroll
    for (int j = 0; j < PP; ++j) {
      const BloomProbe bp = bloom_probe((uint32_t)row[j], n_fb);
      mask[j] = bp.mask;
      fb[j] = filt[bp.block];
    }
    u32x2 pr[PP];
    bool pass[PP];
#pragma unroll
    for (int j = 0; j < PP; ++j) {
      pass[j] = (int64_t)(uint32_t)row[j] < n_bits && (fb[j] & mask[j]) == mask[j];
      pr[j] = ((const u32x2*)bitmap)[pass[j] ? ((uint32_t)row[j] >> 5) : 0u];
    }
#pragma unroll
    for (int j = 0; j < PP; ++j) {
      const uint32_t bit = (uint32_t)row[j] & 31u;
      k[j] = (pass[j] && ((pr[j].x >> bit) & 1u)) ? (int64_t)pr[j].y + __popc(pr[j].x & ((1u << bit) - 1u)) : -1;
    }
  } else {
#pragma unroll
    for (int j = 0; j < PP; ++j) k[j] = sorted_find(ids, n_ids, row[j]);
  }
  float d[PP];
#pragma unroll
  for (int j = 0; j < PP; ++j) d[j] = dnorm[k[j] >= 0 ? k[j] : 0];
#pragma unroll
  for (int j = 0; j < PP; ++j) {
    const bool hit = start + t0 + j < n && h < L.n_heads && k[j] >= 0;
    if (hit) atomicAdd(&counts[k[j]], 1ull);
    // head-order reductions over the group (lane 0 ends with the results)
    uint32_t cnt = hit ? 1u : 0u;
    float mx = hit ? d[j] : -INFINITY, sm = hit ? d[j] : 0.0f;
#pragma unroll
    for (int o = 1; o < G; o <<= 1) {
      const uint32_t c2 = __shfl_down(cnt, o, G);
      const float m2 = __shfl_down(mx, o, G), s2 = __shfl_down(sm, o, G);
      if (h + o < G && (h & (2 * o - 1)) == 0) {
        cnt += c2;
        mx = fmaxf(mx, m2);
        sm = sm + s2;
      }
    }
    if (h == 0 && start + t0 + j < n) {
      n_hit[t0 + j] = (int32_t)cnt;
      dmax[t0 + j] = cnt ? mx : 0.0f;
      dsum[t0 + j] = sm;
    }
  }
}

// ---------------------------------------------------------------------------
// Fused forward: one wavefront per position
// ---------------------------------------------------------------------------
struct OverlayDev {
  const int32_t* ids;
  const int32_t* index;
  int64_t n;
  TableDev rows;
  const uint32_t* bitmap;  // optional rank bitmap of ids (eg_build_id_bitmap)
  int64_t n_bits;
};

struct FwdArgs {
  LayerHash hash[EG_MAX_LAYERS];
  TableDev table[EG_MAX_LAYERS];
  OverlayDev ov[EG_MAX_LAYERS];
  const int64_t* tokens;    // hash mode
  const int32_t* rows_in;   // gather mode: [n_pos, heads] global ids
  const int32_t* slot_var;  // gather mode: [n_pos, heads] overlay row per slot (-1: table)
  const int32_t* seg_start;
  const uint16_t* residual; // bf16 [n_pos, W] or nullptr
  void* out;
  int32_t* rows_out;
  int32_t* vars_out;        // overlay row each slot read (-1: base table); overlay kernels only
  int64_t seq_len;
  int64_t n_pos;
  int32_t n_layers;
  int32_t heads;
  int32_t dim;
  int32_t decode_ctx;       // > 0: position p is the last token of sequence p, tokens [n_pos, decode_ctx]
  int32_t parts;            // wavefronts per position: ceil(W / (NCH * 512))
};

constexpr int kMaxWidth = 4096;  // W = heads * dim
#ifndef EG_NCH_F32
#define EG_NCH_F32 1
#endif
constexpr int kWavesPerBlock = 4;

// One wavefront per (position, column part): part q of position p covers the
// columns [q*NCH*512, (q+1)*NCH*512) of the position's W, NCH 8-value chunks
// per lane, and hashes the heads those columns touch (a head whose row spans
// two parts is hashed by both).  OVL: overlay lookups compiled in.
// ROWS: the caller's row ids in place of the hash (a separate instantiation, so
// that a profile tells the two forms apart).
template <int FMT, int DIM, int NCH, int MAXL, bool F32OUT, bool OVL, int PARTS, bool ROWS>
__global__ __launch_bounds__(256) void forward_kernel(const FwdArgs a) {
  const int lane = threadIdx.x & 63;
  // Wavefront index (n_pos * parts < 2^32), read as wavefront-uniform: the
  // position, column part and head range then live in scalar registers and
  // their address arithmetic leaves the vector ALU.
  const uint32_t wid = __builtin_amdgcn_readfirstlane(blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6));
  const uint32_t parts = PARTS ? (uint32_t)PARTS : (uint32_t)a.parts;     // PARTS: known at compile time
  const uint32_t pu = parts == 1 ? wid : wid / parts;
  const int64_t p = pu;
  if (p >= a.n_pos) return;  // uniform per wavefront
  const int dim = DIM ? DIM : a.dim;
  const int H = a.heads;
  const int W = H * dim;
  const int cb = (int)(wid - pu * parts) * (NCH * 512);  // first column of this wavefront
  const int h_lo = cb / dim;                                // first head it touches
  const int nh = min(H, (cb + NCH * 512 + dim - 1) / dim) - h_lo;  // heads it touches
  // Lane `lane` hashes head hh; the lanes past the heads this wavefront touches
  // repeat its last head, so every load below is issued by every lane without
  // a branch (a load inside a lane-divergent branch is waited for inside it,
  // which would serialise the wavefront's loads).
  const bool own_head = lane < nh;
  const int hh = h_lo + min(lane, nh - 1);

  // 1. Everything the row ids depend on (tokens, segment start, multipliers,
  //    or the caller's row ids) is loaded first: vmcnt retires loads in issue
  //    order, so the hash below then waits for these and not for the residual.
  const int nl = a.n_layers;
  uint64_t raw[EG_MAX_NGRAM];
  uint64_t mult[EG_MAX_LAYERS][EG_MAX_NGRAM];
  HeadConst hconst[EG_MAX_LAYERS];
  int64_t seg0 = 0;
  int64_t tp = p;  // index of position p's own token
  int32_t rid[EG_MAX_LAYERS] = {0, 0};
  static_assert(MAXL >= 1 && MAXL <= EG_MAX_LAYERS, "layer count");
  const bool hashing = !ROWS;
  if (hashing) {
    tp = a.decode_ctx > 0 ? p * a.decode_ctx + (a.decode_ctx - 1) : p;
    seg0 = a.decode_ctx > 0 ? p * a.decode_ctx : seg_start_of(p, a.seq_len, a.seg_start);
    int ng = a.hash[0].ngram_size;
    if (MAXL > 1 && nl > 1 && a.hash[1].ngram_size > ng) ng = a.hash[1].ngram_size;
    // The token index is uniform, but held in a vector register: the tokens are
    // then vector loads, retired in issue order ahead of the residual (scalar
    // loads would be waited for before the residual loads are issued).
    int64_t tpv = tp;
    asm volatile("" : "+v"(tpv));
    load_ctx_tokens(a.tokens, tpv, ng, raw);
#pragma unroll
    for (int l = 0; l < MAXL; ++l)
      if (l < nl) {
        load_head_mult(a.hash[l], hh, mult[l]);
        hconst[l] = load_head_const(a.hash[l], hh);
      }
  } else {
    // caller's ids, [n_layers, n_pos, heads] (eg_forward's rows_out layout)
#pragma unroll
    for (int l = 0; l < MAXL; ++l)
      if (l < nl) rid[l] = a.rows_in[((int64_t)l * a.n_pos + p) * H + hh];
  }

  // 2. The residual stream is read once: streaming (non-temporal) loads, issued
  //    by every lane (a lane past W re-reads the last chunk and stores nothing).
  //    Without a residual (F32OUT) the sum starts from -0: -0 + x == x for every x.
  u32x4 res[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if constexpr (F32OUT) {
      res[c] = u32x4{0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u};
    } else {
      const int e0 = min(cb + (lane + 64 * c) * 8, W - 8);
      res[c] = __builtin_nontemporal_load((const u32x4*)(a.residual + p * W + e0));
    }
  }

  // 3. Row ids of head hh, one per layer.
  if (hashing) {
#pragma unroll
    for (int l = 0; l < MAXL; ++l) {
      if (l < nl) {
        uint64_t ctx[EG_MAX_NGRAM];
        ctx_from(a.hash[l], raw, tp, seg0, ctx);
        rid[l] = row_of(a.hash[l], hh, ctx, mult[l], hconst[l], true);
      }
    }
  }
  // 4. Issue the table (or overlay) row loads of every layer and chunk.  Row
  //    ids handed in by the caller (gather mode) and overlay indices are
  //    checked: an id outside its table reads NaN, never memory.  Base-table
  //    loads are unconditional (an invalid id loads row 0 and is masked) and
  //    go out before the overlay lookup: the lookup's dependent probes then
  //    overlap the row's own latency, and a row the overlay replaces (rare)
  //    costs one wasted load.
  RawChunk tr[MAXL][NCH];
  RawChunk orow[OVL ? MAXL : 1][OVL ? NCH : 1];
  int32_t ovk_keep[OVL ? MAXL : 1];
  uint32_t src[MAXL][NCH];  // 0: base table, 1: overlay, 2: invalid id
#pragma unroll
  for (int l = 0; l < MAXL; ++l) {
    if (l >= nl) break;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int e0 = cb + (lane + 64 * c) * 8;
      const int h = min(e0, W - 8) / dim;
      const int32_t row = __shfl(rid[l], h - h_lo);
      const int off = e0 - h * dim;
      const bool base_ok = e0 < W && (uint32_t)row < (uint64_t)a.table[l].n_rows;
      tr[l][c] = load_raw<FMT>(a.table[l], dim, base_ok ? row : 0, base_ok ? off : 0);
      src[l][c] = base_ok ? 0u : 2u;
    }
    if constexpr (OVL) {
      int32_t ovk = -1;
      const OverlayDev& ov = a.ov[l];
      ovk_keep[l] = -1;
      if (a.slot_var != nullptr) {
        ovk = a.slot_var[p * H + hh];
      } else if (ov.n > 0) {
        const int64_t k = ov.bitmap ? bitmap_find(ov.bitmap, ov.n_bits, rid[l]) : sorted_find(ov.ids, ov.n, rid[l]);
        if (k >= 0) ovk = ov.index ? ov.index[k] : (int32_t)k;
      }
      ovk_keep[l] = ovk;
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const int e0 = cb + (lane + 64 * c) * 8;
        const int h = min(e0, W - 8) / dim;
        const int32_t k = __shfl(ovk, h - h_lo);
        if (e0 < W && k >= 0) {
          src[l][c] = 2;
          if (k < ov.rows.n_rows) {
            orow[l][c] = load_raw_rt(ov.rows, k, e0 - h * dim);
            src[l][c] = 1;
          }
        }
      }
    }
  }

  // Row ids for the backward (stored after every load is issued: a store in
  // between would make later loads wait for it and for all loads before it).
  if (a.rows_out != nullptr && own_head && hh * dim >= cb) {  // the part holding the head's first column
#pragma unroll
    for (int l = 0; l < MAXL; ++l)
      if (l < nl) a.rows_out[((int64_t)l * a.n_pos + p) * H + hh] = rid[l];
  }
  if constexpr (OVL) {
    if (a.vars_out != nullptr && own_head && hh * dim >= cb) {
#pragma unroll
      for (int l = 0; l < MAXL; ++l)
        if (l < nl) a.vars_out[((int64_t)l * a.n_pos + p) * H + hh] = ovk_keep[l];
    }
  }

  // 5. Residual + every layer, fp32, in layer order.
  float acc[NCH][8];
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[c][2 * i] = __uint_as_float(res[c][i] << 16);
      acc[c][2 * i + 1] = __uint_as_float(res[c][i] & 0xffff0000u);
    }
#pragma unroll
  for (int l = 0; l < MAXL; ++l) {
    if (l >= nl) break;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int e0 = cb + (lane + 64 * c) * 8;
      const int off = e0 - (min(e0, W - 8) / dim) * dim;
      float v[8];
      if (OVL && src[l][c] == 1) {
        decode_rt(a.ov[l].rows.fmt, orow[OVL ? l : 0][OVL ? c : 0], off, v);
      } else {
        decode<FMT>(tr[l][c], src[l][c] == 0 ? off : 0, v);
        if (src[l][c] != 0) {
#pragma unroll
          for (int i = 0; i < 8; ++i) v[i] = __uint_as_float(0x7fc00000u);
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[c][i] += v[i];
    }
  }

#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int e0 = cb + (lane + 64 * c) * 8;
    if (e0 < W) {
      if constexpr (F32OUT) {
        u32x4* dst = (u32x4*)((float*)a.out + p * W + e0);
        u32x4 lo, hi;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          lo[i] = __float_as_uint(acc[c][i]);
          hi[i] = __float_as_uint(acc[c][4 + i]);
        }
        dst[0] = lo;
        dst[1] = hi;
      } else {
        u32x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = pack_bf16x2(acc[c][2 * i], acc[c][2 * i + 1]);
        __builtin_nontemporal_store(o, (u32x4*)((uint16_t*)a.out + p * W + e0));
      }
    }
  }
}

// Events of eg_forward_timed: when set, the forward kernel is launched with
// hipExtLaunchKernelGGL so the events carry the dispatch's own start and end.
static thread_local hipEvent_t g_ev_start = nullptr;
static thread_local hipEvent_t g_ev_stop = nullptr;

#define EG_LAUNCH(...)                                                                                  \
  do {                                                                                                  \
    if (g_ev_start != nullptr)                                                                          \
      hipExtLaunchKernelGGL((forward_kernel<__VA_ARGS__>), grid, dim3(256), 0, st, g_ev_start, g_ev_stop, \
                            0u, a);                                                                     \
    else                                                                                                \
      hipLaunchKernelGGL((forward_kernel<__VA_ARGS__>), grid, dim3(256), 0, st, a);                     \
  } while (0)

// One launch: parts = ceil(W / (NCH * 512)) wavefronts per position (PARTS:
// the same number when the caller's shape fixes it, 0 otherwise).
template <int FMT, int DIM, int NCH, int MAXL, bool F32OUT, bool OVL, int PARTS, bool ROWS>
static void launch_nch(FwdArgs a, hipStream_t st) {
  a.parts = (a.heads * a.dim + NCH * 512 - 1) / (NCH * 512);
  const int64_t waves = a.n_pos * a.parts;
  const dim3 grid((unsigned)((waves + kWavesPerBlock - 1) / kWavesPerBlock));
  EG_LAUNCH(FMT, DIM, NCH, MAXL, F32OUT, OVL, PARTS, ROWS);
}

// Specialised residual-add shapes (dim 128): one layer without overlay takes
// W = 2048 in two 1024-column parts (the config-1 shape: 8 waves per SIMD
// without spills; one 2048-column wavefront per position, at 6 waves, and four
// 512-column parts both measured slower) and W = 3072 in two halves; two layers
// take 1536-column parts at W = 3072, 1024-column parts otherwise, overlay
// lookups 1024-column parts.  Everything else goes through the generic kernel.
template <int FMT, bool ROWS>
static bool launch_special(const FwdArgs& a, bool ovl, hipStream_t st) {
  if (a.dim != 128) return false;
  const int W = a.heads * a.dim;
  if (W != 2048 && W != 3072) return false;
  if (a.n_layers == 1 && !ovl) {
    if (W == 2048) launch_nch<FMT, 128, 2, 1, false, false, 2, ROWS>(a, st);
    else launch_nch<FMT, 128, 3, 1, false, false, 2, ROWS>(a, st);
  } else if (a.n_layers == 1) {
    launch_nch<FMT, 128, 2, 1, false, true, 0, ROWS>(a, st);
  } else if (!ovl) {
    if (W == 3072) launch_nch<FMT, 128, 3, 2, false, false, 2, ROWS>(a, st);
    else launch_nch<FMT, 128, 2, 2, false, false, 0, ROWS>(a, st);
  } else {
    launch_nch<FMT, 128, 2, 2, false, true, 0, ROWS>(a, st);
  }
  return true;
}

// f32 output at dim 128, one layer (eg_gather_slots' OverlayEmb gather,
// eg_gather's row reads): the generic kernel's divisions by the runtime dim
// become shifts, and the position's W takes NCH_F32 * 512-column parts.
constexpr int kNchF32 = EG_NCH_F32;
template <int FMT, bool ROWS>
static bool launch_special_f32(const FwdArgs& a, hipStream_t st) {
  if (a.dim != 128 || a.n_layers != 1) return false;
  launch_nch<FMT, 128, kNchF32, 1, true, true, 0, ROWS>(a, st);
  return true;
}

// The reference's real table shape (16 heads of 160 values, W = 2560, one
// layer, no overlay): five 512-column chunks per position.
constexpr int kRealNch = 5;
template <int FMT, bool ROWS>
static bool launch_real(const FwdArgs& a, bool ovl, hipStream_t st) {
  if (a.dim != 160 || a.heads * a.dim != 2560 || a.n_layers != 1 || ovl) return false;
  launch_nch<FMT, 160, kRealNch, 1, false, false, 5 / kRealNch, ROWS>(a, st);
  return true;
}

// Any shape: runtime dim, 1024-column parts, overlays compiled in.
template <int FMT, bool F32OUT, bool ROWS>
static void launch_generic(const FwdArgs& a, hipStream_t st) {
  if (a.n_layers == 1) launch_nch<FMT, 0, 2, 1, F32OUT, true, 0, ROWS>(a, st);
  else launch_nch<FMT, 0, 2, 2, F32OUT, true, 0, ROWS>(a, st);
}

template <bool F32OUT, bool ROWS>
static int launch_forward_as(const FwdArgs& a, hipStream_t st) {
  if (a.n_pos == 0) return EG_OK;
  bool ovl = a.slot_var != nullptr || a.vars_out != nullptr;
  for (int l = 0; l < a.n_layers; ++l) ovl = ovl || a.ov[l].n > 0;
  const int fmt = a.table[0].fmt;
  if (!F32OUT) {
    bool done = false;
    if (fmt == EG_FMT_Q8_0) done = launch_special<EG_FMT_Q8_0, ROWS>(a, ovl, st);
    else if (fmt == EG_FMT_BF16) done = launch_special<EG_FMT_BF16, ROWS>(a, ovl, st);
    else if (fmt == EG_FMT_MXFP8) done = launch_special<EG_FMT_MXFP8, ROWS>(a, ovl, st);
    else if (fmt == EG_FMT_IQ4_NL) done = launch_real<EG_FMT_IQ4_NL, ROWS>(a, ovl, st);
    if (done) return launch_status("forward_kernel");
  } else if (ROWS) {
    bool done = false;
    if (fmt == EG_FMT_Q8_0) done = launch_special_f32<EG_FMT_Q8_0, ROWS>(a, st);
    else if (fmt == EG_FMT_BF16) done = launch_special_f32<EG_FMT_BF16, ROWS>(a, st);
    else if (fmt == EG_FMT_MXFP8) done = launch_special_f32<EG_FMT_MXFP8, ROWS>(a, st);
    if (done) return launch_status("forward_kernel");
  }
  switch (fmt) {
    case EG_FMT_Q8_0: launch_generic<EG_FMT_Q8_0, F32OUT, ROWS>(a, st); break;
    case EG_FMT_BF16: launch_generic<EG_FMT_BF16, F32OUT, ROWS>(a, st); break;
    case EG_FMT_MXFP8: launch_generic<EG_FMT_MXFP8, F32OUT, ROWS>(a, st); break;
    case EG_FMT_IQ4_NL: launch_generic<EG_FMT_IQ4_NL, F32OUT, ROWS>(a, st); break;
    case EG_FMT_F32: launch_generic<EG_FMT_F32, F32OUT, ROWS>(a, st); break;
    default: return set_error(EG_ERR_UNSUPPORTED, "row format %d", fmt);
  }
  return launch_status("forward_kernel");
}

template <bool F32OUT>
static int launch_forward(const FwdArgs& a, hipStream_t st) {
  return a.rows_in != nullptr ? launch_forward_as<F32OUT, true>(a, st) : launch_forward_as<F32OUT, false>(a, st);
}

#undef EG_LAUNCH

// Variable index of each row id (-1 if absent) + per-id read counts.
__global__ __launch_bounds__(256) void lookup_kernel(const int32_t* __restrict__ rows, int64_t n,
                                                     const int32_t* __restrict__ ids,
                                                     const int32_t* __restrict__ index, int64_t n_ids,
                                                     int32_t* __restrict__ out,
                                                     unsigned long long* __restrict__ counts) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t k = n_ids > 0 ? sorted_find(ids, n_ids, rows[i]) : -1;
  if (out != nullptr) out[i] = k < 0 ? -1 : (index ? index[k] : (int32_t)k);
  if (counts != nullptr && k >= 0) atomicAdd(&counts[k], 1ull);
}

static int fill_overlay(const eg_overlay* o, const TableDev& base, OverlayDev* out) {
  memset(out, 0, sizeof(*out));
  if (o == nullptr || o->n == 0) return EG_OK;
  EG_CHECK_ARG(o->n > 0 && o->ids != nullptr, "overlay: n=%lld with NULL ids", (long long)o->n);
  int rc = make_table(&o->rows, &out->rows, "overlay rows");
  if (rc != EG_OK) return rc;
  EG_CHECK_ARG(o->rows.dim == base.dim, "overlay dim %d != table dim %d", o->rows.dim, base.dim);
  EG_CHECK_ARG(o->index != nullptr || o->rows.n_rows >= o->n, "overlay: %lld ids but %lld rows",
               (long long)o->n, (long long)o->rows.n_rows);
  EG_CHECK_ARG(o->bitmap == nullptr || (o->n_bits >= 1 && o->n_bits <= (1LL << 31)),
               "overlay: bitmap with n_bits=%lld", (long long)o->n_bits);
  EG_CHECK_ARG(((uintptr_t)o->bitmap & 7) == 0, "overlay: bitmap must be 8-byte aligned");
  out->ids = o->ids;
  out->index = o->index;
  out->n = o->n;
  out->bitmap = o->bitmap;
  out->n_bits = o->n_bits;
  return EG_OK;
}

}  // namespace eg

using namespace eg;

extern "C" {

const char* eg_last_error(void) { return g_err; }

int eg_abi_version(void) { return EG_ABI_VERSION; }

__global__ __launch_bounds__(256) void bitmap_set_kernel(const int32_t* __restrict__ ids, int64_t n_ids,
                                                         uint32_t* __restrict__ bitmap, int64_t n_bits) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n_ids) return;
  const int64_t r = ids[i];
  if (r >= 0 && r < n_bits) {
    const int64_t nw = (n_bits + 31) >> 5, w = r >> 5;
    atomicOr(&bitmap[2 * w], 1u << (r & 31));
    const BloomProbe bp = bloom_probe((uint32_t)r, (uint32_t)bitmap_filter_blocks(n_bits));
    atomicOr((unsigned long long*)(bitmap + 2 * nw) + bp.block, (unsigned long long)bp.mask);
  }
}

// rank of word w (its pair's second entry) = number of ids below 32 w (a lower
// bound in the sorted ids).
__global__ __launch_bounds__(256) void bitmap_rank_kernel(const int32_t* __restrict__ ids, int64_t n_ids,
                                                          uint32_t* __restrict__ pairs, int64_t words) {
  for (int64_t w = (int64_t)blockIdx.x * 256 + threadIdx.x; w < words; w += (int64_t)gridDim.x * 256) {
    const int64_t key = w * 32;
    int64_t lo = 0, hi = n_ids;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if ((int64_t)ids[mid] < key) lo = mid + 1; else hi = mid;
    }
    pairs[2 * w + 1] = (uint32_t)lo;
  }
}

__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t* __restrict__ a, int64_t len) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < len; i += (int64_t)gridDim.x * 256) a[i] = 0u;
}

int64_t eg_id_bitmap_words(int64_t n_bits) {
  return n_bits < 1 ? 0 : 2 * bitmap_words(n_bits) + 2 * bitmap_filter_blocks(n_bits);
}

int eg_build_id_bitmap(const int32_t* ids, int64_t n_ids, uint32_t* bitmap, int64_t n_bits, void* stream) {
  EG_CHECK_ARG(n_ids >= 0 && n_ids < (1LL << 32) && n_bits >= 1 && n_bits <= (1LL << 31), "n_ids=%lld n_bits=%lld",
               (long long)n_ids, (long long)n_bits);
  EG_CHECK_ARG(bitmap != nullptr && (n_ids == 0 || ids != nullptr), "NULL argument");
  EG_CHECK_ARG(((uintptr_t)bitmap & 7) == 0, "bitmap must be 8-byte aligned");
  const int64_t words = bitmap_words(n_bits);
  const int64_t total = eg_id_bitmap_words(n_bits);
  hipStream_t st = (hipStream_t)stream;
  const int64_t fill_blocks = (total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096;
  hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)fill_blocks), dim3(256), 0, st, bitmap, total);
  if (n_ids > 0)
    hipLaunchKernelGGL(bitmap_set_kernel, dim3((unsigned)((n_ids + 255) / 256)), dim3(256), 0, st, ids, n_ids, bitmap,
                       n_bits);
  const int64_t rank_blocks = (words + 255) / 256 < 4096 ? (words + 255) / 256 : 4096;
  hipLaunchKernelGGL(bitmap_rank_kernel, dim3((unsigned)rank_blocks), dim3(256), 0, st, ids, n_ids, bitmap, words);
  return launch_status("bitmap kernels");
}

int eg_scan_overlay(const eg_hash_spec* spec, const void* tokens, int32_t token_bytes, int64_t n_tokens,
                    int64_t start, const int32_t* ids, int64_t n_ids, const uint32_t* bitmap, int64_t n_bits,
                    const float* dnorm, int32_t* n_hit, float* dnorm_max, float* dnorm_sum, int64_t* read_counts,
                    void* stream) {
  LayerHash L;
  int rc = make_layer_hash(spec, &L);
  if (rc != EG_OK) return rc;
  EG_CHECK_ARG(n_tokens >= 0 && start >= 0 && start <= n_tokens, "n_tokens=%lld start=%lld", (long long)n_tokens,
               (long long)start);
  EG_CHECK_ARG(n_ids >= 1 && n_ids < (1LL << 31), "n_ids=%lld (at least one overlay row)", (long long)n_ids);
  const int64_t m = n_tokens - start;
  if (m == 0) return EG_OK;
  EG_CHECK_ARG(tokens && ids && dnorm && n_hit && dnorm_max && dnorm_sum && read_counts, "NULL argument");
  EG_CHECK_ARG(bitmap == nullptr || (n_bits >= 1 && n_bits <= (1LL << 31)), "n_bits=%lld", (long long)n_bits);
  EG_CHECK_ARG(((uintptr_t)bitmap & 7) == 0, "bitmap must be 8-byte aligned");
  EG_CHECK_ARG(token_bytes == 4 || token_bytes == 8, "token_bytes=%d (4: int32, 8: int64)", token_bytes);
  const int G = L.n_heads <= 16 ? 16 : 32;
  const int64_t threads = (m + kScanPP - 1) / kScanPP * G;
  EG_CHECK_ARG((threads + 255) / 256 < (1LL << 31), "n_tokens=%lld too large for one launch", (long long)n_tokens);
  const dim3 grid((unsigned)((threads + 255) / 256));
  hipStream_t st = (hipStream_t)stream;
  unsigned long long* rc64 = (unsigned long long*)read_counts;
#define EG_SCAN(GG, T)                                                                                            \
  hipLaunchKernelGGL((scan_kernel<GG, T, kScanPP>), grid, dim3(256), 0, st, L, (const T*)tokens, n_tokens, start, \
                     ids, n_ids, bitmap, n_bits, dnorm, n_hit, dnorm_max, dnorm_sum, rc64)
  if (token_bytes == 8) {
    if (G == 16) EG_SCAN(16, int64_t); else EG_SCAN(32, int64_t);
  } else {
    if (G == 16) EG_SCAN(16, int32_t); else EG_SCAN(32, int32_t);
  }
#undef EG_SCAN
  return launch_status("scan_kernel");
}

int eg_hash_rows(const eg_hash_spec* spec, const int64_t* tokens, int64_t n_pos, int64_t seq_len,
                 const int32_t* seg_start, int32_t global_ids, int32_t* rows_out, void* stream) {
  LayerHash L;
  int rc = make_layer_hash(spec, &L);
  if (rc != EG_OK) return rc;
  EG_CHECK_ARG(n_pos >= 0, "n_pos < 0");
  if (n_pos == 0) return EG_OK;
  EG_CHECK_ARG(tokens != nullptr && rows_out != nullptr, "tokens/rows_out is NULL");
  const int64_t n = n_pos * L.n_heads;
  hipLaunchKernelGGL(hash_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, L,
                     tokens, n_pos, seq_len, seg_start, global_ids, rows_out);
  return launch_status("hash_kernel");
}

static int forward_entry(int32_t n_layers, const eg_hash_spec* specs, const eg_table* tables,
                         const eg_overlay* overlays, const int64_t* tokens, int64_t n_pos, int64_t seq_len,
                         const int32_t* seg_start, int32_t decode_ctx, const uint16_t* residual, void* out,
                         int32_t* rows_out, int32_t* vars_out, void* stream) {
  EG_CHECK_ARG(n_layers >= 1 && n_layers <= EG_MAX_LAYERS, "n_layers=%d outside [1, %d]", n_layers,
               EG_MAX_LAYERS);
  EG_CHECK_ARG(decode_ctx >= 0, "decode_ctx < 0");
  EG_CHECK_ARG(specs != nullptr && tables != nullptr, "specs/tables is NULL");
  EG_CHECK_ARG(n_pos >= 0 && n_pos < (1LL << 30), "n_pos=%lld outside [0, 2^30)", (long long)n_pos);
  EG_CHECK_ARG(n_pos == 0 || (tokens != nullptr && out != nullptr), "tokens/out is NULL");
  FwdArgs a;
  memset(&a, 0, sizeof(a));
  for (int l = 0; l < n_layers; ++l) {
    int rc = make_layer_hash(&specs[l], &a.hash[l]);
    if (rc != EG_OK) return rc;
    rc = make_table(&tables[l], &a.table[l], "table");
    if (rc != EG_OK) return rc;
    EG_CHECK_ARG(tables[l].fmt == tables[0].fmt && tables[l].dim == tables[0].dim,
                 "layer %d: format/dim differ from layer 0", l);
    EG_CHECK_ARG(a.hash[l].n_heads == a.hash[0].n_heads, "layer %d: n_heads differ from layer 0", l);
    for (int h = 0; h < a.hash[l].n_heads; ++h)
      EG_CHECK_ARG((int64_t)a.hash[l].offset[h] + a.hash[l].vocab[h] <= tables[l].n_rows,
                   "layer %d head %d: rows [%d, %lld) exceed the table's %lld rows", l, h, a.hash[l].offset[h],
                   (long long)a.hash[l].offset[h] + a.hash[l].vocab[h], (long long)tables[l].n_rows);
    rc = fill_overlay(overlays ? &overlays[l] : nullptr, a.table[l], &a.ov[l]);
    if (rc != EG_OK) return rc;
  }
  a.tokens = tokens;
  a.seg_start = seg_start;
  a.residual = residual;
  a.out = out;
  a.rows_out = rows_out;
  a.vars_out = vars_out;
  a.seq_len = seq_len;
  a.n_pos = n_pos;
  a.n_layers = n_layers;
  a.heads = a.hash[0].n_heads;
  a.dim = tables[0].dim;
  const int W = a.heads * a.dim;
  EG_CHECK_ARG(W <= kMaxWidth, "row width %d > %d", W, kMaxWidth);
  a.decode_ctx = decode_ctx;
  return residual ? launch_forward<false>(a, (hipStream_t)stream) : launch_forward<true>(a, (hipStream_t)stream);
}

int eg_forward(int32_t n_layers, const eg_hash_spec* specs, const eg_table* tables, const eg_overlay* overlays,
               const int64_t* tokens, int64_t n_pos, int64_t seq_len, const int32_t* seg_start,
               const uint16_t* residual, void* out, int32_t* rows_out, void* stream) {
  return forward_entry(n_layers, specs, tables, overlays, tokens, n_pos, seq_len, seg_start, 0, residual, out,
                       rows_out, nullptr, stream);
}

int eg_forward_slots(int32_t n_layers, const eg_hash_spec* specs, const eg_table* tables,
                     const eg_overlay* overlays, const int64_t* tokens, int64_t n_pos, int64_t seq_len,
                     const int32_t* seg_start, const uint16_t* residual, void* out, int32_t* rows_out,
                     int32_t* slot_var_out, void* stream) {
  EG_CHECK_ARG(slot_var_out != nullptr, "slot_var_out is NULL");
  return forward_entry(n_layers, specs, tables, overlays, tokens, n_pos, seq_len, seg_start, 0, residual, out,
                       rows_out, slot_var_out, stream);
}

int eg_forward_decode(int32_t n_layers, const eg_hash_spec* specs, const eg_table* tables,
                      const eg_overlay* overlays, const int64_t* tokens, int64_t n_seq, int32_t ctx_len,
                      const uint16_t* residual, void* out, int32_t* rows_out, void* stream) {
  EG_CHECK_ARG(ctx_len >= 1, "ctx_len=%d < 1", ctx_len);
  return forward_entry(n_layers, specs, tables, overlays, tokens, n_seq, 0, nullptr, ctx_len, residual, out,
                       rows_out, nullptr, stream);
}

int eg_forward_timed(int32_t n_layers, const eg_hash_spec* specs, const eg_table* tables,
                     const eg_overlay* overlays, const int64_t* tokens, int64_t n_pos, int64_t seq_len,
                     const int32_t* seg_start, const uint16_t* residual, void* out, int32_t* rows_out,
                     void* start_event, void* stop_event, void* stream) {
  EG_CHECK_ARG(start_event != nullptr && stop_event != nullptr, "start_event/stop_event is NULL");
  g_ev_start = (hipEvent_t)start_event;
  g_ev_stop = (hipEvent_t)stop_event;
  const int rc = eg_forward(n_layers, specs, tables, overlays, tokens, n_pos, seq_len, seg_start, residual, out,
                            rows_out, stream);
  g_ev_start = nullptr;
  g_ev_stop = nullptr;
  return rc;
}

int eg_forward_rows(int32_t n_layers, const eg_table* tables, const eg_overlay* overlays, const int32_t* rows,
                    int64_t n_pos, int32_t heads, const uint16_t* residual, uint16_t* out, void* stream) {
  EG_CHECK_ARG(n_layers >= 1 && n_layers <= EG_MAX_LAYERS, "n_layers=%d outside [1, %d]", n_layers,
               EG_MAX_LAYERS);
  EG_CHECK_ARG(tables != nullptr, "tables is NULL");
  EG_CHECK_ARG(heads >= 1 && heads <= EG_MAX_HEADS, "heads=%d outside [1, %d]", heads, EG_MAX_HEADS);
  EG_CHECK_ARG(n_pos >= 0 && n_pos < (1LL << 30), "n_pos=%lld outside [0, 2^30)", (long long)n_pos);
  EG_CHECK_ARG(n_pos == 0 || (rows != nullptr && residual != nullptr && out != nullptr),
               "rows/residual/out is NULL");
  FwdArgs a;
  memset(&a, 0, sizeof(a));
  for (int l = 0; l < n_layers; ++l) {
    int rc = make_table(&tables[l], &a.table[l], "table");
    if (rc != EG_OK) return rc;
    EG_CHECK_ARG(tables[l].fmt == tables[0].fmt && tables[l].dim == tables[0].dim,
                 "layer %d: format/dim differ from layer 0", l);
    EG_CHECK_ARG(tables[l].n_rows >= 1, "layer %d: n_rows=%lld (at least one row)", l,
                 (long long)tables[l].n_rows);
    rc = fill_overlay(overlays ? &overlays[l] : nullptr, a.table[l], &a.ov[l]);
    if (rc != EG_OK) return rc;
  }
  a.rows_in = rows;
  a.residual = residual;
  a.out = out;
  a.n_pos = n_pos;
  a.n_layers = n_layers;
  a.heads = heads;
  a.dim = tables[0].dim;
  const int W = heads * a.dim;
  EG_CHECK_ARG(W <= kMaxWidth, "row width %d > %d", W, kMaxWidth);
  return launch_forward<false>(a, (hipStream_t)stream);
}

int eg_lookup_rows(const int32_t* rows, int64_t n, const int32_t* ids, const int32_t* index, int64_t n_ids,
                   int32_t* out, int64_t* counts, void* stream) {
  EG_CHECK_ARG(n >= 0 && n_ids >= 0, "n=%lld n_ids=%lld", (long long)n, (long long)n_ids);
  EG_CHECK_ARG(n == 0 || rows != nullptr, "rows is NULL");
  EG_CHECK_ARG(n_ids == 0 || ids != nullptr, "ids is NULL");
  if (n == 0) return EG_OK;
  hipLaunchKernelGGL(lookup_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, rows, n,
                     ids, index, n_ids, out, (unsigned long long*)counts);
  return launch_status("lookup_kernel");
}

int eg_gather_slots(const eg_table* table, const int32_t* rows, const int32_t* slot_var, int64_t n_pos,
                    int32_t heads, const float* vars, int64_t n_vars, float* out, void* stream) {
  EG_CHECK_ARG(heads >= 1 && heads <= EG_MAX_HEADS, "heads=%d outside [1, %d]", heads, EG_MAX_HEADS);
  EG_CHECK_ARG(n_pos >= 0 && n_pos < (1LL << 30) && n_vars >= 0, "n_pos=%lld n_vars=%lld", (long long)n_pos,
               (long long)n_vars);
  EG_CHECK_ARG(n_pos == 0 || (rows != nullptr && slot_var != nullptr && out != nullptr),
               "rows/slot_var/out is NULL");
  EG_CHECK_ARG(n_vars == 0 || vars != nullptr, "vars is NULL");
  FwdArgs a;
  memset(&a, 0, sizeof(a));
  int rc = make_table(table, &a.table[0], "table");
  if (rc != EG_OK) return rc;
  EG_CHECK_ARG(table->n_rows >= 1, "table: n_rows=%lld (at least one row)", (long long)table->n_rows);
  a.ov[0].rows.payload = (const uint8_t*)vars;
  a.ov[0].rows.n_rows = n_vars;
  a.ov[0].rows.fmt = EG_FMT_F32;
  a.ov[0].rows.dim = table->dim;
  a.rows_in = rows;
  a.slot_var = slot_var;
  a.out = out;
  a.n_pos = n_pos;
  a.n_layers = 1;
  a.heads = heads;
  a.dim = table->dim;
  const int W = heads * a.dim;
  EG_CHECK_ARG(W <= kMaxWidth, "row width %d > %d", W, kMaxWidth);
  return launch_forward<true>(a, (hipStream_t)stream);
}

int eg_gather(const eg_table* table, const eg_overlay* overlay, const int32_t* rows, int64_t n_pos, int32_t heads,
              float* out, void* stream) {
  EG_CHECK_ARG(heads >= 1 && heads <= EG_MAX_HEADS, "heads=%d outside [1, %d]", heads, EG_MAX_HEADS);
  EG_CHECK_ARG(n_pos >= 0 && n_pos < (1LL << 30), "n_pos=%lld outside [0, 2^30)", (long long)n_pos);
  EG_CHECK_ARG(n_pos == 0 || (rows != nullptr && out != nullptr), "rows/out is NULL");
  FwdArgs a;
  memset(&a, 0, sizeof(a));
  int rc = make_table(table, &a.table[0], "table");
  if (rc != EG_OK) return rc;
  EG_CHECK_ARG(table->n_rows >= 1, "table: n_rows=%lld (at least one row)", (long long)table->n_rows);
  rc = fill_overlay(overlay, a.table[0], &a.ov[0]);
  if (rc != EG_OK) return rc;
  a.rows_in = rows;
  a.out = out;
  a.n_pos = n_pos;
  a.n_layers = 1;
  a.heads = heads;
  a.dim = table->dim;
  const int W = heads * a.dim;
  EG_CHECK_ARG(W <= kMaxWidth, "row width %d > %d", W, kMaxWidth);
  return launch_forward<true>(a, (hipStream_t)stream);
}

// GGML wire blocks (the byte form read_rows_raw returns) to f32, one value a
// thread: Q8_0 [fp16 d][32 x int8], IQ4_NL [fp16 d][16 nibble bytes], MXFP8
// [e8m0][32 x e4m3], BF16 and F32 one value a block.  Byte loads: the blocks
// sit at 34-, 18- and 33-byte strides.
__global__ __launch_bounds__(256) void dequant_wire_kernel(int fmt, const uint8_t* __restrict__ raw, int64_t n_values,
                                                           float* __restrict__ out) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n_values; i += (int64_t)gridDim.x * 256) {
    const int64_t b = i >> 5;
    const int j = (int)(i & 31);
    float y;
    if (fmt == EG_FMT_Q8_0) {
      const uint8_t* blk = raw + b * 34;
      y = (float)(int8_t)blk[2 + j] * f16_to_f32((uint16_t)(blk[0] | ((uint32_t)blk[1] << 8)));
    } else if (fmt == EG_FMT_IQ4_NL) {
      const uint8_t* blk = raw + b * 18;
      const uint32_t byte = blk[2 + (j & 15)];
      y = iq4nl_value(j < 16 ? (byte & 15u) : (byte >> 4)) * f16_to_f32((uint16_t)(blk[0] | ((uint32_t)blk[1] << 8)));
    } else if (fmt == EG_FMT_MXFP8) {
      const uint8_t* blk = raw + b * 33;
      y = e4m3_to_f32(blk[1 + j]) * e8m0_to_f32(blk[0]);
    } else if (fmt == EG_FMT_BF16) {
      y = __uint_as_float((uint32_t)(raw[2 * i] | ((uint32_t)raw[2 * i + 1] << 8)) << 16);
    } else {
      y = __uint_as_float((uint32_t)raw[4 * i] | ((uint32_t)raw[4 * i + 1] << 8) | ((uint32_t)raw[4 * i + 2] << 16) |
                          ((uint32_t)raw[4 * i + 3] << 24));
    }
    out[i] = y;
  }
}

int eg_dequant_blocks(int32_t fmt, const void* raw, int64_t n_blocks, float* out, void* stream) {
  EG_CHECK_ARG(fmt >= EG_FMT_BF16 && fmt <= EG_FMT_F32, "fmt=%d is not an eg_row_format", fmt);
  EG_CHECK_ARG(n_blocks >= 0 && n_blocks < (1LL << 40), "n_blocks=%lld outside [0, 2^40)", (long long)n_blocks);
  EG_CHECK_ARG(n_blocks == 0 || (raw != nullptr && out != nullptr), "raw/out is NULL");
  const int64_t per_block = (fmt == EG_FMT_BF16 || fmt == EG_FMT_F32) ? 1 : 32;
  const int64_t n_values = n_blocks * per_block;
  if (n_values == 0) return EG_OK;
  const int64_t blocks = (n_values + 255) / 256 < 16384 ? (n_values + 255) / 256 : 16384;
  hipLaunchKernelGGL(dequant_wire_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, (int)fmt,
                     (const uint8_t*)raw, n_values, out);
  return launch_status("dequant_wire_kernel");
}

}  // extern "C"
