/*
 * engraft_ngram.h -- C ABI of the MI355X (gfx950) Engram/PLE n-gram table path.
 *
 * Plain C: device pointers and sizes, an explicit hipStream_t passed as void*,
 * an int status (EG_OK == 0, negative on error; eg_last_error() gives the
 * message of the calling thread's last failure).  No entry point allocates
 * device memory except where stated; every buffer is caller-owned.  Calls are
 * asynchronous on `stream` and never synchronise unless stated.
 *
 * Reference interfaces replaced (fulvian/engraft-ngram, Python):
 *   eg_hash_rows     PleTable.ngram_addresses        engraft/table.py:111-144
 *                    (+ local_to_global              engraft/lens.py:108-110,
 *                     vectorized ngram_rows          engraft/damage.py:68-104)
 *   eg_gather        PleTable.read_rows(_raw) + dequant_iq4nl
 *                                                    engraft/table.py:90-109,147-169
 *   eg_dequant_blocks  dequant_q8_0 / _bf16 / _iq4_nl / _f32 of the wire form
 *                                                    engraft/replica/dequant.py:71-147
 *                    _read_true_rows                 engraft/replica/distill.py:378-395
 *   eg_forward       RowSet.from_position per position + overlay substitution
 *                    + the residual consumer         engraft/lens.py:126-136,
 *                                                    engraft/replica/model.py:473-495,845-853,
 *                                                    engraft/replica/seq.py:372-444
 *   eg_scatter_grad  autograd of rows_var[idx_r] + index_put (accumulate)
 *   (+ _slots, _plan_slots / _apply)                 engraft/replica/seq.py:433-441
 *   eg_lookup_rows   row_map / sorted-overlay membership + read counts
 *                                                    engraft/replica/seq.py:412-417,
 *                                                    engraft/damage.py:192-197
 *   eg_scan_overlay  the damage scan of a token block  engraft/damage.py:159-224
 *   eg_gather_slots  OverlayEmb.build's base gather + index_put
 *                                                    engraft/replica/seq.py:372-444
 *   eg_descent_step  scatter + torch.optim.Adam step on the overlay rows
 *   (= eg_descent_plan + eg_descent_apply)           engraft/descend_corpus.py:785-790,921-947
 *   eg_forward_decode  the per-token gather of a decode step with the overlay
 *                                                    engraft/replica/model.py:473-495
 *   eg_ple_gate, eg_ple_conv  ple_forward after its two projections
 *   (+ _backward)    and the autograd of it          engraft/replica/layers.py:565-626
 *   eg_ple_rms, eg_ple_conv's other modes  PleReplica engraft/lens.py:221-385
 *   eg_split_bf16, eg_gemm_bf16x3, eg_gemm_f32 (+ _workspace_size),
 *   eg_split_bf16x6, eg_gemm_bf16x6
 *                    ple_forward's projections and their backward
 *                                                    engraft/replica/layers.py:594-606
 */
#ifndef ENGRAFT_NGRAM_H
#define ENGRAFT_NGRAM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EG_ABI_VERSION 4

#define EG_MAX_NGRAM 4   /* context slots per hash (2-, 3- and 4-grams) */
#define EG_MAX_HEADS 32  /* row slots per position and table layer */
#define EG_MAX_LAYERS 2  /* table layers summed by one eg_forward */

enum eg_status {
  EG_OK = 0,
  EG_ERR_ARG = -1,         /* invalid argument (shape, pointer, range) */
  EG_ERR_HIP = -2,         /* a HIP runtime call failed */
  EG_ERR_UNSUPPORTED = -3, /* valid but not built (format/dim combination) */
  EG_ERR_WORKSPACE = -4    /* workspace too small */
};

enum eg_row_format {
  EG_FMT_BF16 = 1,   /* payload bf16 [rows, dim]                                  */
  EG_FMT_Q8_0 = 2,   /* payload int8 [rows, dim] + scales fp16 [rows, dim/32]     */
  EG_FMT_MXFP8 = 3,  /* payload e4m3 [rows, dim] + scales e8m0 u8 [rows, dim/32]  */
  EG_FMT_IQ4_NL = 4, /* payload u8 [rows, dim/32*18], GGML IQ4_NL blocks          */
  EG_FMT_F32 = 5     /* payload f32 [rows, dim]                                   */
};

/* Hash parameters of one table layer (engraft/table.py:60-67).  Head h belongs
 * to order n = 2 + h / heads_per_ngram and reads
 *   global = head_offsets[h] + (XOR_{j<n} ctx[j]*mult_h[j] mod 2^64) % head_vocab_sizes[h]
 * where ctx = [x_t, x_{t-1}, ...] with the reference's EOS rule.  mult_h is
 * layer_multipliers (the reference's mode) unless head_multipliers is given. */
typedef struct eg_hash_spec {
  uint64_t eos_token_id;
  int32_t ngram_size;                    /* 2..EG_MAX_NGRAM                       */
  int32_t heads_per_ngram;               /* n_heads = (ngram_size-1)*heads_per_ngram */
  uint64_t layer_multipliers[EG_MAX_NGRAM];
  const uint64_t* head_multipliers;      /* DEVICE pointer [n_heads][ngram_size] or NULL */
  uint64_t head_vocab_sizes[EG_MAX_HEADS]; /* each in [1, 2^32)                   */
  int64_t head_offsets[EG_MAX_HEADS];    /* offset + vocab <= 2^31 - 1            */
} eg_hash_spec;

/* A table (or an overlay's row store) resident in device memory; rows are
 * indexed by global row id. */
typedef struct eg_table {
  int32_t fmt;          /* eg_row_format */
  int32_t dim;          /* values per row, a multiple of 32, <= 512 */
  int64_t n_rows;
  const void* payload;  /* device */
  const void* scales;   /* device; Q8_0 and MXFP8 only, NULL otherwise */
  int64_t row_stride;   /* bytes from one row of payload to the next; 0: the
                           format's own row size.  IQ4_NL may take more (rows
                           padded to whole 128-byte lines, so that a random row
                           read is one line); every other format 0 */
} eg_table;

/* Replacement rows resolved per id (engraft/replica/model.py:473-495):
 * a slot whose global row equals ids[k] reads row index[k] (or k when index is
 * NULL) of `rows` instead of the base table. */
typedef struct eg_overlay {
  int64_t n;               /* 0: no overlay */
  const int32_t* ids;      /* device, sorted ascending, unique */
  const int32_t* index;    /* device or NULL */
  eg_table rows;           /* rows.dim must equal the base table's dim */
  const uint32_t* bitmap;  /* device or NULL: eg_build_id_bitmap of ids over n_bits rows
                              (covering every row id looked up); resolves the lookups
                              in place of the binary search, same results */
  int64_t n_bits;
} eg_overlay;

const char* eg_last_error(void);
int eg_abi_version(void);

/* Row ids of every position of a flat token stream.
 * tokens int64 [n_pos]; the hash context of position p never reaches before
 * its segment start: seg_start[p] when seg_start != NULL, otherwise
 * (p / seq_len) * seq_len (seq_len <= 0: one sequence).
 * rows_out int32 [n_pos, n_heads]; global_ids = 0 gives local rows. */
int eg_hash_rows(const eg_hash_spec* spec, const int64_t* tokens, int64_t n_pos,
                 int64_t seq_len, const int32_t* seg_start, int32_t global_ids,
                 int32_t* rows_out, void* stream);

/* Fused forward over n_layers (1..EG_MAX_LAYERS) table layers with the same
 * n_heads and dim (W = n_heads*dim):
 *   residual != NULL: out bf16 [n_pos, W] = bf16_rne(f32(residual) + emb_0 + ...)
 *   residual == NULL: out f32  [n_pos, W] = emb_0 + ... (the OverlayEmb base)
 * overlays: NULL or n_layers entries.  rows_out: NULL or int32
 * [n_layers, n_pos, n_heads] global ids (for the backward).  out may alias
 * residual (in-place residual update). */
int eg_forward(int32_t n_layers, const eg_hash_spec* specs, const eg_table* tables,
               const eg_overlay* overlays, const int64_t* tokens, int64_t n_pos,
               int64_t seq_len, const int32_t* seg_start, const uint16_t* residual,
               void* out, int32_t* rows_out, void* stream);

/* eg_forward that also writes, per slot, the overlay row it read:
 * slot_var_out int32 [n_layers, n_pos, n_heads], the row of overlays[l]'s store
 * (its index entry, or the rank of the id among overlays[l].ids when index is
 * NULL), -1 where the slot read the base table.  Over a descent state's
 * overlay (ids = the variables, no index) these are the slots' variables, the
 * idx_r of the reference's OverlayEmb (engraft/replica/seq.py:401-441), which
 * eg_descent_plan_slots groups without a row lookup. */
int eg_forward_slots(int32_t n_layers, const eg_hash_spec* specs, const eg_table* tables,
                     const eg_overlay* overlays, const int64_t* tokens, int64_t n_pos,
                     int64_t seq_len, const int32_t* seg_start, const uint16_t* residual,
                     void* out, int32_t* rows_out, int32_t* slot_var_out, void* stream);

/* Decode step: one new position per sequence.  tokens int64 [n_seq, ctx_len]
 * holds each sequence's last ctx_len tokens (the new one last; the hash never
 * looks before the first); residual / out / rows_out as eg_forward with
 * n_pos = n_seq: the embedding of every sequence's last position
 * (engraft/replica/model.py:473-495 at t = the new token; the engine's
 * per-token gather with the overlay resolved per id). */
int eg_forward_decode(int32_t n_layers, const eg_hash_spec* specs, const eg_table* tables,
                      const eg_overlay* overlays, const int64_t* tokens, int64_t n_seq,
                      int32_t ctx_len, const uint16_t* residual, void* out, int32_t* rows_out,
                      void* stream);

/* eg_forward with the row ids given: rows int32 [n_layers, n_pos, heads]
 * global ids (eg_forward's rows_out layout, e.g. ids hashed once and read
 * again after an overlay update), the rows read, dequantised, substituted by
 * the overlays and added to the bf16 residual exactly as eg_forward does; an
 * id outside its table reads NaN.  It replaces the row reads of
 * RowSet.from_position for known addresses (engraft/lens.py:133-135,
 * engraft/table.py:90-109); with the hash left out it is also the hash-free
 * reference point of eg_forward's time. */
int eg_forward_rows(int32_t n_layers, const eg_table* tables, const eg_overlay* overlays,
                    const int32_t* rows, int64_t n_pos, int32_t heads, const uint16_t* residual,
                    uint16_t* out, void* stream);

/* Streaming copy of `bytes` (a multiple of 16, 16-byte aligned pointers) with
 * the library's own non-temporal 16-byte load/store kernel.  No counterpart in
 * the reference: it measures the device's streaming ceiling that the forward
 * kernels' rooflines are read against. */
int eg_stream_copy(const void* src, void* dst, int64_t bytes, void* stream);

/* eg_forward with the kernel launched through hipExtLaunchKernelGGL, so that
 * start_event / stop_event (hipEvent_t, created by the caller) hold the
 * dispatch's own start and end timestamps.  No counterpart in the reference:
 * a measurement hook for benchmarks (kernel time without the gaps of event
 * packets around the launch). */
int eg_forward_timed(int32_t n_layers, const eg_hash_spec* specs, const eg_table* tables,
                     const eg_overlay* overlays, const int64_t* tokens, int64_t n_pos,
                     int64_t seq_len, const int32_t* seg_start, const uint16_t* residual,
                     void* out, int32_t* rows_out, void* start_event, void* stop_event,
                     void* stream);

/* Gather by explicit global row ids: rows int32 [n_pos, heads] ->
 * out f32 [n_pos, heads*dim] (dequantised, overlay resolved; NULL overlay = base). */
int eg_gather(const eg_table* table, const eg_overlay* overlay, const int32_t* rows,
              int64_t n_pos, int32_t heads, float* out, void* stream);

/* Dequantisation of rows in their GGML wire form (the bytes read_rows_raw
 * returns), n_blocks blocks of format fmt -> out f32:
 *   EG_FMT_Q8_0    34-byte blocks [fp16 d][32 x int8]      -> 32 values, y = f32(q) * f32(d)
 *   EG_FMT_IQ4_NL  18-byte blocks [fp16 d][16 nibble bytes] -> 32 values
 *   EG_FMT_MXFP8   33-byte blocks [e8m0][32 x e4m3]          -> 32 values
 *   EG_FMT_BF16    2-byte blocks -> 1 value (bits << 16); EG_FMT_F32 4 bytes -> 1 value.
 * raw may sit at any byte alignment.  Replaces dequant_q8_0 / dequant_bf16 /
 * dequant_iq4_nl / dequant_f32 (engraft/replica/dequant.py:71-93,127-147). */
int eg_dequant_blocks(int32_t fmt, const void* raw, int64_t n_blocks, float* out, void* stream);

/* ---- descent backward ----------------------------------------------------
 * The overlay variables are R rows with sorted unique global ids
 * (engraft/replica/distill.py:401-453 row_map, ascending).  Every slot (p, h)
 * whose row id is one of them contributes d_out[p, h*dim:(h+1)*dim] to that
 * variable's gradient (the autograd of rows_var[idx_r] + index_put,
 * engraft/replica/seq.py:433-441).  The slots are grouped per variable and
 * each variable's contributions are summed in ascending slot order: the result
 * is bitwise repeatable and independent of scheduling. */

/* Adam hyper-parameters of one step (torch.optim.Adam, engraft/descend_corpus.py:785-790). */
typedef struct eg_adam {
  double lr, beta1, beta2, eps; /* doubles, like torch's Python scalars: lr/(1-beta1^t) and
                                   1-beta1 are formed in double and rounded to fp32 once */
  int64_t step;     /* the step being taken: 1 on the first */
  int32_t dense;    /* 1: every variable row steps, as torch.optim.Adam([rows_var]) does;
                       0: only the rows hit by this batch (sparse / lazy Adam) */
  float l2_coef;    /* mu / ||rows0||^2 of engraft/descend_corpus.py:935-939 (0: no pull
                       term) */
  const float* anchor; /* DEVICE f32 [R, dim]: rows0 of the pull term, row k for variable k
                          (descend_corpus's warm-start rows, :780-781); NULL: rows0 = the base
                          table's rows of the variables' ids (replica/descend.py:141, the true
                          rows) */
} eg_adam;

/* Optimizer state of the R overlay variables, all device memory. */
typedef struct eg_descent_state {
  int64_t n;          /* R */
  int32_t dim;
  const int32_t* ids; /* [R] sorted unique global rows */
  float* master;      /* R fp32 rows of dim (rows_var), row_stride floats apart */
  float* m;           /* R rows: Adam first moment, the same layout */
  float* v;           /* R rows: Adam second moment, the same layout */
  int32_t* stamp;     /* [R] last dense step that hit the row (0 before the first) */
  eg_table quant;     /* requantised copy [R] written after the update (Q8_0 or MXFP8;
                         payload NULL: none) -- the rows a forward overlay reads */
  const int64_t* index;   /* optional eg_build_row_index table of ids (NULL: the ids are
                             searched directly) */
  int64_t index_capacity;
  int64_t row_stride; /* floats from one variable's row of master, m and v to the next:
                         0 or dim for three [R, dim] arrays; 3 dim for one [R][3][dim]
                         buffer with master, m and v at its offsets 0, dim and 2 dim (a
                         variable's state one 1.5 KB run at dim 128: a config-2 step
                         3 % faster); at least dim */
} eg_descent_state;

/* Builds an open-addressing index of sorted unique ids for the backward's
 * lookups: table int64 [capacity] (capacity a power of two >= max(8, 2*n),
 * 16-byte aligned; 64-byte aligned, a lookup reads one memory line), entries
 * (row << 32 | position in ids), -1 when empty, linear probing.  The lookups
 * read aligned groups of 8 entries.  Built once per state. */
int eg_build_row_index(const int32_t* ids, int64_t n, int64_t* table, int64_t capacity, void* stream);

/* Workspace bytes eg_scatter_grad(_slots) / eg_descent_step need for
 * n_slots = n_pos*heads slots and n_var variables (no initial contents needed). */
size_t eg_backward_workspace_size(int64_t n_slots, int64_t n_var);

/* grad_out f32 [n_var, dim] += sum over slots hitting each variable (rows not
 * hit are left untouched: pass a zeroed buffer for the plain gradient).
 * d_out: bf16 (d_out_f32 = 0) or f32 [n_pos, heads*dim]; rows int32 [n_pos, heads]. */
int eg_scatter_grad(const void* d_out, int32_t d_out_f32, const int32_t* rows, int64_t n_pos,
                    int32_t heads, int32_t dim, const int32_t* ids, int64_t n_var,
                    float* grad_out, void* workspace, size_t workspace_bytes, void* stream);

/* One descent step: gradient as eg_scatter_grad, then Adam on state->master/m/v
 * (torch's single-tensor op order, fp32), then requantisation into state->quant.
 * base: the table the variables were read from (needed when opt->l2_coef != 0 and
 * opt->anchor is NULL). */
int eg_descent_step(const void* d_out, int32_t d_out_f32, const int32_t* rows, int64_t n_pos,
                    int32_t heads, const eg_descent_state* state, const eg_adam* opt,
                    const eg_table* base, void* workspace, size_t workspace_bytes, void* stream);

/* The two halves of eg_descent_step, for a descent loop that groups the next
 * step's slots while the current step runs (the grouping depends only on the
 * row ids, which the hash fixes from the tokens: the reference's loop packs a
 * whole pass before its first step, engraft/descend_corpus.py:855-870).
 * eg_descent_plan groups the slots of rows int32 [n_pos, heads] by variable of
 * `state` into `workspace` (eg_backward_workspace_size(n_pos*heads, state->n)
 * bytes); eg_descent_apply is the rest of eg_descent_step (segmented reduce in
 * slot order, Adam, requantisation) from a workspace holding the plan of the
 * same n_pos, heads and state, made on the same stream or ordered before it by
 * the caller.  A workspace holds one plan.  The apply writes it too: it sorts
 * each variable's range of more than 4,096 slot ids in place, into the order
 * the slots are summed in, which leaves the grouping as it was (an apply again
 * from the same plan sums the same way), but applies of one workspace that
 * overlap race.  Plan into a workspace only after the apply that reads it has
 * run.  plan + apply on one workspace is eg_descent_step, bitwise. */
int eg_descent_plan(const int32_t* rows, int64_t n_pos, int32_t heads, const eg_descent_state* state,
                    void* workspace, size_t workspace_bytes, void* stream);
/* eg_descent_plan from the slots' variables instead of their rows: slot_var
 * int32 [n_pos, heads], the variable (row of state->ids) each slot read, any
 * value outside [0, state->n) for none -- what eg_forward_slots writes for the
 * state's overlay.  The reference's backward scatters by the forward's
 * variable indices the same way (engraft/replica/seq.py:433-441, the autograd
 * of index_put by idx_r); no row lookup is needed. */
int eg_descent_plan_slots(const int32_t* slot_var, int64_t n_pos, int32_t heads,
                          const eg_descent_state* state, void* workspace, size_t workspace_bytes,
                          void* stream);
int eg_descent_apply(const void* d_out, int32_t d_out_f32, int64_t n_pos, int32_t heads,
                     const eg_descent_state* state, const eg_adam* opt, const eg_table* base,
                     void* workspace, size_t workspace_bytes, void* stream);

/* eg_descent_step without a workspace argument: it allocates nothing (no
 * hipMalloc, no library allocation).  No counterpart in the reference; it is
 * for callers that cannot allocate device memory (code under HIP stream
 * capture, tight serving loops).  The grouping scratch is a static device array
 * of eg_descent_step_noalloc_max_bytes() (16 MiB) per GPU, held until the
 * process ends; a call whose n_pos*heads slots and state->n variables need more
 * (eg_backward_workspace_size) fails with EG_ERR_WORKSPACE.  Every call on one
 * GPU shares that array: calls that overlap on one GPU (two streams, two
 * threads) race and must be serialised by the caller.  Results are bitwise
 * those of eg_descent_step. */
int eg_descent_step_noalloc(const void* d_out, int32_t d_out_f32, const int32_t* rows, int64_t n_pos,
                            int32_t heads, const eg_descent_state* state, const eg_adam* opt,
                            const eg_table* base, void* stream);
size_t eg_descent_step_noalloc_max_bytes(void);

/* The requantisation eg_descent_step applies after its update, on its own:
 * fp32 rows src [n, dim] -> rows dst_rows[i] (i when dst_rows is NULL) of dst
 * (Q8_0 or MXFP8); a dst_rows entry outside dst is skipped.  No counterpart in
 * the reference, whose overlays stay fp32 (engraft/lens.py:167-198): it makes
 * a descent state's quantised overlay valid before its first step and
 * restores the frozen rows of the masked step (engraft/replica/descend.py:
 * 262-271). */
int eg_quantize_rows(const float* src, int64_t n, int32_t dim, const int32_t* dst_rows,
                     const eg_table* dst, void* stream);

/* ---- per-slot variables (OverlayEmb) ---------------------------------------
 * Variable index of each row id: out[i] = index[k] (k when index is NULL) for
 * rows[i] == ids[k], else -1; counts (optional, int64 [n_ids], accumulated)
 * += the number of reads of each id (engraft/damage.py:192-197 read_count). */
int eg_lookup_rows(const int32_t* rows, int64_t n, const int32_t* ids, const int32_t* index,
                   int64_t n_ids, int32_t* out, int64_t* counts, void* stream);

/* Damage scan of one token block (engraft/damage.py:159-224, fused): positions
 * start..n_tokens-1 of tokens (device, int32 when token_bytes is 4, int64 when
 * 8, the block as one sequence) hash
 * their rows; each row is looked up in the sorted overlay ids (int32 [n_ids],
 * n_ids >= 1) and, per position, n_hit int32 = the rows found, dnorm_max /
 * dnorm_sum f32 = max / sum of dnorm[k] over them (0 when none); read_counts
 * int64 [n_ids] += the reads of every overlay row.  Outputs have n_tokens -
 * start entries.  No per-slot array is written.  bitmap (optional, from
 * eg_build_id_bitmap over the same ids, n_bits covering every row id) replaces
 * the binary search with a probe of the rank bitmap. */
int eg_scan_overlay(const eg_hash_spec* spec, const void* tokens, int32_t token_bytes, int64_t n_tokens,
                    int64_t start, const int32_t* ids, int64_t n_ids, const uint32_t* bitmap,
                    int64_t n_bits, const float* dnorm, int32_t* n_hit, float* dnorm_max,
                    float* dnorm_sum, int64_t* read_counts, void* stream);

/* Rank bitmap of sorted, unique overlay ids for eg_scan_overlay and the
 * forward's overlay lookups: bitmap is uint32 [eg_id_bitmap_words(n_bits)],
 * 8-byte aligned, = 2 * nw + 2 * ceil(nw/64) with nw = ceil(n_bits/32).
 * Pair w < nw: bitmap[2 w] has bit b set for every id 32 w + b < n_bits (all
 * other bits cleared), bitmap[2 w + 1] = the number of ids below 32 w.  Then
 * ceil(nw/64) 64-bit filter blocks: a blocked Bloom filter of the ids below
 * n_bits (each id sets five bits of one block, picked by a hash of the id; no
 * false negatives).  A lookup reads its filter block and, only when that
 * passes, its pair.  No counterpart in the reference: it turns the scan's
 * per-lookup binary search into one or two probes. */
int64_t eg_id_bitmap_words(int64_t n_bits);
int eg_build_id_bitmap(const int32_t* ids, int64_t n_ids, uint32_t* bitmap, int64_t n_bits, void* stream);

/* Gather with per-slot replacement rows (engraft/replica/seq.py:433-441):
 * out f32 [n_pos, heads*dim]; slot (p, h) reads vars[slot_var[p, h]] (f32
 * [n_vars, dim]) when slot_var[p, h] >= 0, else the table row rows[p, h]. */
int eg_gather_slots(const eg_table* table, const int32_t* rows, const int32_t* slot_var,
                    int64_t n_pos, int32_t heads, const float* vars, int64_t n_vars, float* out,
                    void* stream);

/* eg_scatter_grad keyed by per-slot variables: grad_out f32 [n_var, dim] +=
 * the d_out slices of the slots with slot_var == k (slot_var < 0: none),
 * merged deterministically as in eg_scatter_grad. */
int eg_scatter_grad_slots(const void* d_out, int32_t d_out_f32, const int32_t* slot_var,
                          int64_t n_pos, int32_t heads, int32_t dim, int64_t n_var,
                          float* grad_out, void* workspace, size_t workspace_bytes, void* stream);

/* eg_scatter_grad_slots in two halves, for a slot-to-variable map used many
 * times (OverlayEmb's cached plan, engraft/replica/seq.py:382-444, whose
 * backward runs once per step): _plan groups the slots by variable into the
 * workspace (eg_backward_workspace_size(n_pos*heads, n_var) bytes); _apply
 * sums d_out over each variable's slots from that grouping, in the same order
 * and to the same bits as eg_scatter_grad_slots.  overwrite = 1: grad_out =
 * the sums, zero for a variable no slot hits (no zeroed buffer needed);
 * overwrite = 0: grad_out += the sums.  _apply only reads the grouping, except
 * that a variable of more than 4,096 slots is ordered in place: two _apply
 * calls on one workspace must not overlap. */
int eg_scatter_grad_plan_slots(const int32_t* slot_var, int64_t n_pos, int32_t heads, int64_t n_var,
                               void* workspace, size_t workspace_bytes, void* stream);
int eg_scatter_grad_apply(const void* d_out, int32_t d_out_f32, int64_t n_pos, int32_t heads,
                          int32_t dim, int64_t n_var, float* grad_out, int32_t overwrite,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Seeded synthetic table rows [row0, row0+n_rows) (benchmark/test inputs):
 * value j of row r = qtable[mix64(seed*0xD1B54A32D192ED03 + r*dim + j) >> 50]
 * (qtable f32 [16384], device), quantised with the format's rule
 * (BF16: RNE; Q8_0: d = fp16(amax/127), q = rint(x/d); MXFP8: e4m3 with the
 * smallest shared exponent e that keeps amax*2^-e <= 448). */
int eg_synth_table(const eg_table* table, uint64_t seed, const float* qtable,
                   int64_t row0, int64_t n_rows, void* stream);

/* ---- the PLE block consuming the rows (engraft/replica/layers.py:565-626) --
 * After the projections key = emb @ w_key^T [n_pos, hc*n_embd] and
 * value = emb @ w_value^T [n_pos, n_embd] (library GEMMs), per position and
 * stream j: RMS norms of key_j (norm_key) and hidden_j (norm_query),
 * s = <key_j^, hidden_j^> / sqrt(n_embd), gate = sigmoid(sign(s) sqrt(max(|s|, 1e-6))),
 * gated_j = value * gate, normed_j = rmsnorm(gated_j) * norm_conv.
 * normed f32 [n_pos, hc*n_embd]; s_out, gate_out f32 [n_pos, hc]; rstd_out
 * (optional, f32 [n_pos, hc, 3]) the RMS factors 1/sqrt(mean(x^2) + eps) of
 * key, hidden and gated, which eg_ple_gate_backward takes. */
int eg_ple_gate(const float* key, const float* value, const float* hidden, const float* norm_key,
                const float* norm_query, const float* norm_conv, int64_t n_pos, int32_t hc,
                int32_t n_embd, float eps, float* normed, float* s_out, float* gate_out,
                float* rstd_out, void* stream);

/* out = (hidden + value*gate) + silu(conv), conv[t, c] = sum_k conv_w[c, k] *
 * full[hist_rows + t - (taps-1-k)*dilation, c] over the rows that exist
 * (causal_depthwise_conv, layers.py:257-293); full f32 [hist_rows + n_pos,
 * hc*n_embd] = [history; normed]; conv_w f32 [hc*n_embd, taps], taps <= 8.
 * hidden NULL: out = value*gate + silu(conv) (PleReplica.ple_out,
 * engraft/lens.py:334-341); value (and hidden) NULL: out = silu(conv)
 * (PleReplica.conv_out, lens.py:309-332).  shared_history != 0: every
 * position t is its own one-token continuation of the history, the tap at
 * distance 0 reading row hist_rows + t and the others row hist_rows - distance
 * (PleReplica.ple_out_at, lens.py:341-385).  pre (optional, f32 [n_pos,
 * hc*n_embd]) receives conv before the SiLU, for eg_ple_conv_backward. */
int eg_ple_conv(const float* full, int64_t hist_rows, int64_t n_pos, int32_t hc, int32_t n_embd,
                const float* conv_w, int32_t taps, int32_t dilation, int32_t shared_history,
                const float* hidden, const float* value, const float* gate, float* out, float* pre,
                void* stream);

/* Backward of eg_ple_conv (mode 0, own history): d_full f32 [hist_rows + n_pos,
 * hc*n_embd] = the gradient of [history; normed] given d_out f32 [n_pos,
 * hc*n_embd] (the block's output gradient) and d_tail (optional, f32
 * [tail_rows, hc*n_embd]: the gradient of the last tail_rows rows of full, the
 * history the forward returned).  full and conv_w as the forward's; pre
 * (optional) the forward's pre-activation, read in place of recomputing the
 * convolution.  The convolution weights' gradient is not computed.
 * (taps-1)*dilation <= 32.  Replaces the autograd of causal_depthwise_conv +
 * silu (engraft/replica/layers.py:257-293, 614-626). */
int eg_ple_conv_backward(const float* full, int64_t hist_rows, int64_t n_pos, int32_t hc, int32_t n_embd,
                         const float* conv_w, int32_t taps, int32_t dilation, const float* pre,
                         const float* d_out, const float* d_tail, int64_t tail_rows, float* d_full,
                         void* stream);

/* Backward of eg_ple_gate: from d_out and d_normed (the rows of d_full after
 * the history), the gradients of the projections and of the hidden state:
 * d_key f32 [n_pos, hc*n_embd] (of emb @ w_key^T), d_value f32 [n_pos, n_embd]
 * (of emb @ w_value^T), d_hidden f32 [n_pos, hc*n_embd] (d_out included); any
 * output may be NULL.  detach_value / detach_gate drop that factor of
 * gated = value * gate from the gradient (engraft/replica/layers.py:600-604),
 * leaving d_value / d_key untouched.  s, gate, rstd: the forward's outputs.
 * d_s (NULL: not written) f32 [n_pos, hc] receives the score gradient, which
 * eg_ple_weight_grads takes.  hc <= 4, n_embd <= 4096. */
int eg_ple_gate_backward(const float* key, const float* value, const float* hidden, const float* norm_key,
                         const float* norm_query, const float* norm_conv, const float* s, const float* gate,
                         const float* rstd, const float* d_out, const float* d_normed, int64_t n_pos,
                         int32_t hc, int32_t n_embd, int32_t detach_value, int32_t detach_gate,
                         float* d_key, float* d_value, float* d_hidden, float* d_s, void* stream);

/* eg_ple_gate_backward with d_key and d_value written as their bf16 hi / lo
 * planes (hi = rne(x), lo = rne(x - hi); row strides hc*n_embd and n_embd,
 * the layout of eg_split_bf16's output), ready as eg_gemm_bf16x3 operands:
 * no fp32 gradient is stored and split again.  n_embd a multiple of 256;
 * NULL planes skip that gradient. */
int eg_ple_gate_backward_planes(const float* key, const float* value, const float* hidden,
                                const float* norm_key, const float* norm_query, const float* norm_conv,
                                const float* s, const float* gate, const float* rstd, const float* d_out,
                                const float* d_normed, int64_t n_pos, int32_t hc, int32_t n_embd,
                                int32_t detach_value, int32_t detach_gate, void* d_key_hi, void* d_key_lo,
                                void* d_value_hi, void* d_value_lo, float* d_hidden, float* d_s, void* stream);

/* The weight gradients of the PLE block's norms and convolution (the part of
 * ple_forward's autograd that reaches norm_key, norm_query, norm_conv and
 * conv1d, engraft/replica/layers.py:565-626), from the forward's key, value,
 * hidden, gate, rstd, full and pre-activation, eg_ple_gate_backward's d_s and
 * eg_ple_conv_backward's d_normed (= d_full after the history):
 *   d_norm_key[c], d_norm_query[c], d_norm_conv[c]  f32 [hc*n_embd]
 *   d_conv_w[c, k]                                   f32 [hc*n_embd, taps]
 * each sum over the n_pos positions taken in fixed 64-position chunks added in
 * order (deterministic).  Any output may be NULL.  taps <= 8, n_pos >= 1;
 * workspace of eg_ple_weight_grads_workspace_size bytes. */
size_t eg_ple_weight_grads_workspace_size(int64_t n_pos, int32_t hc, int32_t n_embd, int32_t taps);
int eg_ple_weight_grads(const float* key, const float* value, const float* hidden, const float* gate,
                        const float* rstd, const float* d_s, const float* norm_key,
                        const float* norm_query, const float* d_out, const float* d_normed,
                        const float* full, int64_t hist_rows, const float* pre, int64_t n_pos,
                        int32_t hc, int32_t n_embd, int32_t taps, int32_t dilation,
                        float* d_norm_key, float* d_norm_query, float* d_norm_conv,
                        float* d_conv_w, void* workspace, size_t workspace_bytes, void* stream);

/* Per-stream RMS norm: out[r, j, :] = x[r, j, :] / sqrt(mean(x[r, j, :]^2) + eps)
 * * weight[j, :], x and out f32 [n_rows, hc, n_embd], weight f32 [hc, n_embd]
 * (PleReplica._rmsnorm_per_stream, engraft/lens.py:282-287; the reductions of
 * eg_ple_gate, so applied to value*gate it gives eg_ple_gate's normed bit for
 * bit when both calls' pointers are 16-byte aligned, or both are not). */
int eg_ple_rms(const float* x, int64_t n_rows, int32_t hc, int32_t n_embd, const float* weight, float eps,
               float* out, void* stream);

/* The bf16 hi / lo planes of an fp32 matrix for eg_gemm_bf16x3: x f32
 * [rows, cols] with row stride ld -> hi, lo bf16 [rows, kp], kp = cols
 * rounded up to a multiple of 32, hi = rne(x), lo = rne(x - hi), the padding
 * zero.  No counterpart in the reference (part of its fp32 matmuls). */
int eg_split_bf16(const float* x, int64_t rows, int64_t cols, int64_t ld, void* hi, void* lo, void* stream);

/* One K segment of eg_gemm_bf16x3: the eg_split_bf16 planes of A [m, k]
 * and of B [n, k] for each column group (b2_* only read when n2 > 0). */
typedef struct eg_gemm_operands {
  const void* a_hi;
  const void* a_lo;
  int64_t lda;
  const void* b_hi;
  const void* b_lo;
  int64_t ldb;
  const void* b2_hi;
  const void* b2_lo;
  int64_t ldb2;
  int64_t k; /* multiple of 32 */
} eg_gemm_operands;

/* fp32 GEMM on the bf16 matrix cores over n_seg (1 or 2) K segments and two
 * column groups:
 *   C [m, n]   (+)= sum_s A_s B_s^T     C2 [m, n2] (+)= sum_s A_s B2_s^T
 * every operand given as its eg_split_bf16 planes and hi*hi + hi*lo + lo*hi
 * accumulated in fp32 (hi + lo keeps 16 mantissa bits: a relative error
 * up to ~3 x 2^-18 per product, about 1e-5 of the result on random data; a
 * non-finite operand gives NaN).  Planes 16-byte aligned, leading dimensions
 * multiples of 8, each plane under 4 GiB ((rows - 1) * ld + 32 bf16);
 * accumulate = 1 adds to C / C2.  k_slices = 0 cuts the tiles of a partly
 * filled last round of workgroups along K into ranges that fill it;
 * k_slices >= 1 cuts every 256 x 256 output tile into that many K pieces
 * (1: none).  Pieces' partial products go to a workspace of
 * eg_gemm_workspace_size(m, n, n2, k, k_slices) bytes, k the sum of the
 * segments' k (asked on the device that runs the GEMM: the plan follows its
 * CU count), and are summed in K order afterwards (deterministic).  The
 * projections of ple_forward, key = emb w_key^T and value = emb w_value^T as
 * the two column groups of one call, and their backward d_emb = d_key w_key +
 * d_value w_value as two segments with the weights' transposes as B
 * (engraft/replica/layers.py:594-606, where they are torch fp32 matmuls). */
int64_t eg_gemm_workspace_size(int64_t m, int64_t n, int64_t n2, int64_t k, int32_t k_slices);
int eg_gemm_bf16x3(const eg_gemm_operands* ops, int32_t n_seg, int64_t m, int64_t n, int64_t n2, float* c,
                   int64_t ldc, float* c2, int64_t ldc2, int32_t accumulate, int32_t k_slices,
                   void* workspace, int64_t workspace_bytes, void* stream);

/* The three bf16 planes of an fp32 matrix for eg_gemm_bf16x6: hi = rne(x),
 * mid = rne(x - hi), lo = rne(x - hi - mid) (both differences exact in fp32),
 * each bf16 [rows, kp] as eg_split_bf16's.  hi + mid + lo keeps x's 24
 * mantissa bits.  No counterpart in the reference (part of its fp32 matmuls). */
int eg_split_bf16x6(const float* x, int64_t rows, int64_t cols, int64_t ld, void* hi, void* mid, void* lo,
                    void* stream);

/* eg_gemm_bf16x3's GEMM (segments, column groups, K slices, the workspace of
 * eg_gemm_workspace_size) with every operand split into three planes
 * (eg_split_bf16x6) and six of the nine plane products accumulated in fp32:
 * mid*mid + mid*hi + hi*mid + hi*hi over hi_mid (each segment's planes given
 * as hi in the *_hi and mid in the *_lo fields), then lo*hi + hi*lo over
 * hi_lo (hi in *_hi, lo in *_lo) added to it; the same K segments in both.
 * The dropped products (mid*lo, lo*mid, lo*lo) are below 2^-23 of |a||b|, so
 * the result carries an fp32 matmul's error (the tests hold it to the fp32
 * GEMM's bound against float64).  One K segment: one launch, the hi / lo
 * products continuing the hi / mid products' accumulators, when the
 * workspace also covers eg_gemm_workspace_size(m, n, n2, 2 k, k_slices) (that
 * launch's plan runs 2 k steps); else, and for two K segments, two launches
 * on the stream, the second adding to C / C2.  The same reference products as
 * eg_gemm_bf16x3
 * (engraft/replica/layers.py:594-606, torch fp32 matmuls). */
int eg_gemm_bf16x6(const eg_gemm_operands* hi_mid, const eg_gemm_operands* hi_lo, int32_t n_seg, int64_t m,
                   int64_t n, int64_t n2, float* c, int64_t ldc, float* c2, int64_t ldc2, int32_t accumulate,
                   int32_t k_slices, void* workspace, int64_t workspace_bytes, void* stream);

/* One K segment of eg_gemm_f32: A [m, k] and B [n, k] (and B2 [n2, k] for
 * the second column group, only read when n2 > 0), fp32, row-major. */
typedef struct eg_gemm_f32_operands {
  const float* a;
  int64_t lda;
  const float* b;
  int64_t ldb;
  const float* b2;
  int64_t ldb2;
  int64_t k; /* multiple of 32 */
} eg_gemm_f32_operands;

/* The same GEMM as eg_gemm_bf16x3 (two K segments, two column groups, K
 * slices in the same workspace) in fp32 arithmetic on the fp32 matrix cores
 * (v_mfma_f32_32x32x2_f32): every product exact-rounded as an fp32 matmul's,
 * accumulated in fp32.  Operands 16-byte aligned, leading dimensions
 * multiples of 4, k a multiple of 32.  Its tiles are 256 x 256 (one
 * workgroup a CU), so its pieces and workspace follow
 * eg_gemm_f32_workspace_size; with k_slices 0, a partly filled last round
 * runs as one contiguous range of (tile, K step) units a CU, the parts of a
 * tile summed in K order afterwards.  ple_forward's projections with
 * gemm="fp32", the arithmetic of the reference's torch fp32 matmuls
 * (engraft/replica/layers.py:594-606). */
int64_t eg_gemm_f32_workspace_size(int64_t m, int64_t n, int64_t n2, int64_t k, int32_t k_slices);
int eg_gemm_f32(const eg_gemm_f32_operands* ops, int32_t n_seg, int64_t m, int64_t n, int64_t n2, float* c,
                int64_t ldc, float* c2, int64_t ldc2, int32_t accumulate, int32_t k_slices, void* workspace,
                int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ENGRAFT_NGRAM_H */
