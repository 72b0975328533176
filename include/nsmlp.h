/*
 * nsmlp.h -- C ABI of the MI355X-native blockwise-sparse NF4 MLP decode path.
 *
 * Plain C: device pointers, sizes and an opaque HIP stream (void*).  Every
 * function returns 0 on success or a negative status (NSMLP_E*); the message
 * of the last failure on the calling thread is returned by nsmlp_last_error().
 * No function synchronises the stream, allocates device memory behind the
 * caller's back, or copies its inputs: the caller provides every buffer,
 * including the workspace (sized by the *_workspace_bytes functions and
 * zero-initialised once with nsmlp_workspace_init).  One workspace serves one
 * stream at a time; calls that share a workspace on different streams race.
 *
 * Reference interfaces replaced (paths relative to the reference repository;
 * TSM = llama3_neuroplastic/triton_sparse_mlp.py,
 * RT  = llama3_neuroplastic/experiments/streaming_llama_runtime.py).
 *
 * Layout conventions (the reference's bitsandbytes NF4 format):
 *   an [out, in] weight is flattened row-major; byte e/2 holds elements
 *   (e, e+1) with the even element in the HIGH nibble; one fp32 absmax per
 *   qbs consecutive elements; code[16] maps a nibble to its NF4 value.
 *   Sparse block b of the intermediate dimension is rows [32b, 32b+32) of
 *   gate/up and columns [32b, 32b+32) of down.
 *   "Slot" storage (the HBM hot-block table) is block-major:
 *     gate/up packed [slots][32][H/2] u8,  absmax [slots][32][H/qbs] f32
 *     down    packed [slots][H][16]  u8,   absmax [slots][H] f32
 *   Double-quantised absmax (the bitsandbytes nested quant state, which the
 *   reference resolves to fp32 at RT:4621-4625): u8 codes q, stored in slots
 *   as gate/up [slots][16][H/qbs][2] (rows 2p and 2p+1 interleaved, so one
 *   16-bit read gives a row pair) and down [slots][H]; one fp32 absmax2 per
 *   dq_block consecutive absmax of the full row-major weight, a 256-entry
 *   code2 and an fp32 offset:
 *     absmax = fp32(fp32(code2[q] * absmax2[f / dq_block]) + offset)
 *   where f is the absmax's index in the full weight (gate/up [I][H/qbs],
 *   down [H][I/qbs]); both roundings are kept (no fused multiply-add), so
 *   the result equals the reference's resolved fp32 absmax bit for bit.
 */
#ifndef NSMLP_H
#define NSMLP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NSMLP_OK 0
#define NSMLP_EINVAL (-22)   /* bad shape / argument                    */
#define NSMLP_ENOSPC (-28)   /* workspace too small                     */
#define NSMLP_EHIP (-5)      /* HIP runtime or launch error             */
#define NSMLP_ENODEV (-19)   /* no usable gfx950 device                 */

#define NSMLP_ROUTE_SORTED 1     /* sel in (score desc, index asc) order (torch.topk order) */
#define NSMLP_ROUTE_LEGACY_ABS 2 /* scores = |latent| . score_w, no bias, no clamp (RT:4332-4334) */

#define NSMLP_DOWN_BLOCK_MAJOR 0 /* down blocks as [n][H][16], absmax [n][H]          */
#define NSMLP_DOWN_GATHERED 1    /* down blocks as [H][n][16], absmax [H][n] (RT:4491) */

/* Message of the last failing call on this thread ("" if none). */
const char* nsmlp_last_error(void);

/* ABI version (major*100 + minor). */
int nsmlp_version(void);

/* 1 if device `device` is a gfx950 GPU usable by this library, else 0. */
int nsmlp_device_supported(int device);

/* Fault injection for tests of a caller's failure handling: the reference
 * runtime's failure counter for its single-kernel decode (off after three
 * failures, RT:5626-5637), its fallback on any v1 exception (RT:5681-5685)
 * and its out-of-memory test by message (runtime/_helpers.py:301-308).
 * spec = "name=kind[:count],..." arms the named compute entry points (name
 * without the nsmlp_ prefix, or * for all of them) to fail before they touch
 * the device: kind oom (NSMLP_EHIP, the message says "out of memory"), hip
 * (NSMLP_EHIP), inval, nospc or nodev (NSMLP_EINVAL / _ENOSPC / _ENODEV);
 * count = how many calls fail (default every call).  NULL or "" disarms.
 * The environment variable NSMLP_FAULT_INJECT sets the same at load time.
 * Process-wide; returns NSMLP_EINVAL for a bad spec (the rules stay as they
 * were). */
int nsmlp_fault_inject(const char* spec);

/* Zero the counter region of a workspace; call once after allocating it.
 * The first int32 of a workspace is a status word, set by the kernels and
 * kept until the caller clears it:
 *   NSMLP_STATUS_BLOCK_UNAVAILABLE: a selected block id was out of range, or
 *     not resident with no host copy (such a block contributed zero; the
 *     reference's gather raises there, RT:4530-4578);
 *   NSMLP_STATUS_FIXED_RANGE: a grouped prefill down partial was outside the
 *     fixed-point range (|v| >= 2^23, inf or nan); those outputs are wrong. */
#define NSMLP_STATUS_BLOCK_UNAVAILABLE 1
#define NSMLP_STATUS_FIXED_RANGE 2
int nsmlp_workspace_init(void* ws, size_t ws_bytes, void* stream);

/* Status hand-over (version >= 103): ORs the status word of `ws` into *dst
 * (device memory, or pinned host memory through its device pointer, see
 * nsmlp_host_device_pointer; the caller zeroes it once) and clears the word,
 * in stream order, in one kernel (no memset: it may be captured in a graph).
 * The caller reads *dst once the stream has passed that point (an event), so
 * the launches in between are not stalled.  dst == NULL (version >= 104):
 * the word is only cleared (e.g. before a call whose status is checked). */
int nsmlp_workspace_take_status(void* ws, int32_t* dst, void* stream);

/* Block-source counts (version >= 104).  The decode kernels count the
 * selected blocks of every call that they read from HBM slots and from host
 * copies into two counters of the workspace's counter region, kept until
 * taken like the status word.  This takes them: dst[0] += blocks read from
 * HBM slots, dst[1] += blocks read from host copies (int64, device memory or
 * pinned host memory through its device pointer, 8-byte aligned), and the
 * counters are cleared, in stream order, in one kernel.  Replaces the
 * runtime status counters of RT:1694-1779 (incremented at RT:3926, 3934,
 * 5263, 5279, 5328; the reference counts its decode_mlp_* entries once per
 * gate and once per up projection, its decode_down_* entries once per
 * block).  Decode calls only (the reference counts in the decode phase). */
int nsmlp_workspace_take_block_counts(void* ws, int64_t* dst, void* stream);

/* ------------------------------------------------------------------ router
 * Replaces RT:4311-4352 (_route_sparse_mlp) together with RT:4209-4238
 * (_compute_sparse_basis_latent), for `rows` tokens:
 *   latent = fp16(x . enc_w[r] + enc_b[r]); if basis_top_k < R keep the
 *   basis_top_k largest |latent| (ties: lowest index), zero the rest;
 *   score  = max(fp16(latent . score_w[j] + score_b[j]), 0)
 *            (NSMLP_ROUTE_LEGACY_ABS: fp16(|latent| . score_w[j]));
 *   if down_block_norm: score = fp16(score * down_block_norm[j]);
 *   sel[t] = the k largest scores, ties broken by the lowest block index,
 *   in ascending block order (the order of the reference's ordered_blocks,
 *   RT:4873) or, with NSMLP_ROUTE_SORTED, in (score desc, index asc) order.
 * Every dot product is computed exactly and rounded once to fp16 (RNE), so
 * the selection does not depend on summation order.
 * x [rows][H], enc_w [R][H], enc_b [R] (nullable), score_w [NB][R],
 * score_b [NB] (nullable), down_block_norm [NB] fp16 (nullable): fp16.
 * latent_out [rows][R] / scores_out [rows][NB] fp16, nullable.
 * Limits: H <= 65535, R <= 1024, NB <= 65535, 1 <= k <= NB.
 */
size_t nsmlp_route_workspace_bytes(int rows, int H, int R, int NB, int k);
int nsmlp_route_f16(const void* x, int rows, int H, const void* enc_w, const void* enc_b, int R, int basis_top_k,
                    const void* score_w, const void* score_b, const void* down_block_norm, int NB, int flags, int k,
                    int32_t* sel, void* latent_out, void* scores_out, void* ws, size_t ws_bytes, void* stream);

/* ------------------------------------------------- fused decode (M = 1)
 * One token through the blockwise-sparse MLP over the selected blocks:
 *   y = sum_{b in sel} Wd[:, b] (silu(Wg_b x) * (Wu_b x))   (fp32 inside, one fp16 rounding)
 * Replaces the gather + dispatch of RT:5104-5524 (_sparse_mlp_forward_fast)
 * for a decode token: block b is read from its HBM slot lookup[b] when
 * lookup[b] >= 0 and from the host-resident copy (block-major, indexed by b)
 * otherwise, with no host round trip (RT:4867) and no gathered copy
 * (RT:3644-3702).
 */
typedef struct nsmlp_slot_table {
  int H;            /* hidden size (gate/up in, down out)              */
  int I;            /* intermediate size (NB * 32)                     */
  int qbs;          /* NF4 quant block size (multiple of 32, divides H) */
  int n_slots;      /* HBM slots                                        */
  const int32_t* lookup;             /* [NB] slot of block b, -1 = not resident; NULL = identity */
  const uint8_t* gate_packed;        /* [n_slots][32][H/2] */
  const float* gate_absmax;          /* [n_slots][32][H/qbs] */
  const uint8_t* up_packed;
  const float* up_absmax;
  const uint8_t* down_packed;        /* [n_slots][H][16] */
  const float* down_absmax;          /* [n_slots][H] */
  /* Host-resident copy of every block (pinned, device-accessible pointers),
   * same block-major layout indexed by block id; NULL when all selected
   * blocks are resident. */
  const uint8_t* host_gate_packed;
  const float* host_gate_absmax;
  const uint8_t* host_up_packed;
  const float* host_up_absmax;
  const uint8_t* host_down_packed;
  const float* host_down_absmax;
  const float* code;                 /* [16] NF4 code book (device) */
  const void* down_bias;             /* [H] fp16 or NULL */
  /* Double-quantised absmax (version >= 101).  dq_block == 0: the fp32
   * *_absmax above are read.  dq_block > 0 (a power of two; bitsandbytes
   * uses 256): the fp32 *_absmax are ignored and the u8 codes below are
   * read instead. */
  int dq_block;
  const uint8_t* gate_qabsmax;       /* [n_slots][16][H/qbs][2] u8 (row pairs interleaved) */
  const uint8_t* up_qabsmax;
  const uint8_t* down_qabsmax;       /* [n_slots][H] u8 */
  const uint8_t* host_gate_qabsmax;  /* host copies (with the host packed copies) */
  const uint8_t* host_up_qabsmax;
  const uint8_t* host_down_qabsmax;
  const float* gate_absmax2;         /* [ceil(I*H/qbs / dq_block)] f32 (device) */
  const float* up_absmax2;
  const float* down_absmax2;         /* [ceil(H*I/qbs / dq_block)] f32 (device) */
  const float* gate_code2;           /* [256] f32 second-level code book (device) */
  const float* up_code2;
  const float* down_code2;
  float gate_offset;
  float up_offset;
  float down_offset;
} nsmlp_slot_table;

size_t nsmlp_decode_workspace_bytes(int H, int k);
int nsmlp_decode_slots_f16(const nsmlp_slot_table* table, const void* x, const int32_t* sel, int k, void* out,
                           void* ws, size_t ws_bytes, void* stream);
/* The same with the decode loop's residual add fused into the output
 * (version >= 104; RT:7774): out[o] = fp16(residual[o] + fp16(mlp(x)[o])),
 * as nsmlp_decode_layer_add_f16 does it, for callers that route first (e.g.
 * to promote the selected blocks into HBM slots before the decode reads
 * them, so a missed block crosses the host link once: RT:4094-4131). */
int nsmlp_decode_slots_add_f16(const nsmlp_slot_table* table, const void* x, const void* residual,
                               const int32_t* sel, int k, void* out, void* ws, size_t ws_bytes, void* stream);

/* Router + fused decode for one decode token (the decode branch of
 * RT:5833-5923 _mlp_forward_dispatch: route, then sparse MLP), entirely on
 * the device.  sel_out [k] receives the selected blocks in ascending order. */
typedef struct nsmlp_router {
  int R;
  int basis_top_k;
  int NB;
  int flags;                 /* NSMLP_ROUTE_LEGACY_ABS or 0 */
  const void* enc_w;         /* [R][H] fp16 */
  const void* enc_b;         /* [R] fp16 or NULL */
  const void* score_w;       /* [NB][R] fp16 */
  const void* score_b;       /* [NB] fp16 or NULL */
  const void* down_block_norm; /* [NB] fp16 or NULL */
} nsmlp_router;

size_t nsmlp_layer_workspace_bytes(int H, int R, int NB, int k);
int nsmlp_decode_layer_f16(const nsmlp_router* router, const nsmlp_slot_table* table, const void* x, int k,
                           int32_t* sel_out, void* out, void* ws, size_t ws_bytes, void* stream);

/* The same layer call with the decode loop's residual add fused into the
 * output (version >= 102; RT:7774, hidden = residual + mlp_out):
 * out[o] = fp16(residual[o] + fp16(mlp(x)[o])), the fp16 add torch does.
 * residual [H] fp16; out may alias residual or x (in-place hidden update). */
int nsmlp_decode_layer_add_f16(const nsmlp_router* router, const nsmlp_slot_table* table, const void* x,
                               const void* residual, int k, int32_t* sel_out, void* out, void* ws, size_t ws_bytes,
                               void* stream);

/* No-allocation variant of nsmlp_decode_layer_f16 / _add_f16 (version >= 103).
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, hosts that
 * forbid hipMalloc).  It takes no workspace: its scratch is a file-scope
 * device array of the library, 256 KiB per device (each GPU holds its own
 * copy until the process ends), whose address is looked up once per device;
 * it calls no hipMalloc, hipFree or allocating library routine.  Same
 * kernels and results as nsmlp_decode_layer_f16 (with residual != NULL, as
 * nsmlp_decode_layer_add_f16), for the streaming shapes: hidden size a
 * multiple of 2048 up to 16384, num_blocks <= 4096, k <= 2048, and a scratch
 * need of at most 256 KiB (k up to about 1800); other shapes fail with
 * NSMLP_EINVAL and a message.  The scratch's status word and block counts
 * are cleared at the start of every call (by its first kernel), so they hold
 * that call's alone.  status_out (nullable, device or pinned host memory,
 * zeroed once by the caller): the call's status word is ORed into it (see
 * nsmlp_workspace_take_status).  Every
 * call on a device shares that device's scratch, which keeps the last call's
 * contents: calls that overlap on one GPU (other streams, other threads)
 * race. */
int nsmlp_decode_layer_noalloc_f16(const nsmlp_router* router, const nsmlp_slot_table* table, const void* x,
                                   const void* residual, int k, int32_t* sel_out, void* out, int32_t* status_out,
                                   void* stream);

/* --------------------------------------- reference-signature entry points
 * Replaces TSM:1378-1509 (triton_sparse_mlp_decode_4bit_single_kernel_sm75):
 * x [H] fp16; gathered gate/up packed [top_k][32][H/2] u8 with absmax
 * [top_k][32][H/qbs] f32; down packed [H][top_k][16] u8 with absmax
 * [H][top_k] f32; code tables [16] f32 (one per projection); out [H] fp16.
 * out_accum [>= H] f32 receives the fp32 result before rounding (the
 * reference's scratch, TSM:1476-1508).  block_size must be 32.
 */
/* Chunked prefill over a slot table: M tokens, each with its own k selected
 * blocks (the multi-token decode branch, RT:4857-4908 + RT:5104-5524 with the
 * per-row mask of RT:5453: a token's gate/up are masked to its own blocks):
 *   out[t] = sum over b in sel[t] of Wd_b (silu(Wg_b x_t) * (Wu_b x_t))
 * x [M][H] fp16 (16-byte aligned), sel [M][k] int32 block ids (e.g. from
 * nsmlp_route_f16 with rows = M; an id repeated in a row counts once), out
 * [M][H] fp16.  Grouped per block on MFMA: fp16 operands (gate/up weights as
 * fp16(code * absmax), as the reference's dequant fallback rounds them,
 * RT:5439-5447; down weights as fp16 codes with the absmax applied to each
 * block's product in fp32), fp32 accumulation, act rounded to fp16 (RT:5459),
 * the down sums accumulated in fixed point (independent of scheduling).
 * M <= 65536 and M*H*2, M*k*64 < 2^31.  The workspace grows with M: when
 * the tokens' blocks cover most of the layer (M k >= 2 NB) the down runs as
 * the dense GEMM over an act matrix [M][I] fp16 with S fp32 partials [M][H]
 * (at the 405B shape about 0.36 MB per token, 2.9 GB at 8192 tokens): run
 * long prompts in chunks (the reference's prefill is chunked too). */
size_t nsmlp_prefill_workspace_bytes(int H, int NB, int M, int k);
int nsmlp_prefill_slots_f16(const nsmlp_slot_table* table, const void* x, int M, const int32_t* sel, int k, void* out,
                            void* ws, size_t ws_bytes, void* stream);

/* Dense-guard prefill MLP (version >= 102): replaces RT:5775-5831
 * (_dense_guard_mlp_forward_exact_chunked_4bit), every intermediate block for
 * every token, with the reference's rounding points: weights fp16(code *
 * absmax), g = fp16(x Wg^T), act = fp16(fp16(silu(g)) * fp16(x Wu^T)),
 * out = fp16(act Wd^T + down_bias) (+ residual: fp16(residual + out)).
 * x [M][H] fp16 (16-byte aligned), residual [M][H] fp16 or NULL, out [M][H]
 * fp16.  H % 256 == 0, I % 128 == 0; blocks read from their HBM slots or
 * host copies.  Deterministic.  The tokens run in chunks of at most 1024
 * (version >= 104; each token's result is that of one call over all tokens),
 * so the workspace is bounded by the 1024-token size (at the 405B shape
 * about 0.37 GB). */
size_t nsmlp_dense_mlp_workspace_bytes(int H, int I, int M);
int nsmlp_dense_mlp_slots_f16(const nsmlp_slot_table* table, const void* x, int M, const void* residual, void* out,
                              void* ws, size_t ws_bytes, void* stream);

/* ------------------------------------------------ hot-block cache (device)
 * Promotion of missed blocks into the table's fixed-capacity slots, as
 * stream-ordered kernels with no host round trip.  Replaces the host-side
 * promotion of RT:2809-3018 (the down bank's fixed-capacity update, applied
 * here to whole blocks: gate/up rows and down columns share a slot) with the
 * slot plan of RT:2576-2617: the novel entries of blocks (valid ids not
 * resident, first occurrence, in order; at most `capacity`) take the free
 * slots from active_count on, then the slots of lowest score (ties: lowest
 * slot); a promoted block scores fp32(base + (i + 1) * 1e-3), base = max
 * active score + 1 (fp64), i its novel index; active_count grows by the free
 * slots used.  With NSMLP_CACHE_GROW_ONLY only free slots are used (the gate/up
 * hot cache, which only grows).  The lookup entries of evicted blocks become
 * -1.  The promoted blocks are copied from the table's host copies into the
 * table's slots (written in place), after the work already queued on the
 * stream.  slot_out (nullable): [n] slot given to each entry, -1 otherwise. */
typedef struct nsmlp_cache_state {
  int capacity;           /* slots: the table's n_slots (<= 8192) */
  int32_t* lookup;        /* [NB] the table's lookup, updated in place */
  int32_t* slot_block;    /* [capacity] block held by each slot, -1 = none */
  float* slot_score;      /* [capacity] replacement scores */
  int32_t* active_count;  /* [1] slots in use (device) */
} nsmlp_cache_state;
#define NSMLP_CACHE_GROW_ONLY 1
size_t nsmlp_cache_workspace_bytes(int n);  /* starts with the counter region, as every workspace */
int nsmlp_cache_promote(const nsmlp_slot_table* table, const nsmlp_cache_state* cache, const int32_t* blocks, int n,
                        int flags, int32_t* slot_out, void* ws, size_t ws_bytes, void* stream);
/* Calibration hit counts (replaces RT:2205-2243 without the host copy):
 * counts[b] += row_weights[r] (1 when NULL) for every entry b of row r of
 * blocks [rows][k] with 0 <= b < NB, added in row order and entry order as
 * a row-by-row index_add_ adds them.  The reference's recency weights are
 * ((r + 1) / rows) ** power in fp32. */
int nsmlp_cache_record_f32(float* counts, int NB, const int32_t* blocks, int rows, int k, const float* row_weights,
                           void* stream);

size_t nsmlp_single_kernel_workspace_bytes(int H, int top_k);
int nsmlp_single_kernel_decode_f16(const void* x, const uint8_t* gate_packed, const float* gate_absmax,
                                   const float* gate_code, const uint8_t* up_packed, const float* up_absmax,
                                   const float* up_code, const uint8_t* down_packed, const float* down_absmax,
                                   const float* down_code, void* out, float* out_accum, int H, int block_size,
                                   int qbs, int top_k, void* ws, size_t ws_bytes, void* stream);

/* Replaces TSM:1519-1585 (triton_fused_sparse_mlp_decode_4bit) for one row,
 * as RT:5651-5675 calls it: the two gate/up output linears, silu * up and the
 * down input linear fused into the two decode kernels (fp32 inside, one fp16
 * rounding).  x [H] fp16; active_idx [kk] int32 slots in 0..A-1 (< 0 are
 * skipped; a slot listed twice is counted twice by the down projection, as
 * in the reference's input linear); flat_mask [A*32] fp16 (nullable = 1);
 * gate/up packed [A*32][H] NF4 (absmax per qbs elements) with biases [A*32]
 * fp16 (nullable); down packed [H][A*32] NF4 with quant block 32 (absmax
 * [H][A]) and down_bias [H] fp16 (nullable); out [H] fp16.
 */
size_t nsmlp_fused_decode_workspace_bytes(int H, int kk);
int nsmlp_fused_decode_gathered_f16(const void* x, int H, const int32_t* active_idx, int kk, int A,
                                    const void* flat_mask, const uint8_t* gate_packed, const float* gate_absmax,
                                    const float* gate_code, const void* gate_bias, const uint8_t* up_packed,
                                    const float* up_absmax, const float* up_code, const void* up_bias,
                                    const uint8_t* down_packed, const float* down_absmax, const float* down_code,
                                    const void* down_bias, int qbs, void* out, void* ws, size_t ws_bytes,
                                    void* stream);

/* Replaces TSM:1340-1375 (triton_sparse_output_linear_4bit) with row-major
 * NF4 semantics (the reference's Triton kernel indexes a transposed payload,
 * TSM:634-635; this computes what its callers pass, RT:4630-4660):
 *   out[t][s*32 + j] = (sum_c W[s*32 + j][c] x[t][c] + bias[s*32 + j]) * flat_mask[t][s*32 + j]
 * for every slot s listed in active_idx[t] (entries < 0 are skipped), and
 * 0 elsewhere.  W [A*32][in_dim] NF4 (absmax per qbs elements), x [rows][in_dim],
 * flat_mask [rows][A*32] fp16 (nullable = 1), bias [A*32] fp16 (nullable),
 * active_idx [rows][kk] int32, out [rows][A*32] fp16.
 */
size_t nsmlp_output_linear_workspace_bytes(int rows, int kk, int in_dim);
int nsmlp_output_linear_nf4_f16(const void* x, int rows, int in_dim, const int32_t* active_idx, int kk, int A,
                                const void* flat_mask, const uint8_t* packed, const float* absmax, const float* code,
                                int qbs, const void* bias, int block_size, void* out, void* ws, size_t ws_bytes,
                                void* stream);

/* Replaces TSM:1303-1337 (triton_sparse_input_linear_4bit) with row-major
 * NF4 semantics (RT:5651-5675 passes the gathered down weight [H][A*32] with
 * quant block 32, i.e. absmax [H][A]; runtime/lm_head.py:461-473 passes the
 * LM head with blocks of 256 columns, all active):
 *   out[t][o] = sum_{s in active_idx[t]} sum_{j < B} W[o][s*B + j] x[t][s*B + j] + bias[o]
 * B = block_size, a multiple of 32; entries < 0 or past in_features skipped.
 * W [out_features][in_features] NF4 (absmax per qbs elements),
 * x [rows][in_features], out [rows][out_features] fp16.
 */
int nsmlp_input_linear_nf4_f16(const void* x, int rows, int in_features, const int32_t* active_idx, int kk,
                               const uint8_t* packed, const float* absmax, const float* code, int qbs,
                               int out_features, const void* bias, int block_size, void* out, void* stream);

/* Dense NF4 matrix (no bias, version >= 102): the LM head the reference keeps on the GPU
 * (runtime/lm_head.py:267-350 materialises it, bitsandbytes' flat layout:
 * packed [out][in/2], high nibble first, absmax over qbs consecutive
 * elements of the flat row-major weight).  dq_block > 0 (power of two):
 * absmax is double-quantised, absmax = code2[qabsmax[i]] * absmax2[i /
 * dq_block] + offset (two fp32 roundings), and the fp32 absmax is ignored. */
typedef struct nsmlp_nf4_matrix {
  int out_features;
  int in_features;       /* multiple of 32, <= 16384 */
  int qbs;               /* power of two >= 32 dividing in_features */
  const uint8_t* packed; /* [out][in/2], 16-byte aligned */
  const float* absmax;   /* [out*in/qbs] f32 (dq_block == 0) */
  const float* code;     /* [16] NF4 code book (device) */
  int dq_block;
  const uint8_t* qabsmax; /* [out*in/qbs] u8 */
  const float* absmax2;   /* [ceil(out*in/qbs / dq_block)] f32 */
  const float* code2;     /* [256] f32 */
  float offset;
} nsmlp_nf4_matrix;

/* Replaces runtime/lm_head.py:450-474 (_lm_head_forward: the NF4 LM head
 * through triton_sparse_input_linear_4bit with every input block active):
 *   out[t][o] = sum_c W[o][c] x[t][c],  t < rows
 * x [rows][in] fp16 (16-byte aligned), out [rows][out] fp16, out_f32
 * [rows][out] (nullable) the same sums before the fp16 rounding.  One pass
 * over the weight per two rows.  in_features > 16384: use
 * nsmlp_input_linear_nf4_f16 with every block active. */
int nsmlp_dense_linear_nf4_f16(const nsmlp_nf4_matrix* w, const void* x, int rows, void* out, float* out_f32,
                               void* stream);

/* silu(gate) * up elementwise in fp32, rounded to fp16 (TSM:1577-1578). */
int nsmlp_silu_mul_f16(const void* gate, const void* up, void* out, long long n, void* stream);

/* ----------------------------------------------------- slot-table helpers
 * Row-block gather (gate/up): dst block i = src block blocks[i], i.e. the
 * byte range [b*32*in/2, (b+1)*32*in/2) and absmax range [b*32*in/qbs, ...)
 * of the row-major weight (RT:4530-4578, RT:2722-2786).  src_blocks is the
 * number of blocks in the source; ids outside [0, src_blocks) leave their
 * destination block untouched (likewise ids >= in/32 for the down gather).
 */
int nsmlp_gather_row_blocks(const uint8_t* src_packed, const float* src_absmax, int src_blocks,
                            const int32_t* blocks, int n, int in_features, int qbs, uint8_t* dst_packed,
                            float* dst_absmax, void* stream);

/* Down-proj column gather (RT:4455-4528 _load_down_proj_cold_cols,
 * RT:2619-2720): for block b, bytes src[o][16b .. 16b+16) and absmax
 * src_absmax[o][(32b)/qbs] of the row-major [out][in] weight, written
 * block-major ([n][out][16], [n][out]) or gathered ([out][n][16], [out][n]). */
int nsmlp_gather_down_columns(const uint8_t* src_packed, const float* src_absmax, const int32_t* blocks, int n,
                              int out_features, int in_features, int qbs, int dst_layout, uint8_t* dst_packed,
                              float* dst_absmax, void* stream);

/* The same two gathers for double-quantised absmax: the u8 codes of a row
 * block are written in the slot layout [n][16][in/qbs][2] (rows 2p, 2p+1
 * interleaved); the down codes as [n][out] (or [out][n]).  src_packed and
 * dst_packed may both be NULL to gather the codes only.  Replace the same
 * reference code, with the nested state kept instead of resolved
 * (RT:4621-4625). */
int nsmlp_gather_row_blocks_q8(const uint8_t* src_packed, const uint8_t* src_qabsmax, int src_blocks,
                               const int32_t* blocks, int n, int in_features, int qbs, uint8_t* dst_packed,
                               uint8_t* dst_qabsmax, void* stream);
int nsmlp_gather_down_columns_q8(const uint8_t* src_packed, const uint8_t* src_qabsmax, const int32_t* blocks, int n,
                                 int out_features, int in_features, int qbs, int dst_layout, uint8_t* dst_packed,
                                 uint8_t* dst_qabsmax, void* stream);

/* Double quantisation of an fp32 absmax vector (bitsandbytes
 * compress_statistics, restated; the reference reads the result back with
 * dequantize_blockwise + offset at RT:4621-4625 and safetensor_loader.py:
 * 403-406): a = absmax - offset; per dq_block consecutive entries absmax2 =
 * max |a|, q = index of the code2 entry nearest to a * fp32(1 / absmax2)
 * (ties: the lower index; code2 ascending, 256 entries).  The caller gives
 * the offset (bitsandbytes: the mean of absmax). */
int nsmlp_absmax_dq_quantize(const float* absmax, long long n, int dq_block, const float* code2, float offset,
                             uint8_t* q, float* absmax2, void* stream);
/* Its inverse, as the runtime resolves it (RT:4621-4625):
 * out[i] = fp32(fp32(code2[q[i]] * absmax2[i / dq_block]) + offset). */
int nsmlp_absmax_dq_dequantize(const uint8_t* q, long long n, int dq_block, const float* code2, const float* absmax2,
                               float offset, float* out, void* stream);

/* Device-side address of pinned host memory (hipHostMalloc'd, e.g. a torch
 * pinned tensor) for the slot table's host_* pointers: misses are read by the
 * kernels directly over the host link (the reference stages them through
 * pinned buffers and H2D copies, RT:3437-3493, safetensor_loader.py:172-201). */
int nsmlp_host_device_pointer(const void* host, void** device_ptr);

/* -------------------------------------------------------- synthetic data
 * Seeded synthetic weights for benchmarks (counter-based; the value of
 * element i depends only on (seed, i)):
 *   nsmlp_synth_normal_f16: out[i] = fp16(std * N(0,1)).
 *   nsmlp_synth_nf4:        w[i] = std * N(0,1) quantised to NF4 (absmax per qbs).
 *   nsmlp_nf4_quantize_f32: NF4 quantisation of given fp32 values (the
 *   restated bitsandbytes nf4 algorithm: nearest code by midpoint thresholds,
 *   even element in the high nibble; an all-zero block stores code 7).
 */
int nsmlp_synth_normal_f16(uint64_t seed, long long n, float std, void* out, void* stream);
int nsmlp_synth_nf4(uint64_t seed, long long n, int qbs, float std, uint8_t* packed, float* absmax, void* stream);
int nsmlp_nf4_quantize_f32(const float* w, long long n, int qbs, uint8_t* packed, float* absmax, void* stream);
int nsmlp_synth_normal_f32(uint64_t seed, long long n, float std, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NSMLP_H */
