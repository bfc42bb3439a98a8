/*
 * qmoe_capi.h -- C ABI of libqmoe.so, the MI355X (gfx950) kernels for the
 * Qwen3-30B-A3B decoder-layer hot path: residual RMSNorm, router top-k,
 * expert dispatch (histogram / scan / permute), the grouped SwiGLU expert
 * GEMM (MFMA, prefill) and GEMV (decode), the weighted combine, the QKV
 * projection with per-head RMSNorm + RoPE epilogue, and causal GQA attention
 * over a contiguous KV cache.
 *
 * Conventions shared by every entry point
 *   - All tensor arguments are caller-owned device pointers; outputs and
 *     workspaces are allocated by the caller.  No entry point allocates,
 *     frees or synchronises the host.
 *   - An empty batch (T, rows, M, n or B * S of zero) is valid: the call
 *     launches nothing and returns 0, and the buffers sized by that count
 *     may be NULL.  Weights, caches and norm weights are still required.
 *     qmoe_moe_permute / qmoe_moe_route still write the dispatch metadata
 *     for zero pairs (all counts 0, no tiles).
 *   - bf16 values are passed as qmoe_bf16 (the raw 16-bit pattern).
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream),
 *     so every call can be captured into a HIP graph.
 *   - Return 0 on success; QMOE_ERR_INVALID when an argument is rejected
 *     before anything is launched; QMOE_ERR_HIP when the HIP runtime reports
 *     an error.  qmoe_last_error() then describes the failure (thread-local).
 *
 * Each declaration names the reference interface (charleshong3/nki-moe-7013)
 * whose behaviour it replaces.
 */
#ifndef QMOE_CAPI_H
#define QMOE_CAPI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t qmoe_bf16;
typedef void* qmoe_stream_t;

#define QMOE_OK 0
#define QMOE_ERR_INVALID 1
#define QMOE_ERR_HIP 2

/* GEMM epilogue modes for qmoe_gemm. */
#define QMOE_GEMM_STORE_BF16 0 /* C[bf16] = A.B^T            */
#define QMOE_GEMM_STORE_F32 1  /* C[f32]  = A.B^T            */
#define QMOE_GEMM_ADD_F32 2    /* C[f32] += A.B^T (residual) */

/* Packing granularity of the fused gate/up weight: packed rows
 * [64j, 64j+32) are gate rows [32j, 32j+32), the next 32 the matching up rows. */
#define QMOE_W13_GROUP 32

/* Blocked layout of the down weight: w2 is bf16 [E][I/8][H][8], element
 * (e, ib, h, ii) = W2[e][h][8*ib + ii] (W2[e] = the [H, I] down matrix).  An
 * 8-unit slice of one expert's down matrix is one contiguous H x 16-byte run. */
#define QMOE_W2_BLOCK 8

/* Largest row tile (tile_m of qmoe_moe_permute) qmoe_moe_experts_grouped takes. */
#define QMOE_GROUPED_MAX_TILE_M 256

/* Length of the dispatch `meta` array (i32): (n_tiles, n_active, error, -),
 * then the work counters of qmoe_moe_experts_grouped. */
#define QMOE_META_INTS 24

/* Workgroups of the decode block's expert kernel (one per MI355X CU); sets
 * the size of its partial-output workspace. */
#define QMOE_DECODE_BLOCK_WGS 256

/* Largest T * H qmoe_moe_decode_block_noalloc accepts (its static scratch is
 * QMOE_DECODE_BLOCK_STATE_BYTES + QMOE_DECODE_BLOCK_WGS * this many floats,
 * 16.25 MiB per GPU). */
#define QMOE_DECODE_BLOCK_NOALLOC_MAX_TH 16384

/* Bytes at the start of a decode-block workspace that carry state from one
 * call to the next (the single-launch T = 1 path's call counters and
 * exchange slots); the per-workgroup partials follow them.  The status word
 * (u32) of that state sits at QMOE_DECODE_BLOCK_STATUS_OFFSET. */
#define QMOE_DECODE_BLOCK_STATE_BYTES 262144
#define QMOE_DECODE_BLOCK_STATUS_OFFSET 1024

/* ABI version qmoe_version() returns.  2: the dispatch meta array holds
 * QMOE_META_INTS ints (was 4), and decode-block workspaces start with
 * QMOE_DECODE_BLOCK_STATE_BYTES of call-to-call state (zeroed before first use).
 * 3: qmoe_moe_experts_grouped takes the tile table non-const (word 3 of each
 * live row counts finished gate_up panels during the call), and
 * qmoe_attn_prefill_ws / qmoe_attn_prefill_workspace are new. */
#define QMOE_VERSION 3

int qmoe_version(void);
const char* qmoe_last_error(void);

/* Residual RMSNorm.  h = x (+ delta); y = bf16(w * h * rsqrt(mean(h^2) + eps)).
 *   x, delta, h_out: f32 [rows, H] (delta and h_out may be NULL; h_out may alias x)
 *   w: bf16 [H]; y_out: bf16 [rows, H]
 * Replaces: the decoder layer's input/post-attention RMSNorm and residual add,
 *   NeuronQwen3MoeDecoderLayer.forward qwen_with_nki.py:10179-10207 with
 *   CustomRMSNorm (fp32 upcast -> normalise -> x weight -> cast) restated at
 *   qwen_with_nki.py:1372-1384; _nki_rmsnorm_kernel 1286-1342. */
int qmoe_rmsnorm_residual(const float* x, const float* delta, const qmoe_bf16* w,
                          int64_t rows, int64_t H, float eps, float* h_out,
                          qmoe_bf16* y_out, qmoe_stream_t stream);

/* Router: logits = x . w_router^T (+ bias) in fp32; softmax over E; top-k;
 * renormalise the k weights to sum 1.  Ties pick the lower expert index.
 *   x: bf16 [T, H]; w_router: bf16 [E, H]; bias: f32 [E] or NULL
 *   topk_idx: i32 [T, k] (descending weight); topk_w: f32 [T, k];
 *   logits: f32 [T, E] (required).  Limits: E <= 256, k <= 16, H % 8 == 0.
 * Replaces: NxDI RouterTopK invoked as mlp.router(normed_hidden)
 *   qwen_with_nki.py:8589-8590 with router dtype fp32 / softmax 9886-9888 and
 *   normalize_top_k_affinities 9894, 2399-2405. */
int qmoe_router_topk(const qmoe_bf16* x, const qmoe_bf16* w_router, const float* bias,
                     int64_t T, int64_t H, int64_t E, int64_t k, int32_t* topk_idx,
                     float* topk_w, float* logits, qmoe_stream_t stream);

/* qmoe_router_topk with a caller-owned workspace of workspace_bytes (at least
 * qmoe_router_workspace(T, H, E) to be used): for T > 16 the logits GEMM then
 * runs split-K (its E = 128 columns give few tiles over the long K = H), the
 * slices summed in a fixed order by the top-k launch, so results repeat
 * bit for bit (they may differ from the unsplit call in the last bits of the
 * logits).  A NULL or smaller workspace: the unsplit path.  Same limits.
 * Replaces: the router of qmoe_router_topk (qwen_with_nki.py:8589-8590,
 *   9886-9888, 9894, 2399-2405). */
int qmoe_router_topk_ws(const qmoe_bf16* x, const qmoe_bf16* w_router, const float* bias,
                        int64_t T, int64_t H, int64_t E, int64_t k, int32_t* topk_idx,
                        float* topk_w, float* logits, void* workspace, int64_t workspace_bytes,
                        qmoe_stream_t stream);

/* Workspace bytes qmoe_router_topk_ws / qmoe_moe_route_ws use for T tokens
 * (0: that size never splits; -1 for bad sizes).
 * Replaces: nothing in the reference (a sizing helper of this library). */
int64_t qmoe_router_workspace(int64_t T, int64_t H, int64_t E);

/* Expert dispatch metadata (histogram, exclusive scan, stable permutation).
 *   topk_idx: i32 [T, k]
 *   counts: i32 [E]; offsets: i32 [E+1]; slot_token: i32 [T*k] (token of each
 *   expert-sorted slot, stable by token); token_slot: i32 [T*k] (slot of pair
 *   t*k+j); active: i32 [E] (experts with rows, ascending);
 *   tiles: i32 [max_tiles, 4] = (expert, slot_begin, slot_end, 0) in chunks of
 *   tile_m rows; meta: i32 [QMOE_META_INTS] = (n_tiles, n_active, error, -,
 *   work counters): error is 1 when an id is outside [0, E) (then n_tiles =
 *   n_active = 0 and the slot maps are the identity); meta[3] is not touched;
 *   meta[4..23] are set to 0 (the grouped expert GEMMs' work queues).
 *   max_tiles = rows of `tiles`, at least ceil(T*k / tile_m) + E.  With
 *   max_tiles >= qmoe_moe_permute_tiles(T, k, E, tile_m) and T*k > 4096 the
 *   work is spread over one workgroup per 1024 pairs, using the rows past
 *   ceil(T*k / tile_m) + E as scratch; otherwise one workgroup does it all.
 * Replaces: the block metadata ExpertMLPsV2 builds for
 *   torch_blockwise_matmul_inference (token_position_to_id / block_to_expert,
 *   qwen_with_nki.py:5872-5881, 5478-5479; dedup 5656-5667 made unnecessary). */
int qmoe_moe_permute(const int32_t* topk_idx, int64_t T, int64_t k, int64_t E,
                     int64_t tile_m, int64_t max_tiles, int32_t* counts, int32_t* offsets,
                     int32_t* slot_token, int32_t* token_slot, int32_t* active,
                     int32_t* tiles, int32_t* meta, qmoe_stream_t stream);

/* Rows of `tiles` for which qmoe_moe_permute / qmoe_moe_route spread the
 * placement over several workgroups: ceil(T*k / tile_m) + E + ceil(C*(E+1)/4)
 * with C = ceil(T*k / 1024) chunks when 4096 < T*k <= 4096 * 1024 (the sizes
 * that path covers), else ceil(T*k / tile_m) + E (-1 for a non-positive k, E
 * or tile_m).
 * Replaces: nothing in the reference (a sizing helper of this library). */
int64_t qmoe_moe_permute_tiles(int64_t T, int64_t k, int64_t E, int64_t tile_m);

/* Routing in one call: router logits + top-k (as qmoe_router_topk) followed by
 * the dispatch metadata (as qmoe_moe_permute), same argument meanings.
 * Replaces: the router + dispatch-metadata step in front of ExpertMLPsV2
 *   (qwen_with_nki.py:8589-8590, 9886-9894, 5872-5881). */
int qmoe_moe_route(const qmoe_bf16* x, const qmoe_bf16* w_router, const float* bias, int64_t T,
                   int64_t H, int64_t E, int64_t k, int64_t tile_m, int64_t max_tiles,
                   float* logits, int32_t* topk_idx, float* topk_w, int32_t* counts,
                   int32_t* offsets, int32_t* slot_token, int32_t* token_slot, int32_t* active,
                   int32_t* tiles, int32_t* meta, qmoe_stream_t stream);

/* qmoe_moe_route with the router workspace of qmoe_router_topk_ws.
 * Replaces: as qmoe_moe_route (qwen_with_nki.py:8589-8590, 9886-9894,
 *   5872-5881). */
int qmoe_moe_route_ws(const qmoe_bf16* x, const qmoe_bf16* w_router, const float* bias, int64_t T,
                      int64_t H, int64_t E, int64_t k, int64_t tile_m, int64_t max_tiles,
                      float* logits, int32_t* topk_idx, float* topk_w, int32_t* counts,
                      int32_t* offsets, int32_t* slot_token, int32_t* token_slot, int32_t* active,
                      int32_t* tiles, int32_t* meta, void* workspace, int64_t workspace_bytes,
                      qmoe_stream_t stream);

/* The whole MoE block at decode shape (T <= 8):
 *   xin = x, or bf16(rmsnorm(h) * rms_w) written to x_out
 *   out[t] = residual[t] + sum_j topk_w[t,j] * expert_{topk_idx[t,j]}(xin[t])
 * At T = 1 with H = 2048, I = 768, k = 8, E <= 256 on a device with at least
 * QMOE_DECODE_BLOCK_WGS compute units it is one launch (router, top-k,
 * experts and combine; the workgroups exchange the router logits, the SwiGLU
 * outputs and per-expert row sums through the workspace header).  Otherwise
 * three launches: router logits (with the post-attention RMSNorm fused when
 * h is given); the expert kernel (top-k in every workgroup, then work items
 * of one touched expert and 8 intermediate units each: gate/up rows, SwiGLU,
 * and the matching down block, accumulated into a per-workgroup partial
 * output); and a fixed-order reduction of the partials with the residual.
 *   x: bf16 [T,H] or NULL; h: f32 [T,H] or NULL (exactly one of x, h);
 *   rms_w: bf16 [H] and x_out: bf16 [T,H] (with h); w_router: bf16 [E,H];
 *   bias: f32 [E] or NULL; w13: bf16 [E,2I,H] packed (QMOE_W13_GROUP);
 *   w2: bf16 [E, I/8, H, 8] blocked (QMOE_W2_BLOCK); residual: f32 [T,H] or
 *   NULL (may alias out and h); outputs logits f32 [T,E], topk_idx i32 [T,k],
 *   topk_w f32 [T,k]; out: f32 [T,H].
 *   workspace: device memory of at least qmoe_moe_decode_block_workspace(T, H)
 *   bytes, filled with zeros before its first use and otherwise left to the
 *   library: its first QMOE_DECODE_BLOCK_STATE_BYTES carry call counters
 *   from one call to the next (calls sharing a workspace, whatever their T,
 *   must not overlap in time).  The 32-bit word at byte offset
 *   QMOE_DECODE_BLOCK_STATUS_OFFSET becomes nonzero if a call's cross-
 *   workgroup wait ever gave up (that call's outputs are NaN); it is never
 *   set on a device where all QMOE_DECODE_BLOCK_WGS workgroups run at once.
 *   Deterministic: every sum runs in a fixed order.
 *   Limits: T <= 8, T*k <= 64, E <= 256, k <= 16, H in {512, 1024, 2048,
 *   4096}, I % 32 == 0, I <= 1536.
 * Replaces: the decode MoE path of NeuronQwen3MoeDecoderLayer.forward
 *   (post_attention_layernorm -> router -> forward_selective_loading ->
 *   residual add, qwen_with_nki.py:10203-10207, 3456-3478) in the fusion order
 *   of _nki_fused_moe_block_decoder_forward and _nki_fused_moe_block_kernel
 *   (8518-8711, 2184-2374: RMSNorm -> router -> experts -> residual). */
int qmoe_moe_decode_block(const qmoe_bf16* x, const float* h, const qmoe_bf16* rms_w, float eps,
                          const qmoe_bf16* w_router, const float* bias, const qmoe_bf16* w13,
                          const qmoe_bf16* w2, const float* residual, int64_t T, int64_t H,
                          int64_t I, int64_t E, int64_t k, float* logits, int32_t* topk_idx,
                          float* topk_w, void* workspace, int64_t workspace_bytes,
                          qmoe_bf16* x_out, float* out, qmoe_stream_t stream);

/* Workspace bytes qmoe_moe_decode_block needs for T tokens of width H
 * (QMOE_DECODE_BLOCK_STATE_BYTES + QMOE_DECODE_BLOCK_WGS * T * H floats); -1
 * for negative sizes.
 * Replaces: nothing in the reference (its kernels allocate their own HBM
 *   scratch, e.g. qwen_with_nki.py:1858); the caller owns memory here. */
int64_t qmoe_moe_decode_block_workspace(int64_t T, int64_t H);

/* qmoe_moe_decode_block without the workspace argument: its workspace (the
 * call-to-call state and the partial outputs) is a static device array
 * inside the library (16.25 MiB, zero when the library loads, one copy per
 * GPU, held until the process ends), so this call allocates nothing, not
 * even on its first use on a device.  Same arguments, kernels, limits and results as
 * qmoe_moe_decode_block, plus T * H <= QMOE_DECODE_BLOCK_NOALLOC_MAX_TH (T <= 8
 * at H = 2048); larger sizes are rejected with QMOE_ERR_INVALID.  The device is
 * the current device, which must be the stream's.  Every call on one GPU shares
 * that GPU's array: calls that overlap in time on one GPU (other streams,
 * other host threads) race and must be ordered by the caller.  Nothing needs
 * clearing between calls.
 * Replaces: nothing in the reference (no counterpart); it is for callers that
 *   cannot allocate device memory (code under HIP graph capture, tight
 *   serving loops, harnesses that forbid hipMalloc). */
int qmoe_moe_decode_block_noalloc(const qmoe_bf16* x, const float* h, const qmoe_bf16* rms_w,
                                  float eps, const qmoe_bf16* w_router, const float* bias,
                                  const qmoe_bf16* w13, const qmoe_bf16* w2,
                                  const float* residual, int64_t T, int64_t H, int64_t I,
                                  int64_t E, int64_t k, float* logits, int32_t* topk_idx,
                                  float* topk_w, qmoe_bf16* x_out, float* out,
                                  qmoe_stream_t stream);

/* Decode expert MLPs without the combine (bandwidth-bound GEMV form; each
 * touched expert's weights are streamed once for all tokens routed to it).
 *   x: bf16 [T, H]; w13: bf16 [E, 2I, H] packed (QMOE_W13_GROUP);
 *   w2: bf16 [E, I/8, H, 8] blocked (QMOE_W2_BLOCK); offsets/slot_token/active/meta
 *   from qmoe_moe_permute;
 *   act: f32 [T*k, I] workspace; y_slot: f32 [T*k, H] unweighted expert outputs.
 *   Limits: T <= 64, H in {512, 1024, 2048, 4096}, I % 32 == 0, I <= 1536.
 * Replaces: ExpertMLPsV2.forward_selective_loading (decode), restated at
 *   qwen_with_nki.py:3456-3478; _nki_batched_moe_kernel 1847-1982. */
int qmoe_moe_experts_gemv(const qmoe_bf16* x, const qmoe_bf16* w13, const qmoe_bf16* w2,
                          const int32_t* offsets, const int32_t* slot_token,
                          const int32_t* active, const int32_t* meta, int64_t T, int64_t H,
                          int64_t I, int64_t E, int64_t k, float* act, float* y_slot,
                          qmoe_stream_t stream);

/* Prefill expert MLPs as two grouped GEMMs on bf16 MFMA:
 *   act[s]    = bf16(silu(x[tok(s)] . Wg[e]^T) * (x[tok(s)] . Wu[e]^T))
 *   y_slot[s] = bf16(act[s] . W2[e]^T)
 *   x: bf16 [T, H]; w13: bf16 [E, 2I, H] packed; w2: bf16 [E, I/8, H, 8] blocked;
 *   slot_token/tiles/meta from qmoe_moe_permute with tile_m <=
 *   QMOE_GROUPED_MAX_TILE_M (256 is the efficient choice: every tile is one
 *   256 x 256 MFMA tile, partial tiles run only their live 32-row blocks);
 *   max_tiles >= ceil(T*k / QMOE_GROUPED_MAX_TILE_M) + E;
 *   act: bf16 [T*k, I] workspace; y_slot: bf16 [T*k, H].
 *   Work distribution: one persistent workgroup per CU takes (tile, weight
 *   panel) items from per-XCD queues whose counters live in meta[4..21]
 *   (zeroed by the permute; the last workgroup puts them back to zero).
 *   With I % 64 == 0 and act 128-byte aligned both GEMMs run in one launch:
 *   the workgroups take the gate_up items first and then the down items, a
 *   down item waiting until its tile's gate_up items are done; word 3 of
 *   each live tile row counts them (0 from the permute, 0 again once the
 *   launch completes), and meta[2] gets bit 1 if such a wait ever gave up.
 *   Calls that share one meta array or tile table must not overlap.
 *   Limits: H % 256 == 0, I % 32 == 0; x, act and one expert's w13 each
 *   below 2 GiB.
 * Replaces: _nki_cte_moe_left_gate_up_kernel qwen_with_nki.py:5341-5369 (left)
 *   and _nki_cte_moe_down_scatter_kernel 4967-5040 (right), dispatched by
 *   _patched_torch_blockwise_matmul_inference 5872-6003. */
int qmoe_moe_experts_grouped(const qmoe_bf16* x, const qmoe_bf16* w13, const qmoe_bf16* w2,
                             const int32_t* slot_token, int32_t* tiles,
                             int32_t* meta, int64_t max_tiles, int64_t T, int64_t H,
                             int64_t I, int64_t E, int64_t k, qmoe_bf16* act,
                             qmoe_bf16* y_slot, qmoe_stream_t stream);

/* Weighted unpermute-combine, deterministic (fixed order j = 0..k-1, fp32):
 *   out[t] = residual[t] + sum_j topk_w[t,j] * y_slot[token_slot[t*k+j]]
 *   y_slot: f32 or bf16 (y_is_bf16) [T*k, H]; residual: f32 [T, H] or NULL
 *   (may alias out); out: f32 [T, H].
 * Replaces: the affinity multiply + scatter-add of the right kernel
 *   (_allblk_fused_down_aff_scatter qwen_with_nki.py:4583-4710; fp32
 *   accumulator variant 5043-5121) and the decode sum(out * aff) 3467-3478,
 *   plus the residual add at 10207. */
int qmoe_moe_combine(const void* y_slot, int y_is_bf16, const int32_t* token_slot,
                     const float* topk_w, const float* residual, int64_t T, int64_t k,
                     int64_t H, float* out, qmoe_stream_t stream);

/* qmoe_moe_combine, then the RMSNorm of each finished row:
 *   x_out[t] = bf16(rms_w * out[t] * rsqrt(mean(out[t]^2) + eps))
 * (the next decoder layer's input norm), with the bits of qmoe_moe_combine
 * followed by qmoe_rmsnorm_residual on `out`.  One launch, a workgroup per
 * token row.  rms_w: bf16 [H]; x_out: bf16 [T, H]; H % 4 == 0, H <= 8192.
 * Replaces: the MoE output's residual add (qwen_with_nki.py:10207) and the
 *   next layer's input_layernorm (10185-10189). */
int qmoe_moe_combine_norm(const void* y_slot, int y_is_bf16, const int32_t* token_slot,
                          const float* topk_w, const float* residual, int64_t T, int64_t k, int64_t H,
                          float* out, const qmoe_bf16* rms_w, float eps, qmoe_bf16* x_out,
                          qmoe_stream_t stream);

/* Dense GEMM C = A . B^T with an epilogue mode (QMOE_GEMM_*); bf16 inputs,
 * fp32 accumulation.  A: bf16 [M, K] (row stride lda); B: bf16 [N, K];
 * C: [M, N] with row stride ldc.  Limits: K % 64 == 0 and A, B below
 * 2 GiB when M > 16 (MFMA path); K % 512 == 0 when M <= 16 and
 * M*K <= 32768 (GEMV path).
 * Replaces: the o_proj / lm_head ColumnParallelLinear projections of the
 *   NxDI attention base and model (qwen_with_nki.py:10277-10282);
 *   _nki_lm_head_kernel 1766-1805. */
int qmoe_gemm(const qmoe_bf16* A, int64_t lda, const qmoe_bf16* B, int64_t M, int64_t N,
              int64_t K, int mode, void* C, int64_t ldc, qmoe_stream_t stream);

/* C += A . B^T (fp32 C[M, N], row stride N), then x_out = bf16(rms_w *
 * C * rsqrt(mean(C^2 over the row) + eps)) for every row: the o_proj's
 * residual add and the post-attention RMSNorm of a prefill chunk.  With a
 * split-K plan and workspace (as qmoe_gemm_ws) the norm runs inside the
 * launch that adds the slices; otherwise qmoe_gemm then
 * qmoe_rmsnorm_residual.  Either way the bits of those two calls.
 *   A: bf16 [M, K] (lda); B: bf16 [N, K]; rms_w: bf16 [N]; x_out: bf16
 *   [M, N]; N % 4 == 0, N <= 8192.
 * Replaces: the attention output projection into the residual and the
 *   post-attention RMSNorm of the decoder layer (qwen_with_nki.py:10200-10205;
 *   o_proj 10089-10099). */
int qmoe_gemm_ws_add_rmsnorm(const qmoe_bf16* A, int64_t lda, const qmoe_bf16* B, int64_t M, int64_t N,
                             int64_t K, float* C, const qmoe_bf16* rms_w, float eps, qmoe_bf16* x_out,
                             void* workspace, int64_t workspace_bytes, qmoe_stream_t stream);

/* qmoe_gemm with a caller-owned workspace for split-K: when the problem has
 * too few output tiles to occupy the GPU (prefill-size o_proj, 640 x 2048
 * with K = 4096; the router logits, 640 x 128 with K = 2048), K is split into
 * slices whose fp32 partial tiles go to `workspace` and a second launch adds
 * them in slice order and applies `mode` (deterministic: no atomics).  Other
 * problems, or a workspace smaller than qmoe_gemm_ws_workspace(M, N, K)
 * bytes, take the qmoe_gemm path.  Same arguments and limits as qmoe_gemm.
 * Calls sharing a workspace must not overlap.
 * Replaces: the same projections as qmoe_gemm (o_proj qwen_with_nki.py:10089-
 *   10099; router linear 8589-8590) at prefill sizes. */
int qmoe_gemm_ws(const qmoe_bf16* A, int64_t lda, const qmoe_bf16* B, int64_t M, int64_t N,
                 int64_t K, int mode, void* C, int64_t ldc, void* workspace, int64_t workspace_bytes,
                 qmoe_stream_t stream);

/* Workspace bytes qmoe_gemm_ws uses for an M x N x K problem (0: it does not
 * split K for this shape); -1 for negative sizes.
 * Replaces: nothing in the reference (caller-owned scratch). */
int64_t qmoe_gemm_ws_workspace(int64_t M, int64_t N, int64_t K);

/* One-row GEMV with the input RMSNorm fused into its activation staging:
 *   C[n] (mode as qmoe_gemm) = bf16(rms_w * h * rsqrt(mean(h^2) + eps)) . B[n]^T
 *   h: f32 [K] (the residual stream row); rms_w: bf16 [K]; B: bf16 [N, K].
 *   The normalised row has the same bits as qmoe_rmsnorm_residual's output,
 *   so C matches qmoe_rmsnorm_residual followed by qmoe_gemm, in one launch.
 *   Limits: K in {512, 1024, 2048, 4096}.
 * Replaces: input_layernorm feeding the attention's QKV projection in the
 *   decoder layer (qwen_with_nki.py:10155-10213, NKIRMSNorm 1286-1415). */
int qmoe_gemv_rmsnorm(const float* h, const qmoe_bf16* rms_w, float eps, const qmoe_bf16* B, int64_t N,
                      int64_t K, int mode, void* C, qmoe_stream_t stream);

/* QKV projection with per-head RMSNorm over head_dim and RoPE fused into the
 * epilogue; K/V written straight into the contiguous cache.
 *   x: bf16 [B*S, H]; wqkv: bf16 [(Hq+2*Hkv)*D, H] (q rows, then k, then v);
 *   q_norm_w, k_norm_w: bf16 [D]; rope_cos, rope_sin: f32 [max_pos, D/2];
 *   positions: i32 [B*S] (RoPE position == cache index of the token);
 *   q_out: bf16 [B*S, Hq, D]; k_cache, v_cache: bf16 [B, Hkv, S_max, D];
 *   workspace: f32, qmoe_qkv_norm_rope_workspace(B*S, H, Hq, Hkv, D) bytes
 *   (decode-size token counts run the projection as an all-CU GEMV into it;
 *   NULL allowed when that size is 0).
 *   Limits: D == 128, H % 64 == 0, positions < S_max and < max_pos.
 * Replaces: NeuronQwen3MoEAttention (qwen_with_nki.py:10081-10109): QKV
 *   projection, q_layernorm/k_layernorm (10102-10103) before RoPE
 *   (RotaryEmbedding base=rope_theta 10083-10087), KV-cache update. */
int qmoe_qkv_norm_rope(const qmoe_bf16* x, const qmoe_bf16* wqkv, const qmoe_bf16* q_norm_w,
                       const qmoe_bf16* k_norm_w, const float* rope_cos, const float* rope_sin,
                       int64_t max_pos, const int32_t* positions, int64_t B, int64_t S,
                       int64_t H, int64_t Hq, int64_t Hkv, int64_t D, int64_t S_max, float eps,
                       qmoe_bf16* q_out, qmoe_bf16* k_cache, qmoe_bf16* v_cache, float* workspace,
                       qmoe_stream_t stream);

/* The second half of qmoe_qkv_norm_rope's decode path on its own, for callers
 * that produce the raw projection another way (qmoe_gemv_rmsnorm with the
 * input RMSNorm fused in): per (token, head) RMSNorm over head_dim and RoPE
 * for q and k, q to q_out, k / v rows into the cache at positions[t].
 *   qkv: f32 [B*S, (Hq + 2*Hkv)*D] before normalisation; other arguments as
 *   qmoe_qkv_norm_rope.  Limits: D == 128, B*S <= 16.
 * Replaces: q_layernorm/k_layernorm, RoPE and the KV-cache update of
 *   NeuronQwen3MoEAttention (qwen_with_nki.py:10102-10103, 10083-10087,
 *   9943-9946). */
int qmoe_qkv_finish(const float* qkv, const qmoe_bf16* q_norm_w, const qmoe_bf16* k_norm_w,
                    const float* rope_cos, const float* rope_sin, int64_t max_pos, const int32_t* positions,
                    int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t D, int64_t S_max, float eps,
                    qmoe_bf16* q_out, qmoe_bf16* k_cache, qmoe_bf16* v_cache, qmoe_stream_t stream);

/* Workspace bytes of qmoe_qkv_norm_rope for T = B*S token rows: T * (Hq +
 * 2*Hkv) * D * 4 when T <= 16 and H in {512, 1024, 2048, 4096} with T*H <=
 * 32768 (the GEMV path), else 0; -1 for negative sizes.
 * Replaces: nothing in the reference (its kernels allocate their own HBM
 *   scratch); the caller owns memory here. */
int64_t qmoe_qkv_norm_rope_workspace(int64_t T, int64_t H, int64_t Hq, int64_t Hkv, int64_t D);

/* Causal GQA flash attention for a prefill chunk.  Query s of batch b sits at
 * cache index start + s and sees cache entries [0, start + s].
 *   q: bf16 [B*S, Hq, D]; k_cache, v_cache: bf16 [B, Hkv, S_max, D];
 *   out: bf16 [B*S, Hq*D].  Limits: D == 128, Hq % Hkv == 0, S_max <= 2^22.
 * Replaces: the NxDI attention base's context-encoding attention
 *   (flash kernel attention_isa_kernel, qwen_with_nki.py:25-28, 1251). */
int qmoe_attn_prefill(const qmoe_bf16* q, const qmoe_bf16* k_cache, const qmoe_bf16* v_cache,
                      int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t D, int64_t S_max,
                      int64_t start, float scale, qmoe_bf16* out, qmoe_stream_t stream);

/* qmoe_attn_prefill with a workspace, which lets a launch with fewer query
 * tiles (B * Hq * ceil(S/128)) than the GPU has CUs split the key range of
 * its longer tiles over several workgroups (at most one per CU in all); the
 * last split of a tile to finish merges the partials in split order, so the
 * result is deterministic (it differs from qmoe_attn_prefill's in rounding).
 * Larger launches, or a workspace smaller than
 * qmoe_attn_prefill_workspace(B, S, Hq, D) bytes, run as qmoe_attn_prefill.
 * The workspace must be zero before its first use; every call leaves its
 * counters at zero again.  Calls sharing a workspace must not overlap.
 * Replaces: as qmoe_attn_prefill (qwen_with_nki.py:25-28, 1251). */
int qmoe_attn_prefill_ws(const qmoe_bf16* q, const qmoe_bf16* k_cache, const qmoe_bf16* v_cache,
                         int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t D, int64_t S_max,
                         int64_t start, float scale, void* workspace, int64_t workspace_bytes,
                         qmoe_bf16* out, qmoe_stream_t stream);

/* Workspace bytes of qmoe_attn_prefill_ws on the current device (-1 for bad
 * sizes).
 * Replaces: nothing in the reference (a sizing helper of this library). */
int64_t qmoe_attn_prefill_workspace(int64_t B, int64_t S, int64_t Hq, int64_t D);

/* qmoe_attn_decode for contexts known to fit a bucket: ctx_len[b] <= max_ctx
 * <= S_max (larger values are clamped to max_ctx).  The launch is sized for
 * max_ctx instead of the cache capacity S_max (the row stride), so a decode
 * graph captured per context bucket launches no workgroups for cache rows no
 * query can see; partial needs qmoe_attn_decode_workspace(B, Hq, D, max_ctx)
 * floats.
 * Replaces: the per-bucket token-generation graphs of NxDI (main.py:156-161;
 *   qwen_with_nki.py:10892-10916) for the attention step. */
int qmoe_attn_decode_bucket(const qmoe_bf16* q, const qmoe_bf16* k_cache, const qmoe_bf16* v_cache,
                            const int32_t* ctx_len, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                            int64_t S_max, int64_t max_ctx, float scale, float* partial, qmoe_bf16* out,
                            qmoe_stream_t stream);

/* One decode step of the attention from the raw QKV projection: the finish of
 * qmoe_qkv_finish (q/k RMSNorm, RoPE, the new K/V row into the cache at
 * positions[b]) and qmoe_attn_decode_bucket in one split launch + the merge,
 * with the same result bits as those two calls.  Row b sees cache entries
 * [0, positions[b]], at most the first max_ctx of them (a position at or
 * past max_ctx still writes its K/V row); a position outside [0,
 * min(S_max, max_pos)) writes nothing and gets zeros.
 *   qkv: f32 [B, (Hq + 2*Hkv)*D] (qmoe_gemv_rmsnorm / qmoe_gemm with
 *   QMOE_GEMM_STORE_F32); q_norm_w, k_norm_w: bf16 [D]; rope_cos, rope_sin:
 *   f32 [max_pos, D/2]; k_cache, v_cache: bf16 [B, Hkv, S_max, D]; partial:
 *   qmoe_attn_decode_workspace(B, Hq, D, max_ctx) floats; out: bf16 [B, Hq*D].
 *   Limits as qmoe_attn_decode_bucket.
 * Replaces: q_layernorm/k_layernorm, RoPE, the KV-cache update and the
 *   token-generation attention of NeuronQwen3MoEAttention
 *   (qwen_with_nki.py:10102-10103, 10083-10087, 9943-9946; main.py:156-161). */
int qmoe_attn_decode_fused(const float* qkv, const qmoe_bf16* q_norm_w, const qmoe_bf16* k_norm_w,
                           const float* rope_cos, const float* rope_sin, int64_t max_pos, const int32_t* positions,
                           int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t S_max, int64_t max_ctx,
                           float eps, float scale, qmoe_bf16* k_cache, qmoe_bf16* v_cache, float* partial,
                           qmoe_bf16* out, qmoe_stream_t stream);

/* S consecutive queries per batch row, at cache positions start..start+S-1
 * (start: device int32[1], clamped into [0, S_max - S]); query s attends to
 * keys [0, start + s].  Computed as B*S single-query problems (the split +
 * merge of qmoe_attn_decode over the full capacity), which suits the few-token
 * chunks of speculative verification better than the tiled prefill kernel.
 *   q: bf16 [B*S][Hq][D]; k_cache, v_cache: [B][Hkv][S_max][D] (the chunk's
 *   rows already written); partial: qmoe_attn_decode_workspace(B*S, Hq, D,
 *   S_max) floats; out: bf16 [B*S][Hq*D].  Limits as qmoe_attn_decode, B*S < 65536.
 * Replaces: the attention of the speculation driver's verification forward
 *   over the candidate chunk (_spec_generate qwen_with_nki.py:575-1211). */
int qmoe_attn_decode_chunk(const qmoe_bf16* q, const qmoe_bf16* k_cache, const qmoe_bf16* v_cache,
                           const int32_t* start, int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t D,
                           int64_t S_max, float scale, float* partial, qmoe_bf16* out,
                           qmoe_stream_t stream);

/* qmoe_attn_prefill with the chunk start in device memory (start: i32 [1],
 * read by the kernel and clamped into [0, S_max - S]), so that one captured
 * launch serves every position: the multi-token verification step of
 * prompt-lookup speculative decoding (S = spec_len query tokens at
 * start..start+S-1 against the cache).
 * Replaces: the speculation model's verification pass over the candidate
 *   tokens (`_spec_generate`, qwen_with_nki.py:575-1211; spec_len 5, line 74). */
int qmoe_attn_prefill_at(const qmoe_bf16* q, const qmoe_bf16* k_cache, const qmoe_bf16* v_cache,
                         int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t D, int64_t S_max,
                         const int32_t* start, float scale, qmoe_bf16* out, qmoe_stream_t stream);

/* Decode attention (split-KV flash decoding on MFMA: one partial per 64
 * cache entries, then a merge), one query per batch row that sees cache
 * entries [0, ctx_len[b]).
 *   q: bf16 [B, Hq, D]; ctx_len: i32 [B] (1 <= ctx_len <= S_max);
 *   partial: f32 workspace of qmoe_attn_decode_workspace(B, Hq, D, S_max) floats;
 *   out: bf16 [B, Hq*D].  Limits: D == 128, Hq / Hkv <= 16.
 * Replaces: the NxDI attention base's token-generation attention over the KV
 *   cache [B, Hkv, S, D] (qwen_with_nki.py:9943-9946). */
int64_t qmoe_attn_decode_workspace(int64_t B, int64_t Hq, int64_t D, int64_t S_max);
int qmoe_attn_decode(const qmoe_bf16* q, const qmoe_bf16* k_cache, const qmoe_bf16* v_cache,
                     const int32_t* ctx_len, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                     int64_t S_max, float scale, float* partial, qmoe_bf16* out,
                     qmoe_stream_t stream);

/* Token embedding gather into the fp32 residual stream:
 *   out[i, :] = float(table[ids[i], :]);  table: bf16 [V, H]; ids: i64 [n];
 *   out: f32 [n, H].  An id outside [0, V) writes a zero row and sets
 *   err[0] = 1 (err: i32, cleared by the caller); nothing traps on the GPU.
 *   Limits: H % 4 == 0.
 * Replaces: the model's ParallelEmbedding lookup (qwen_with_nki.py:10250-10256)
 *   and the NKI embedding gather _nki_embedding_kernel (1541-1578). */
int qmoe_embed(const qmoe_bf16* table, int64_t V, int64_t H, const int64_t* ids, int64_t n,
               float* out, int32_t* err, qmoe_stream_t stream);

/* Greedy token per row: out[r] = argmax_j x[r, j] (first maximum; NaN ranks
 * highest, first NaN wins), in two launches with no memset, so it replays
 * correctly inside a HIP graph.  x: f32 rows of n (row stride ldx); out: i64
 * [rows]; workspace of qmoe_argmax_workspace(rows) bytes.
 * Replaces: greedy selection over the lm_head logits in the generation loop
 *   (main.py:557-569 with do_sample off; the reference's on-device sampling
 *   path and _nki_lm_head_kernel 1766-1805 produce the logits it reads). */
int qmoe_argmax(const float* x, int64_t rows, int64_t n, int64_t ldx, void* workspace,
                int64_t workspace_bytes, int64_t* out, qmoe_stream_t stream);

/* Workspace bytes of qmoe_argmax for `rows` rows (-1 for rows < 0).
 * Replaces: nothing in the reference; the caller owns memory here. */
int64_t qmoe_argmax_workspace(int64_t rows);

#ifdef __cplusplus
}
#endif

#endif /* QMOE_CAPI_H */
