/*
 * af3_mi355x.h — C ABI of libaf3_mi355x.so, the gfx950 (MI355X) HIP
 * implementation of agent-factory-3's MXFP4 MoE expert hot path.
 *
 * Conventions (every entry point):
 *   - pointers are device pointers; bf16 tensors are passed as uint16_t* bit
 *     patterns; MXFP4 weights as packed uint8 blocks + uint8 e8m0 scales;
 *   - `stream` is a hipStream_t (torch.cuda.current_stream().cuda_stream);
 *     work is enqueued on it, nothing synchronises the host;
 *   - the library never allocates, frees or keeps pointers: callers own all
 *     outputs and workspaces;
 *   - return 0 on success, a negative value for an argument error, or a
 *     positive hipError_t; af3_last_error() gives the message (per thread).
 *
 * Reference citations are file:line in ycchen-tw/agent-factory-3,
 * src/agent_factory_3/models/gpt_oss/.
 */
#ifndef AF3_MI355X_H
#define AF3_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ABI version (2: af3_moe_gemm_f8 takes trans_w after w_scales; 1 had no trans_w). */
int af3_abi_version(void);

/* Message of the last failing call on this host thread. */
const char* af3_last_error(void);

/* MXFP4 -> bf16.  Replaces kernels.py:206-235 (mxfp4_to_bf16_triton) and the
 * quantization.py:89-99 wrapper mxfp4_to_bf16.  blocks [n_groups][16] u8,
 * scales [n_groups] u8, out [n_groups][32] bf16; bit-exact with
 * kernels.py:120-158 for every (nibble, scale) pair. */
int af3_mxfp4_to_bf16(const uint8_t* blocks, const uint8_t* scales, uint16_t* out, int64_t n_groups,
                      void* stream);

/* Clamped SwiGLU forward.  Replaces kernels.py:451-490 (_swiglu_forward_triton).
 * gate_up [M][ld_in] interleaved (gate even, up odd), out [M][ld_out];
 * gate_save/up_save (both or neither) receive the clamped gate/up. */
int af3_swiglu_fwd(const uint16_t* gate_up, int64_t ld_in, uint16_t* out, int64_t ld_out, uint16_t* gate_save,
                   uint16_t* up_save, int64_t ld_save, int64_t M, int64_t N, float alpha, float limit,
                   void* stream);

/* Clamped SwiGLU backward from saved clamped gate/up.  Replaces
 * kernels.py:556-582 (_swiglu_backward); grad_gu [M][ld_gu] interleaved. */
int af3_swiglu_bwd(const uint16_t* grad_out, int64_t ld_grad, const uint16_t* gate, const uint16_t* up,
                   int64_t ld_save, uint16_t* grad_gu, int64_t ld_gu, int64_t M, int64_t N, float alpha,
                   float limit, void* stream);

/* Same backward from the raw interleaved pre-activation (clamps internally);
 * used by SwiGLUFunction (quantization.py:424-444) so the forward need not
 * store gate/up. */
int af3_swiglu_bwd_raw(const uint16_t* grad_out, int64_t ld_grad, const uint16_t* gate_up, int64_t ld_in,
                       uint16_t* grad_gu, int64_t ld_gu, int64_t M, int64_t N, float alpha, float limit,
                       void* stream);

/* Workspace bytes needed by af3_routing_replay / af3_routing_topk. */
size_t af3_routing_workspace_bytes(int64_t n_tokens, int n_expts_tot, int n_expts_act);

/* Routing from given expert ids.  Replaces quantization.py:593-636
 * (routing_replay).  logits [T][ld] bf16, expt_indx [T][K] int32 ->
 * gate_scal [T*K] bf16 (softmax over the K gathered logits, expert-sorted),
 * hist [E], topk_indx [T*K] (sorted row -> flat t*K+j), gate_indx [T*K]
 * (flat -> sorted row), token_offs_raw [E+1].  Ids outside [0,E) are dropped
 * (gate_indx = -1, trailing sorted slots topk_indx = -1). */
int af3_routing_replay(const uint16_t* logits, int64_t ld_logits, const int32_t* expt_indx, int64_t n_tokens,
                       int n_expts_tot, int n_expts_act, uint16_t* gate_scal, int32_t* hist, int32_t* topk_indx,
                       int32_t* gate_indx, int32_t* token_offs_raw, void* workspace, size_t ws_bytes,
                       void* stream);

/* Allocation-free variant of af3_routing_replay (no counterpart in the
 * reference): same arguments and outputs without the workspace, which comes
 * from a built-in per-device scratch array of af3_routing_scratch_bytes()
 * (4 MiB: T*K up to ~500k rows at E = 128).  For callers that cannot
 * allocate device memory (HIP graph capture, tight serving loops).  Makes no
 * allocation; a shape needing more than the array returns AF3_EINVAL with a
 * message.  Calls that overlap on one device share its array and race: issue
 * them on one stream.  The first call on a device takes the array's address
 * (hipGetSymbolAddress). */
size_t af3_routing_scratch_bytes(void);
int af3_routing_replay_noalloc(const uint16_t* logits, int64_t ld_logits, const int32_t* expt_indx,
                               int64_t n_tokens, int n_expts_tot, int n_expts_act, uint16_t* gate_scal,
                               int32_t* hist, int32_t* topk_indx, int32_t* gate_indx, int32_t* token_offs_raw,
                               void* stream);

/* Top-K routing.  Replaces triton_kernels.routing.routing as called at
 * quantization.py:651,664 (torch restatement: routing_torch_dist,
 * quantization.py:551-590 at world size 1).  Same outputs as above. */
int af3_routing_topk(const uint16_t* logits, int64_t ld_logits, int64_t n_tokens, int n_expts_tot,
                     int n_expts_act, uint16_t* gate_scal, int32_t* hist, int32_t* topk_indx, int32_t* gate_indx,
                     int32_t* token_offs_raw, void* workspace, size_t ws_bytes, void* stream);

/* Router logits.  Replaces nn.functional.linear(hidden_states,
 * router.weight, router.bias) in mlp_forward (quantization.py:653-654):
 * logits[t][e] = bf16(sum_k x[t][k] w[e][k] + bias[e]) with fp32 sums.
 * x [T][ldx] bf16, w [E][ldw] bf16, bias [E] bf16 or NULL, logits
 * [T][ld_logits] bf16; hidden % 64 == 0, E <= 256, rows 16-byte aligned. */
int af3_router_logits(const uint16_t* x, int64_t ldx, const uint16_t* w, int64_t ldw, const uint16_t* bias,
                      int64_t n_tokens, int hidden, int n_expts, uint16_t* logits, int64_t ld_logits, void* stream);

/* Tile metadata.  Replaces triton_kernels.routing.compute_expt_data_torch
 * (quantization.py:588,627).  block_ms_dev [n_block_ms] (device) ->
 * token_offs_pad [n_block_ms][E+1], block_pid_map [n_block_ms][max_tiles]
 * with entries (block << 16) | expert or -1. */
int af3_expt_data(const int32_t* hist, int n_expts_tot, const int32_t* block_ms_dev, int n_block_ms, int max_tiles,
                  int32_t* token_offs_pad, int32_t* block_pid_map, void* stream);

/* Work order of the block_m-row tiles for af3_moe_gemm: the entries of the
 * af3_expt_data block_pid_map for this block_m (token_offs_pad = its padded
 * tile offsets), permuted so that full tiles come first in expert order and
 * each expert's partial last tile follows by decreasing row count, -1 past
 * the tile count.  No counterpart in the reference (its block_pid_map,
 * compute_expt_data_torch, is in expert order and that order is kept there);
 * the grouped GEMM takes either map.  n_expts_tot <= 4096, block_m <= 512.
 * max_tiles should be >= sum_e ceil(hist[e] / block_m); a smaller one gives a
 * truncated order (no write past order[max_tiles - 1]). */
int af3_tile_order(const int32_t* hist, int n_expts_tot, int block_m, const int32_t* token_offs_pad, int max_tiles,
                   int32_t* order, void* stream);

/* Grouped GEMM through frozen MXFP4 expert weights, dequant fused into the
 * tile load.  Replaces mxfp4_to_bf16 + matmul_ogs at quantization.py:358-362
 * (trans_w = 0; forward, A6/A8) and quantization.py:409-418 (trans_w = 1;
 * dX backward, A9/A11), without the scatter (see af3_moe_combine).
 *   trans_w 0: Y[r][n] = sum_k X[a(r)][k] W[e][n][k],  blocks [E][N][K/32][16]
 *   trans_w 1: Y[r][n] = sum_k X[a(r)][k] W[e][k][n],  blocks [E][K][N/32][16]
 *   + sum_j L[r][j] Bx[e][n][j] (trans 0) / Bx[e][j][n] (trans 1)  if lora_r > 0
 *   Y = bf16((acc + bias[e][n]) * gammas[r])   (bias fp32 [E][N], gammas bf16 or fp32)
 * a(r) = gather_indx ? gather_indx[r] / gather_div : r; rows r of expert e
 * are [token_offs[e], token_offs[e+1]); block_pid_map / tile_offs are the
 * af3_expt_data map and token_offs_pad for BM = block_m (128 or 256); the
 * number of valid m-tiles is read from tile_offs[n_expts] on the device.
 * tile_cfg picks the block tile; 0 = the default for block_m and trans_w:
 * block_m 128 -> 26 (forward, 128 x 256 work items, two blocks per CU) and
 * 28 (input gradient, same shape); block_m 256 -> 22 / 23 (256 x 256); the
 * general fallbacks 4 / 2 / 9 where a default's alignment or K % 64 == 0
 * requirement fails.  tile_cfg / 100 = m-tiles per work group of the
 * 22 / 23 / 26 / 28 order (default 4; 2 for 26 / 28).  tile_cfg |
 * AF3_W_FWD_TILED: w_blocks is the af3_mxfp4_tile_fwd copy of the weights
 * (trans_w 0, the tile_cfg 26 forward only; AF3_EUNSUPPORTED, nothing
 * launched, when another kernel is selected: the caller then passes the
 * row-major blocks).  tile_cfg | AF3_X_OFFSETS_32: the caller vouches that
 * every row of x the call reads lies within 4 GiB of x (a(r) * ldx * 2 + K * 2
 * <= 2^32), so the tile_cfg 26 forward may address x by a scalar base and
 * 32-bit lane offsets (the Python layer sets it when x's whole extent is
 * below 4 GiB); without it every address is 64-bit. */
#ifndef AF3_W_FWD_TILED
#define AF3_W_FWD_TILED 0x10000
#endif
#ifndef AF3_X_OFFSETS_32
#define AF3_X_OFFSETS_32 0x20000
#endif
/* tile_cfg | AF3_S_DX_TILED (trans_w 1, the tile_cfg 28 input gradient only,
 * else AF3_EUNSUPPORTED with nothing launched): w_scales is the
 * af3_mxfp4_tile_dx_scales copy of the scales. */
#ifndef AF3_S_DX_TILED
#define AF3_S_DX_TILED 0x40000
#endif
int af3_moe_gemm(const uint16_t* x, int64_t ldx, const int32_t* gather_indx, int gather_div,
                 const uint8_t* w_blocks, const uint8_t* w_scales, int trans_w, const float* bias,
                 const void* gammas, int gammas_f32, const uint16_t* lora_l, int64_t ld_l, const uint16_t* lora_b,
                 int lora_r, const int32_t* token_offs, const int32_t* block_pid_map, const int32_t* tile_offs,
                 int max_tiles, int block_m, int tile_cfg, int n_expts, int N, int K, uint16_t* y, int64_t ldy,
                 void* stream);

/* Forward-tiled copy of packed MXFP4 weights for the tile_cfg 26 forward.
 * No counterpart in the reference (its matmul_ogs reads the weights as
 * stored, quantization.py:358-362); a byte permutation made once per frozen
 * weight: blocks [n_mats][N][K/32][16] -> out [n_mats][N/32][K/64][2][32][16],
 * out[e][n/32][kt][h][n%32] = blocks[e][n][2 kt + h], so the words one
 * k-step of the forward's wave needs from 32 weight rows are one contiguous
 * KB (row-major they are 32 bytes of 32 different 128-byte lines).  The
 * scales stay as they are.  N % 32 == 0, K % 64 == 0, 16-byte aligned, out
 * the same size as blocks and not overlapping it. */
int af3_mxfp4_tile_fwd(const uint8_t* blocks, int64_t n_mats, int N, int K, uint8_t* out, void* stream);

/* Tiled copy of the e8m0 scales for the tile_cfg 28 input gradient.  No
 * counterpart in the reference (its matmul_ogs reads the stored scales,
 * quantization.py:409-418); a byte permutation made once per frozen weight:
 * scales [n_mats][K][N/32] (the trans_w 1 view: K = the reduction rows) ->
 * out [n_mats][K/64][ceil(N/256)][8][64], out[e][k/64][n/256][(n/32)%8][k%64]
 * = scales[e][k][n/32], 127 past N/32, so the scale bytes one wave needs for
 * a 64-deep k-step (its two 32-column blocks x 64 rows) are 128 contiguous
 * bytes; then one flag byte per (matrix, 256-column n-tile): 1 when a scale
 * byte of its columns lies outside [2, 252] (the kernel then takes the exact
 * integer conversion for that n-tile).  K % 64 == 0, N % 32 == 0; out holds
 * n_mats * ceil(N/256) * (K/64 * 512 + 1) bytes and does not overlap scales. */
int af3_mxfp4_tile_dx_scales(const uint8_t* scales, int64_t n_mats, int K, int N, uint8_t* out, void* stream);

/* af3_moe_gemm with the gpt-oss clamped SwiGLU (kernels.py:394-582 math)
 * fused into the epilogue, so the activation never makes a separate pass
 * through HBM.  Replaces the SwiGLUFunction.backward that follows the
 * down-projection dX product (quantization.py:409-418, 442-444: epi 1,
 * trans_w 1, y <- dGU [rows][2N] from the bf16 product dI and the saved
 * interleaved pre-activation glu [rows][2N], ld_glu) and the
 * SwiGLUFunction.forward that follows the gate_up product (quantization.py:
 * 516-525, 432-439: epi 2, trans_w 0, y <- the bf16 pre-activation [rows][N]
 * and glu <- its SwiGLU [rows][N/2]).  Results equal the unfused sequence bit
 * for bit.  Returns AF3_EUNSUPPORTED (-2) when the selected tile configuration
 * has no fused epilogue (epi 2: tile_cfg 22 / 26, epi 1: 23 / 28); the caller
 * then runs the unfused pair. */
int af3_moe_gemm_swiglu(const uint16_t* x, int64_t ldx, const int32_t* gather_indx, int gather_div,
                        const uint8_t* w_blocks, const uint8_t* w_scales, int trans_w, const float* bias,
                        const void* gammas, int gammas_f32, const uint16_t* lora_l, int64_t ld_l,
                        const uint16_t* lora_b, int lora_r, const int32_t* token_offs, const int32_t* block_pid_map,
                        const int32_t* tile_offs, int max_tiles, int block_m, int tile_cfg, int n_expts, int N, int K,
                        uint16_t* y, int64_t ldy, int epi, void* glu, int64_t ld_glu, float alpha, float limit,
                        void* stream);

/* af3_moe_gemm (no LoRA segment) with a per-row scale of the A operand on
 * the accumulator: y = bf16((acc * a_row_scale[a(r)] + bias[e][n]) * gammas[r]),
 * a(r) the A row of output row r (a_row_scale has one fp32 per row of x).
 * Replaces matmul_ogs with PrecisionConfig(lhs InFlexData(scale,
 * scale_mode="per_token")) in the fp8 mode, quantization.py:338-356 (forward)
 * and 382-408 (dX), fed with the E4M3 codes' values as bf16.  Returns
 * AF3_EUNSUPPORTED (-2) when the selected tile configuration has no scaled
 * epilogue (only tile_cfg 22, 23, 26 and 28 have one). */
int af3_moe_gemm_rowscale(const uint16_t* x, int64_t ldx, const int32_t* gather_indx, int gather_div,
                          const uint8_t* w_blocks, const uint8_t* w_scales, int trans_w, const float* bias,
                          const void* gammas, int gammas_f32, const int32_t* token_offs, const int32_t* block_pid_map,
                          const int32_t* tile_offs, int max_tiles, int block_m, int tile_cfg, int n_expts, int N,
                          int K, uint16_t* y, int64_t ldy, const float* a_row_scale, void* stream);

/* fp8 mode on the block-scaled MFMA (v_mfma_scale_f32_32x32x64_f8f6f4):
 * x_e4m3 [rows][ldx bytes] per-token E4M3 codes (ldx % 16 == 0) times the
 * MXFP4 weights, y = bf16((acc * a_row_scale[a(r)] + bias) * gammas), products
 * and layouts as af3_moe_gemm.
 *   trans_w 0 (forward): each 16-byte group and its e8m0 byte go to the MFMA
 *   unconverted.  Replaces matmul_ogs(x_fp8, w_fp8_t, ...) with the per-token
 *   PrecisionConfig at quantization.py:331-356 (the reference's E5M2 weights
 *   hold the same values).
 *   trans_w 1 (input gradient, N % 64 == 0): the weights converted to E5M2 in
 *   registers (the reference's mxfp4_to_fp8_e5m2_colmajor values, kernels.py:
 *   238-312, for every scale byte).  Replaces matmul_ogs(grad_fp8, w_fp8, ...)
 *   at quantization.py:382-408.
 * block_m 256, no LoRA; AF3_EUNSUPPORTED when a requirement fails. */
int af3_moe_gemm_f8(const uint8_t* x_e4m3, int64_t ldx, const int32_t* gather_indx, int gather_div,
                    const uint8_t* w_blocks, const uint8_t* w_scales, int trans_w, const float* bias,
                    const void* gammas, int gammas_f32, const int32_t* token_offs, const int32_t* block_pid_map,
                    const int32_t* tile_offs, int max_tiles, int block_m, int tile_cfg, int n_expts, int N, int K,
                    uint16_t* y, int64_t ldy, const float* a_row_scale, void* stream);

/* MXFP4 -> fp8 E5M2, row-major.  Replaces kernels.py:20-108
 * (mxfp4_to_fp8_e5m2_triton): blocks [n_groups][16], scales [n_groups] ->
 * out [n_groups][32] bytes, bit-exact with the reference's int32 rule and its
 * uint16 (lo | hi << 8) stores, also for scale bytes outside the format. */
int af3_mxfp4_to_fp8_e5m2(const uint8_t* blocks, const uint8_t* scales, uint8_t* out, int64_t n_groups,
                          void* stream);

/* MXFP4 [E][N][G][16] -> fp8 E5M2 [E][G*32][N] (N contiguous).  Replaces
 * kernels.py:238-312 (mxfp4_to_fp8_e5m2_colmajor), each value truncated to a
 * byte as its stores do. */
int af3_mxfp4_to_fp8_e5m2_colmajor(const uint8_t* blocks, const uint8_t* scales, uint8_t* out, int E, int N, int G,
                                   void* stream);

/* Per-token dynamic quantization to fp8 E4M3FN.  Replaces kernels.py:319-388
 * (dynamic_quantize_per_token): x [M][ldx] bf16 -> out [M][ld_out] codes and
 * scale [M] fp32 = max(row amax, 1e-12) / 448; codes = E4M3(x * (1 / scale)),
 * round to nearest even, saturating at 448 (IEEE division for both quotients).
 * out_bf16 (optional, [M][ld_bf16]) receives the codes' values as bf16. */
int af3_quantize_per_token_e4m3(const uint16_t* x, int64_t ldx, int64_t M, int K, uint8_t* out, int64_t ld_out,
                                float* scale, uint16_t* out_bf16, int64_t ld_bf16, void* stream);

/* Scatter-sum over each token's K expert rows (the k-reduction matmul_ogs
 * performs for scatter_indx, quantization.py:532-541 and 409-418):
 * out[t] = bf16(sum_j rows[src_indx[t*K+j]]) in fp32; -1 entries skipped. */
int af3_moe_combine(const uint16_t* rows, int64_t ld_rows, const int32_t* src_indx, int64_t n_tokens, int K, int N,
                    uint16_t* out, int64_t ld_out, void* stream);

/* Expert-LoRA skinny row product (no counterpart in the reference, which has
 * no expert LoRA; convention dW = scale * B @ A of model_trainer.py:665,711):
 *   trans_b 0: out[r][j] = scale * sum_k X[a(r)][k] Wl[e][j][k]
 *   trans_b 1: out[r][j] = scale * sum_k X[a(r)][k] Wl[e][k][j]        */
int af3_lora_rows(const uint16_t* x, int64_t ldx, const int32_t* gather_indx, int gather_div, const uint16_t* wl,
                  int trans_b, float scale, const int32_t* token_offs, const int32_t* block_pid_map, int max_tiles,
                  int n_expts, int n_out, int K, uint16_t* out, int64_t ld_out, void* stream);

/* Expert-LoRA weight gradient over each expert's rows (no counterpart in the
 * reference):  G[e][m][n] = scale * sum_{r in rows(e)} bf16(rs(r) A[a(r)][m]) B[b(r)][n]
 * rs = optional bf16 per-row multiplier; G bf16 [E][M][N].  Rows are split
 * into chunk_rows-row chunks (chunk_map / chunk_offs = block_pid_map /
 * token_offs_pad of af3_expt_data for BM = chunk_rows); per-chunk fp32
 * partials go to `partials`, then are summed per expert in chunk order. */
size_t af3_lora_wgrad_workspace_bytes(int max_chunks, int M, int N);
int af3_lora_wgrad(const uint16_t* a, int64_t lda, const int32_t* a_gather, int a_div, const uint16_t* a_rowscale,
                   const uint16_t* b, int64_t ldb, const int32_t* b_gather, int b_div, float scale,
                   const int32_t* token_offs, int n_expts, int M, int N, const int32_t* chunk_map,
                   const int32_t* chunk_offs, int max_chunks, int chunk_rows, float* partials, size_t partial_bytes,
                   uint16_t* g, void* stream);

/* Both expert-LoRA backward products that read the wide gradient, in one pass
 * over it (no counterpart in the reference):
 *   u[i][n]    = bf16(scale_u * sum_k Big[b(i)][k] Bl[e(i)][k][n])        = af3_lora_rows, trans_b 1
 *   G[e][k][n] = bf16(sum_{i in rows(e)} bf16(rs(i) Big[b(i)][k]) Small[i][n]) = af3_lora_wgrad
 * Big [.][ld_big] bf16 (W columns) with rows b(i) = big_gather[i] / big_div
 * (identity when big_gather is NULL), rs = optional bf16 big_rowscale [n_rows],
 * Small [n_rows][r] bf16 compact, Bl [E][W][r], u [n_rows][r], G [E][W][r];
 * r = 16 or 32, W % 8 == 0.  Chunking and the fp32 partial sums follow
 * af3_lora_wgrad; the workspace also holds u's per-column-group partial sums.
 * Rows of u at or past token_offs[n_expts] (entries dropped for an expert id
 * outside [0, E)) are written as zeros.
 * Returns AF3_EUNSUPPORTED (nothing launched) for shapes it does not cover. */
size_t af3_lora_u_wgrad_workspace_bytes(int max_chunks, int64_t n_rows, int W, int r);
int af3_lora_u_wgrad(const uint16_t* big, int64_t ld_big, const int32_t* big_gather, int big_div,
                     const uint16_t* big_rowscale, const uint16_t* small, const uint16_t* bl, float scale_u,
                     const int32_t* token_offs, int n_expts, int64_t n_rows, int W, int r, const int32_t* chunk_map,
                     const int32_t* chunk_offs, int max_chunks, int chunk_rows, void* workspace, size_t ws_bytes,
                     uint16_t* u, uint16_t* g, void* stream);

/* Expert-LoRA merge for weight sync.  The reference merges attention LoRA
 * into bf16 weights for sglang (model_trainer.py:653-719: fp32 base + fp32
 * (B @ A) * scaling, one cast to bf16); this is the same merge for the expert
 * adapters over the MXFP4 weight:
 *   W'[e][n][k] = bf16(float(deq(W[e])[n][k]) + scaling * sum_j B[e][n][j] A[e][j][k])
 * blocks [E][N][K/32][16], scales [E][N][K/32], lora_a [E][r][K], lora_b [E][N][r]
 * (bf16, r % 8 == 0); deq = the rule of af3_mxfp4_to_bf16.  layout 0: out
 * [E][N][K]; layout 1: out [E][K][N] (transformers' GptOssExperts parameter
 * layout, modeling_gpt_oss.py:75-77). */
int af3_mxfp4_lora_merge(const uint8_t* blocks, const uint8_t* scales, const uint16_t* lora_a, const uint16_t* lora_b,
                         float scaling, uint16_t* out, int E, int N, int K, int r, int layout, void* stream);

/* Routing-weight gradient of the down projection.  The reference returns no
 * gradient for gamma (quantization.py:421; forward quantization.py:532-541
 * scales row r by gamma[r]); this computes it for trainable routers:
 *   out[r] = <d_act[r], act[r]> / gammas[r] + <dy[gather[r] / gdiv], bias[e(r)]>
 * d_act = the down projection's input gradient (gamma-scaled) [R][ld_d], act =
 * its input [R][ld_a] (N columns, bf16), dy [.][ld_dy] and bias [E][H] fp32
 * optional (bias == NULL drops the second term), e(r) from token_offs [E+1]
 * (expert-sorted rows), fp32 sums, deterministic. */
int af3_gamma_grad(const uint16_t* d_act, int64_t ld_d, const uint16_t* act, int64_t ld_a, int N, const uint16_t* dy,
                   int64_t ld_dy, const int32_t* gather, int gdiv, const float* bias, int H, const int32_t* token_offs,
                   int n_expts, const uint16_t* gammas, int64_t R, float* out, void* stream);

/* LM-head log-probabilities and entropy without materialised logits.  Replaces
 * the reference's efficient_entropy_forward (trainer/losses/kernels.py:511-700,
 * mainloop 157-292, epilogue 296-385) for reduction "none", one rank:
 * z = hidden [M][ldh] @ weight [V][ldw]^T / temperature (bf16, fp32 accumulation),
 * logprobs = z[label] - lse, entropy = lse - E_p[z]; lse and ez = E_p[z] are kept
 * for the backward.  A label outside [0, V) contributes z = 0.  Workspace:
 * af3_lm_head_workspace_bytes(M, V) bytes (per-tile partials + label logits). */
size_t af3_lm_head_workspace_bytes(int M, int V);
int af3_lm_head_logprobs(const uint16_t* hidden, int64_t ldh, const uint16_t* weight, int64_t ldw, int M, int V, int H,
                         const int64_t* labels, float temperature, float* logprobs, float* entropy, float* lse,
                         float* ez, void* workspace, size_t ws_bytes, void* stream);

/* Logits gradient of the above (the d_logits of trainer/losses/kernels.py:829-839):
 * dz[m][v] = (g[m] (onehot - p) - dentropy[m] p (z - ez[m])) / temperature in bf16,
 * g[m] = dlogprobs[m * dlp_stride] * dlp_scale (stride 0 for a scalar "sum"/"mean"
 * gradient, dlp_scale = 1/M for "mean").  d_hidden = dz @ weight and
 * d_weight = dz^T @ hidden are plain GEMMs left to the caller. */
int af3_lm_head_dlogits(const uint16_t* hidden, int64_t ldh, const uint16_t* weight, int64_t ldw, int M, int V, int H,
                        const int64_t* labels, float temperature, const float* lse, const float* ez,
                        const float* dlogprobs, int64_t dlp_stride, float dlp_scale, const float* dentropy,
                        uint16_t* dz, int64_t lddz, void* stream);

/* The same logits gradient for the vocabulary entries v_begin .. v_begin + v_count - 1
 * only (dz [M][lddz], column j = entry v_begin + j): the per-split d_logits of the
 * reference's default backward, BackwardEnum._Split_Dlogits_N
 * (trainer/losses/kernels.py:1528-1585, kernel 1278-1380), which bounds the
 * gradient buffer to [M][split] and runs the two GEMMs per split. */
int af3_lm_head_dlogits_range(const uint16_t* hidden, int64_t ldh, const uint16_t* weight, int64_t ldw, int M,
                              int v_begin, int v_count, int H, const int64_t* labels, float temperature,
                              const float* lse, const float* ez, const float* dlogprobs, int64_t dlp_stride,
                              float dlp_scale, const float* dentropy, uint16_t* dz, int64_t lddz, void* stream);

/* The forward's statistics when the logits of a vocabulary chunk come from a
 * library GEMM (fp32 output): the per-row softmax partial of the columns
 * v_begin .. v_begin + v_count - 1 of z = logits [M][ldl] / temperature, the
 * online max / sum-exp of the reference's forward kernel (trainer/losses/
 * kernels.py:296-385) over one chunk: partial [M] float4 = (max, sum exp(z -
 * max), sum exp(z - max) z, 0); zlab[m] = z[m][labels[m]] for the rows whose
 * label lies in the chunk (other rows untouched).  af3_lm_head_reduce combines
 * n_parts such partials per row ([n_parts][M] float4) into logprobs, entropy,
 * lse and ez exactly as af3_lm_head_logprobs does (a label outside [0, V)
 * contributes z = 0). */
int af3_lm_head_chunk_stats(const float* logits, int64_t ldl, int M, int v_begin, int v_count, const int64_t* labels,
                            float temperature, void* partial, float* zlab, void* stream);
int af3_lm_head_reduce(const void* partials, int M, int n_parts, const float* zlab, const int64_t* labels, int V,
                       float* logprobs, float* entropy, float* lse, float* ez, void* stream);

/* af3_lm_head_dlogits_range's logits gradient from precomputed fp32 logits of
 * the chunk (logits [M][ldl], column j = entry v_begin + j): the d_logits of
 * trainer/losses/kernels.py:829-839 per split (1528-1585) when a library GEMM
 * recomputed the split's logits. */
int af3_lm_head_dz_chunk(const float* logits, int64_t ldl, int M, int v_begin, int v_count, const int64_t* labels,
                         float temperature, const float* lse, const float* ez, const float* dlogprobs,
                         int64_t dlp_stride, float dlp_scale, const float* dentropy, uint16_t* dz, int64_t lddz,
                         void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AF3_MI355X_H */
