/* neural_amd: C ABI of the MI355X (gfx950) GPT-OSS-120B MoE hot path.
 *
 * Every entry point takes raw device pointers, plain sizes and the hipStream_t to launch on; it allocates nothing,
 * never synchronises and never reads device data on the host, so it can be recorded into a hipGraph.  Return value:
 * 0 = launched, -1 = invalid arguments (nothing launched), -2 = launch error (hipGetLastError), -3 = a size beyond
 * the kernel's fixed limits (nothing launched), -4 = the device cannot hold every workgroup of a launch that needs
 * them resident together (nothing launched).
 *
 * Data conventions: bf16 tensors are arrays of uint16 bit patterns; expert slots follow the store layout of the
 * reference (neural/moe/layout.py:143-186): gate_codes [5760][90][16] | down_codes [2880][90][16] | scales, with raw
 * (one E8M0 byte per group, 13,219,200 B) or PS4 (46-byte rows: base + 4-bit deltas, 12,839,040 B) scale rows.
 *
 * Each declaration names the reference interface it replaces (file:line under the reference repository).
 */
#ifndef NEURAL_AMD_H
#define NEURAL_AMD_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Library ABI version (1). */
int na_version(void);

/* Device self-check of the E2M1 -> bf16 conversion the kernels use: out = 768 uint16 (see csrc/abi.hip). */
int na_selftest_fp4(void* out, hipStream_t stream);

/* Decode GEMV over expert slots.  Replaces neural/q80/mxfp4_kernels.py:474-489 (mxfp4_gemv) and, with `active`,
 * :542-569 (mxfp4_gemv_masked).
 *   x        bf16 [1, K] (per_expert_x = 0) or [E, K] (per_expert_x = 1), K = 2880
 *   blocks   u8 view [cap, N, 90, 16] with slot stride sb_slot bytes (rows contiguous)
 *   scales   u8 view [cap, N, 90] (packed = 0) or [cap, N, 46] (packed = 1), slot stride ss_slot bytes
 *   slots    int64 [E] physical slot of each output row block
 *   active   optional per-slot weight (active_dtype 1 = bf16, 2 = fp32, 0 = none): a zero writes +0 rows and reads
 *            no weights; NaN or nonzero computes
 *   out      bf16 [E, N], N even
 *   pairs_per_wave  row pairs streamed per wavefront: 1, 2 or 4 (<= 0: default 2)
 *   events   NULL, or two hipEvent_t that the dispatch stamps at its start and end (measurement only) */
int na_mxfp4_gemv(const void* x, int per_expert_x, const void* blocks, long long sb_slot, const void* scales,
                  long long ss_slot, int packed, const int64_t* slots, int E, const void* active, int active_dtype,
                  void* out, int N, int K, int pairs_per_wave, void* const* events, hipStream_t stream);

/* Fused decode expert body for B <= 8 tokens: gate_up GEMV (+ bias, clamped SwiGLU), down GEMV (+ bias, x routing
 * weight) and, when `out` is not NULL, the top-k combine; three launches.  Replaces the reference's b_body
 * (server.py:508-518: gate_up GEMV -> + bias -> clamped SwiGLU (neural/q80/expert_runtime.py:63-72) -> down GEMV ->
 * + bias -> routing-weighted sum) and its graph twin _ExpertGraphV4._compute (neural/q80/expert_runtime.py:1361-1427),
 * for an all-resident pool.
 *   x          bf16 [B, 2880] (post-attention RMSNorm output)
 *   topk_ids   int64 [B, 4] expert ids within the layer; topk_w bf16 [B, 4] routing weights.  Ids outside [0, 128)
 *              contribute +0 and read no weights.
 *   pool       u8 [n_slots, slot_bytes]; slot of expert id e = slot_tab ? slot_tab[expert_base + e] : expert_base + e
 *   bias_gu    bf16 [*, 5760] / bias_dn bf16 [*, 2880] rows indexed by expert_base + e (NULL = no bias)
 *   h_scratch  bf16 [4B, 2880]: activations; yw_scratch bf16 [4B, 2880]: weighted expert outputs, row 4b + k
 *   out        bf16 [B, 2880] = bf16(sum_k fp32(yw[4b + k])) in top-k order, or NULL to leave the combine to the
 *              consumer (yw_scratch then holds the result).  Calls that overlap on one device must not share scratch.
 *   alpha, limit  activation constants (1.702, 7.0)
 *   gu_pairs_per_wave / dn_pairs_per_wave  row pairs streamed per wavefront, 1, 2 or 4 (<= 0: defaults 4 / 2)
 *   events     NULL, or 6 hipEvent_t: start/stop of the gate_up, down and combine kernels, timestamped by the
 *              dispatches themselves (hipExtLaunchKernel); for measurement only, not for graph capture
 * Each distinct expert's weights are read once per call for all tokens routed to it. */
int na_moe_decode(const void* x, const int64_t* topk_ids, const void* topk_w, int B, const void* pool,
                  long long slot_bytes, int packed, const int64_t* slot_tab, long long expert_base,
                  const void* bias_gu, const void* bias_dn, void* h_scratch, void* yw_scratch, void* out, float alpha,
                  float limit, int gu_pairs_per_wave, int dn_pairs_per_wave, void* const* events, hipStream_t stream);

/* Router GEMV + top-4 + softmax.  Replaces fused_core.py:417-441 (k_router, logits part) and :460-486 (k_topk,
 * selection and weights; the slot-table and host-pack bookkeeping of the offload design are not part of it).
 *   xn bf16 [B, 2880], w_router bf16 [n_exp, 2880], b_router bf16 [n_exp] or NULL, n_exp <= 128
 *   logits fp32 [B, n_exp] scratch; counter: one uint32 that must be 0 before the first call (left at 0)
 *   ids_out int64 [B, 4], w_out bf16 [B, 4] */
int na_router_topk(const void* xn, int B, const void* w_router, const void* b_router, int n_exp, float* logits,
                   unsigned int* counter, int64_t* ids_out, void* w_out, hipStream_t stream);

/* Device self-check of the fp32 -> bf16 rounding the kernels use (gfx950 v_cvt_pk_bf16_f32, single and paired)
 * against an integer round-to-nearest-even: n floats in, three uint16 [n] outputs (hardware, hardware pair, integer). */
int na_selftest_bf16(const float* in, void* out_hw, void* out_pk, void* out_int, long long n, hipStream_t stream);

/* Device self-check of the MFMA operand layout the tile kernels use: d [16, 16] fp32 = a [16, 32] x b [32, 16] bf16. */
int na_selftest_mfma(const void* a, const void* b, float* d, hipStream_t stream);

/* Device self-checks of the t950 decode kernels' arithmetic (no reference counterpart): the activation quantiser
 * (rows x 2880 bf16 -> hi, lo E4M3 codes [rows][2880] and E8M0 bytes sc [rows][2][90]) and one block-scaled MFMA
 * in the kernels' operand order (a: E4M3 [16][128], sa: E8M0 [16][4], tile: one full t950 k-tile of 1024 bytes,
 * sb: E8M0 [16][4] per output row and group; d: fp32 [16][16]). */
int na_selftest_x8(const void* in, int rows, void* hi, void* lo, void* sc, hipStream_t stream);
int na_selftest_mfma8(const void* a, const void* sa, const void* tile, const void* sb, float* d, hipStream_t stream);

/* Matrix-core rate probe (measurement only; no reference counterpart): `blocks` workgroups of 4 waves, each wave
 * running `iters` x 4 independent MFMAs on register operands: kind 0 the block-scaled v_mfma_scale_f32_16x16x128_f8f6f4
 * (E4M3 x E2M1, 65,536 flops each), kind 1 v_mfma_f32_16x16x32_bf16 (16,384 flops each).  out: float [4 blocks].
 * events: NULL or 2 hipEvent_t timestamped by the dispatch. */
int na_bench_mfma_rate(int kind, int blocks, int iters, float* out, void* const* events, hipStream_t stream);

/* ---- gfx950 tile layout ("t950", weight_repr "mxfp4_g32_t950").  No counterpart in the reference's store; it is
 * this build's resident layout, a lossless permutation of the reference's slot (neural/moe/layout.py:143-186,
 * tools/scale_pack.py:6-12): 540 blocks of 16 rows, each 22.5 KiB of codes group-major (byte 256 g + 16 n + b = code
 * byte b of row n, group g: one 16-byte load per lane of a 1024-byte k-tile is the FP4 B operand of
 * v_mfma_scale_f32_16x16x128_f8f6f4) followed by 16 x 96-byte E8M0 scale rows.  13,271,040 bytes per slot. */
long long na_t950_slot_bytes(void);

/* Repack n_slots store slots (raw, or PS4 with src_ps4 = 1; row stride src_stride) into t950 (row stride dst_stride).
 * Replaces the role of the reference's offline store converters tools/pack_store.py / tools/build_store.py for the
 * GPU-resident layout: lossless, src and dst must not overlap. */
int na_repack_to_t950(const void* src, long long src_stride, int src_ps4, void* dst, long long dst_stride,
                      int n_slots, hipStream_t stream);

/* Inverse of na_repack_to_t950: t950 -> raw (dst_ps4 = 0) or canonical PS4 (dst_ps4 = 1: base = row minimum, the
 * encoding of tools/scale_pack.py:49-64). */
int na_repack_from_t950(const void* src, long long src_stride, void* dst, long long dst_stride, int dst_ps4,
                        int n_slots, hipStream_t stream);

/* na_moe_decode over a t950 pool (slot_bytes >= 13,271,040, 16-byte aligned): the same contract as na_moe_decode
 * (server.py:508-518), computed with the block-scaled v_mfma_scale_f32_16x16x128_f8f6f4: the E2M1 codes and E8M0
 * scales as stored, the activations as two E4M3 rows (hi + lo) with one E8M0 scale per 32-element block, which hold
 * every bf16 element exactly down to 2^-13 of its block's largest magnitude (fp32 accumulation as the reference's).
 * k_split = waves per workgroup splitting K in the expert-major kernels (4 or 8; <= 0: 4).
 * down_mode 0: for B = 1 with an output, two launches: gate_up, then one down workgroup per 16 output rows that
 *   holds every distinct expert of the token and sums the top-k outputs itself (events = 4: gate_up, down);
 *   otherwise as down_mode 1.
 * down_mode 1: three launches: gate_up, expert-major down, combine (events = 6). */
int na_moe_decode_t950(const void* x, const int64_t* topk_ids, const void* topk_w, int B, const void* pool,
                       long long slot_bytes, const int64_t* slot_tab, long long expert_base, const void* bias_gu,
                       const void* bias_dn, void* h_scratch, void* yw_scratch, void* out, float alpha, float limit,
                       int k_split, int down_mode, void* const* events, hipStream_t stream);

/* Words (uint32) of the sync buffer na_moe_decode_t950_one needs (95,488 bytes). */
long long na_moe_one_sync_words(void);

/* The expert body of one token (B = 1) over a t950 pool in a single launch: the same contract and the same bits as
 * na_moe_decode_t950 (server.py:508-518, b_body; seam neural/moe/gptoss_adapter.py:267-284), out required.  720
 * workgroups each run one (expert, 16-row block) of gate_up and write their h as tagged words (a 32-bit payload and
 * the launch's number per 64-bit word), load the matching down row block, read their expert's h row once it carries
 * the launch's number, run the down block and write its weighted outputs the same way; one workgroup of each output
 * block sums the top-k.  h_scratch and yw_scratch are not used (NULL allowed): h and the weighted outputs live in
 * sync.  sync: na_moe_one_sync_words uint32, zero before the first call, owned by one stream (calls that overlap on
 * one sync buffer race); word 0 (a wait that gave up) stays set once raised.  Returns -4 where the device cannot hold
 * the 720 workgroups at once.  events: NULL or 2 recorded events (the launch's start and stop). */
int na_moe_decode_t950_one(const void* x, const int64_t* topk_ids, const void* topk_w, const void* pool,
                           long long slot_bytes, const int64_t* slot_tab, long long expert_base, const void* bias_gu,
                           const void* bias_dn, void* h_scratch, void* yw_scratch, void* out, float alpha,
                           float limit, unsigned int* sync, void* const* events, hipStream_t stream);

/* na_moe_decode_t950_one routed by the layer's 128 router logits instead of ids and weights (the router's output
 * in the reference's decode core, fused_core.py:417-502, before k_topk): every workgroup selects the top 4 and their
 * softmax weights itself with the router's own rule (largest bf16 value first, lowest index on ties; weights
 * bf16(exp(v_k - v_0) / sum)), so the selection costs no separate step between the router and the expert body.
 * logits: fp32 [128] (bf16 values, as the router rounds them).  ids_out (int64 [4]) and wts_out (bf16 [4]) receive
 * the selection when given (both or neither).  Otherwise the contract of na_moe_decode_t950_one, on the same sync
 * buffer layout; the same bits as na_moe_decode_t950_one given the router's ids and weights. */
int na_moe_decode_t950_one_logits(const void* x, const float* logits, int64_t* ids_out, void* wts_out,
                                  const void* pool, long long slot_bytes, const int64_t* slot_tab,
                                  long long expert_base, const void* bias_gu, const void* bias_dn, void* out,
                                  float alpha, float limit, unsigned int* sync, void* const* events,
                                  hipStream_t stream);

/* 1 when the current device holds the single-launch expert body's 720 workgroups at once (both forms), else 0:
 * the condition under which na_moe_decode_t950_one(_logits) launch instead of returning -4. */
int na_moe_one_resident(void);

/* na_moe_decode_t950 that allocates nothing and takes no scratch: h and the weighted expert outputs live in a
 * file-scope device array of the library (368,640 bytes per device, for B <= 8; its address is looked up once per
 * device on the first call there, with that device current).  No counterpart in the reference: it is for callers
 * that cannot allocate or pass a workspace (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  out must not be NULL; B > 8 returns -3.  Every call on a device shares the array and leaves its last
 * contents there: calls that overlap on one device (two streams, two threads) race.  Results equal
 * na_moe_decode_t950's bit for bit. */
int na_moe_decode_t950_noalloc(const void* x, const int64_t* topk_ids, const void* topk_w, int B, const void* pool,
                               long long slot_bytes, const int64_t* slot_tab, long long expert_base,
                               const void* bias_gu, const void* bias_dn, void* out, float alpha, float limit,
                               int k_split, int down_mode, hipStream_t stream);

/* ---- decode attention (GQA 64 query / 8 KV heads, head_dim 64, learned sinks, sliding window, rolling cache) */

/* Floats of workspace na_decode_attention needs for B sequences and n_split chunks (-1 if out of range). */
long long na_attn_workspace_floats(int B, int n_split);

/* Decode attention of B sequences, one query each.  Replaces fused_core.py:145-208 (k_attn, n_split = 1) and
 * :211-382 (SplitAttn, k_attn_s1..s4, n_split > 1), entry :385-398 (decode_attention).
 *   q        bf16 [B, 64 * 64] (RoPE applied); sinks bf16 [64]
 *   kc, vc   bf16 [B, 8, cache_rows, 64]; key position j in row j, or j % ring when ring > 0 (then cache_rows == ring
 *            and window > 0, ring >= window)
 *   pos      int64 [B] on the device: attended keys [lo, pos], lo = max(pos - window + 1, 0) (window = 0: lo = 0)
 *   out      bf16 [B, 64 * 64]
 *   n_split  chunks per (sequence, KV head), 1..64; n_split > 1 needs work (na_attn_workspace_floats floats) and
 *            counters (uint32 [B * 8], zero before the first call; every completed call leaves them zero).  Calls
 *            sharing work/counters must not overlap.
 *   events   NULL or 2 hipEvent_t (start/stop of the launch, timestamped by the dispatch) */
int na_decode_attention(const void* q, const void* kc, const void* vc, long long cache_rows, const void* sinks,
                        const int64_t* pos, void* out, int B, float scaling, int window, int ring, int n_split,
                        float* work, unsigned int* counters, void* const* events, hipStream_t stream);

/* Prompt attention of T tokens at positions p0 .. p0+T-1 (causal, sliding window when window > 0, learned sinks).
 * Replaces fused_core.py:684-759 (k_prefill_attn), entry :762-784 (prefill_attention).
 *   q        bf16 [T, 64, 64] (RoPE applied), contiguous; out bf16 [T, 64, 64]; sinks bf16 [64]
 *   ring = 0 kc, vc bf16 [8, cache_rows, 64] already holding positions < p0 + T (p0 + T <= cache_rows); k_new/v_new
 *            unused
 *   ring > 0 (window > 0, ring >= window, cache_rows == ring) kc, vc are the rolling cache holding positions
 *            p0-ring .. p0-1 in rows j % ring; k_new, v_new bf16 [T, 8, 64] with element strides (sk_t, sk_h) and
 *            (sv_t, sv_h), multiples of 8, last dimension contiguous, are the block's own K / V.  The ring is not
 *            updated: call na_ring_write after the attention.
 *   events   NULL or 2 hipEvent_t (start/stop of the launch)
 * Ring and linear mode give bit-identical outputs for the same key values.  T = 0 launches nothing and returns 0
 * (the pointers of an empty prompt may be NULL). */
int na_prefill_attention(const void* q, const void* kc, const void* vc, long long cache_rows, const void* k_new,
                         const void* v_new, long long sk_t, long long sk_h, long long sv_t, long long sv_h,
                         const void* sinks, void* out, long long p0, int T, float scaling, int window, int ring,
                         void* const* events, hipStream_t stream);

/* The last min(T, ring) positions of a block (K / V rows [T, 8, 64] with element strides as above) into their ring
 * slots position % ring of kc, vc [8, ring, 64].  Replaces fused_core.py:787-800 (ring_write). */
int na_ring_write(void* kc, void* vc, int ring, const void* k_new, const void* v_new, long long sk_t, long long sk_h,
                  long long sv_t, long long sv_h, long long p0, int T, hipStream_t stream);

/* ---- prefill (prompt) products */

/* out[e][m][n] = bf16(sum_k x[m][k] w_e[n][k]) for e < E (weights of slot slots[e]), m < M.  Replaces
 * neural/q80/mxfp4_kernels.py:202-231 (mxfp4_gemm / mxfp4_gemm_into; any E and M).
 *   x        bf16 [M, K], K = 2880 (16-byte aligned rows)
 *   blocks   layout 0 (raw) / 1 (PS4): u8 view [cap, N, 90, 16], slot stride sb_slot; scales [cap, N, 90 | 46] with
 *            slot stride ss_slot.  layout 2: blocks = the matrix's first t950 row block of slot 0, stride sb_slot.
 *   out      bf16 [E, M, N], N a multiple of 192 */
int na_mxfp4_gemm(const void* x, int M, int K, const void* blocks, long long sb_slot, const void* scales,
                  long long ss_slot, int layout, const int64_t* slots, int E, void* out, int N, hipStream_t stream);

/* One ragged GEMM launch over GroupedGemmPlan tile descriptors.  Replaces mxfp4_kernels.py:242-295 and :385-419.
 *   tiles    int64 [ntiles][5] = (x address, out address, slot, pair rows M, tile pm): rows [pm * block_m,
 *            min(M, (pm + 1) * block_m)) of the pair; x rows K = 2880 bf16, out rows N bf16 (16-byte aligned)
 *   block_m  power of two >= 16; N a multiple of 192 */
int na_mxfp4_gemm_grouped(const void* blocks, long long sb_slot, const void* scales, long long ss_slot, int layout,
                          const int64_t* tiles, int ntiles, int block_m, int N, int K, hipStream_t stream);

/* Bytes of workspace na_moe_prefill needs for T tokens (-1 if out of range): about 53 KB per token (the quantised
 * x rows, the quantised h and the bf16 outputs of the 4 T pairs, the order and the tile table). */
long long na_moe_prefill_workspace_bytes(int T);

/* Where na_moe_prefill keeps its routing tables inside the workspace of T tokens (no counterpart in the reference,
 * whose routing tables are torch tensors: server.py:2246-2254 stable argsort, bincount; mxfp4_kernels.py:298-315
 * tile rows).  offsets (9 values) <- byte offsets of counts (int32 [128]: pairs per expert), ntiles (int32 [1]),
 * order (int32 [4 T]: pair indices p = 4 t + k sorted by expert, stable in p; the first sum(counts) entries are
 * valid), tiles (int32 [max_tiles][4] = (expert, first sorted position, rows <= 64, 0), ntiles valid), the quantised
 * x rows, the quantised h rows, the bf16 pair outputs, then the total bytes and max_tiles.  For tests and tools that
 * inspect the routing of a call; returns 0, or -1 for T outside [1, 2^20]. */
int na_moe_prefill_workspace_layout(int T, long long* offsets);

/* One MoE layer over T prompt tokens, all experts resident.  Replaces server.py:1837-1936 (moe_prefill) with the
 * expert products of _expert_gemms :1977-2040 for resident experts; five launches: pair counts (with x quantised
 * into exact E4M3 hi + lo rows), stable expert order + 64-token tiles, gate_up + bias + clamped SwiGLU on the
 * block-scaled FP8 x FP4 MFMA (h out as E4M3 hi + lo rows), down + bias + routing weight, top-k sum.
 *   x [T, 2880] bf16; topk_ids int64 [T, 4] (ids outside [0, 128) contribute +0); topk_w bf16 [T, 4]
 *   pool / slot_bytes / slot_tab / expert_base / biases as na_moe_decode; layout 0 raw, 1 PS4, 2 t950
 *   workspace: na_moe_prefill_workspace_bytes(T) bytes, 16-byte aligned
 *   out [T, 2880] bf16 = bf16(sum_k fp32(yw[t, k])) in top-k order
 *   events  NULL or 10 hipEvent_t (start/stop of the five launches) */
int na_moe_prefill(const void* x, const int64_t* topk_ids, const void* topk_w, int T, const void* pool,
                   long long slot_bytes, int layout, const int64_t* slot_tab, long long expert_base,
                   const void* bias_gu, const void* bias_dn, void* workspace, long long ws_bytes, void* out,
                   float alpha, float limit, void* const* events, hipStream_t stream);

/* ---- dense decode core of one token (bf16 weights; rounding points of the reference's eager core,
 *      neural/moe/gptoss_core_graphs.py:55-109, and of its fused twin fused_core.py) */

/* mid = embed[seq[*pos]] (seq[0] when pos is NULL); the position is clamped into [0, seq_len), the id into
 * [0, vocab).  Replaces the embedding lookup ahead of the layer loop (gptoss_core_graphs.py:113-140 embeds on the
 * host; here the id stays on the device).
 *   emb bf16 [vocab, 2880]; seq int64 [seq_len]; pos int64 [1] or NULL; mid bf16 [2880] */
int na_core_embed(const void* emb, long long vocab, const int64_t* seq, long long seq_len, const int64_t* pos,
                  void* mid, hipStream_t stream);

/* Residual combine + input RMSNorm + fused Q|K|V GEMV + bias + YaRN RoPE + K/V cache write.  Replaces
 * fused_core.py:72-142 (_combine, k_qkv).
 *   x = mid (g NULL: first layer) or bf16(mid + bf16(g + bf16(c))) (c fp32 [2880] or NULL = 0; g bf16 [2880]);
 *   xbuf bf16 [2880] <- x; in_w bf16 [2880]; W bf16 [5120, 2880] (q 4096 | k 512 | v 512 rows); bias bf16 [5120];
 *   pos int64 [1]; inv_freq fp32 [32]; kc, vc bf16 [8, cache_rows, 64]: position pos in row pos, or pos % ring when
 *   ring > 0 (then cache_rows == ring); a row outside [0, cache_rows) is not written; q bf16 [4096] <- RoPE'd
 *   query */
int na_core_qkv(const void* mid, const void* g, const float* c, void* xbuf, const void* in_w, const void* W,
                const void* bias, const int64_t* pos, const float* inv_freq, void* kc, void* vc, long long cache_rows,
                int ring, void* q, float eps, float att_scale, hipStream_t stream);

/* mid = bf16(xbuf + bf16(att . Wo^T + bo)).  Replaces fused_core.py:401-414 (k_oproj).
 *   att bf16 [4096]; Wo bf16 [2880, 4096]; bo, xbuf, mid bf16 [2880] */
int na_core_oproj(const void* att, const void* Wo, const void* bo, const void* xbuf, void* mid, hipStream_t stream);

/* Post-attention RMSNorm + router GEMV + top-4 + softmax, one launch.  Replaces fused_core.py:417-441 (k_router) and
 * :460-502 (k_topk, without the host residency lookup: every expert is resident).
 *   mid bf16 [2880]; post_w bf16 [2880]; Wr bf16 [128, 2880]; br bf16 [128]; hn bf16 [2880] <- normed mid
 *   logits fp32 [128] scratch; counter uint32 [1], zero before the first call (every completed call leaves it zero)
 *   ids int64 [4], wts bf16 [4] <- top-4 by repeated argmax (lowest index on ties), bf16(exp(v - v0) / sum) */
int na_core_router(const void* mid, const void* post_w, float eps, const void* Wr, const void* br, void* hn,
                   float* logits, unsigned int* counter, int64_t* ids, void* wts, hipStream_t stream);

/* The serving bookkeeping of a layer's routing, after na_core_router (one launch).  Replaces the stores of
 * fused_core.py:417-441 (k_router: bx, pack[:H]) and :443-502 (k_topk's _emit and near misses) that feed the expert
 * body and the host.  hn bf16 [2880], ids int64 [4], wts bf16 [4]: na_core_router's outputs; logits fp32 [128]: its
 * logits (needed for near_miss).  slot_tab int64 (NULL: every expert resident at slot base + id), base = layer * 128.
 * Outputs: bx bf16 [2880] <- hn (or NULL); pack fp32 [2880 + 12] (+4 with near_miss, or NULL) <- hn | weights | ids
 * | resident flags (| ids of ranks 5-8); bslots int64 [4] (slot, 0 if not resident), bgids int64 [4] (base + id),
 * bw bf16 [4] (weight, +0 if not resident). */
int na_core_route_pack(const void* hn, const float* logits, const int64_t* ids, const void* wts,
                       const int64_t* slot_tab, long long base, void* bx, float* pack, int near_miss, int64_t* bslots,
                       int64_t* bgids, void* bw, hipStream_t stream);

/* The attention block of one decode layer in ONE launch: na_core_qkv, na_decode_attention (B = 1), na_core_oproj and
 * na_core_router, with their arguments and results (fused_core.py:581-629: k_qkv, k_attn / SplitAttn, k_oproj,
 * k_router + k_topk), as four phases of one grid.  Each phase issues its loads (weights; the cache rows of earlier
 * positions) before it waits for the phase it needs, whose results it reads as tagged words (each 64-bit word a
 * 32-bit payload and the launch's generation number, polled by the reader; bounded waits), so weight streams and
 * cache reads overlap the phases before them.  Differences from the four calls: c and g feed o_proj's residual too
 * (it is recomputed per row, not read from xbuf); mid is updated in place; results are bit-identical.  ids and wts
 * may both be NULL: the block then stops at the router's logits (and hn), leaving the top-4 selection to the expert
 * body that reads them (na_moe_decode_t950_one_logits), which saves the wait for every logit at the block's end.
 *   sync   uint32 [na_core_attn_block_sync_words()] (52,224 bytes: the error word, the generation word, the
 *          attention's split counters, the tagged words of the phases' results and the router's entry count, on
 *          256-byte lines), zero before
 *          the first call and owned by one stream (calls that overlap on one buffer race); every completed call
 *          leaves the counters zero and advances the generation word (uint32 64) by one; word 0 is an error flag that
 *          a wait which gave up after its poll limit raises (and nothing clears): that call's outputs are not
 *          valid.
 *   n_split chunks of the attention (1..64); attn_work: na_attn_workspace_floats(1, n_split) floats (n_split > 1)
 *   events NULL or 2 hipEvent_t (start / stop of the launch) */
long long na_core_attn_block_sync_words(void);
int na_core_attn_block(void* mid, const void* g, const float* c, void* xbuf, const void* in_w, const void* Wqkv,
                       const void* bqkv, const int64_t* pos, const float* inv_freq, void* kc, void* vc,
                       long long cache_rows, int ring, void* q, float eps, float att_scale, const void* sinks,
                       float scaling, int window, int n_split, float* attn_work, void* att, const void* Wo,
                       const void* bo, const void* post_w, const void* Wr, const void* br, void* hn, float* logits,
                       int64_t* ids, void* wts, unsigned int* sync, void* const* events, hipStream_t stream);

/* uint64 entries of the part buffer na_core_lm_tail needs for a vocabulary (-1 if vocab <= 0). */
long long na_core_lm_partials(int vocab);

/* Decode tail: residual combine + final RMSNorm, lm_head GEMV, argmax (first index of the maximum), one launch.
 * Replaces server.py:521-525 (t_body).  Every workgroup forms the final norm itself and streams its share of lm_head's
 * rows; the grid's last workgroup reads every workgroup's best key (tagged words in part) and takes the argmax.
 *   mid, g, c as na_core_qkv; final_w bf16 [2880]; Wl bf16 [vocab, 2880]; hn bf16 [2880] <- the final norm;
 *   logits_out bf16 [vocab] or NULL; part uint64 [na_core_lm_partials(vocab)], 8-byte aligned, any initial contents,
 *   owned by one stream (calls that overlap on one part buffer race); its first uint32 is an error word that a wait
 *   that gave up raises (never cleared by the call); tok int64 [1] <- argmax
 *   pos int64 [1] (p = *pos): pred[p + 1] <- tok (pred int64 [seq_len] or NULL); seq[p + 1] <- tok unless
 *   p + 1 < *n_forced (n_forced int64 [1] or NULL); *pos <- p + 1 when step_pos.  Needs pos for seq/pred/step_pos. */
int na_core_lm_tail(const void* mid, const void* g, const float* c, const void* final_w, float eps, const void* Wl,
                    int vocab, void* hn, void* logits_out, unsigned long long* part, int64_t* tok, int64_t* pos,
                    int step_pos, int64_t* seq, const int64_t* n_forced, int64_t* pred, long long seq_len,
                    hipStream_t stream);

/* na_core_lm_tail with sampling (reference server.py:1576-1583, t_body_sample): when *temp > 0 the token is
 * argmax_v(logit_v / temp + g_v), g_v = -log(-log(clamp(u_v, 1e-12, 1 - 1e-7))) in fp32 (Gumbel-max: a draw from
 * softmax(logits / temp)), first index on ties; when *temp <= 0 it is the greedy argmax of na_core_lm_tail.
 *   temp  fp32 [1] on the device
 *   u     fp32 [vocab] uniform draws in [0, 1) (the reference's u_dev, refreshed by the caller per step), or NULL:
 *         u_v = top 24 bits of splitmix64(splitmix64(*seed ^ p) ^ v) * 2^-24 with p = *pos (the step's input
 *         position), so a captured step draws fresh numbers at every position with no host work
 *   seed  uint64 [1] on the device, or NULL (0) */
int na_core_lm_tail_sample(const void* mid, const void* g, const float* c, const void* final_w, float eps,
                           const void* Wl, int vocab, void* hn, void* logits_out, unsigned long long* part,
                           int64_t* tok, int64_t* pos, int step_pos, int64_t* seq, const int64_t* n_forced,
                           int64_t* pred, long long seq_len, const float* temp, const float* u,
                           const unsigned long long* seed, hipStream_t stream);

/* ---- dense core over T prompt tokens (prefill), one row per workgroup; the GEMMs between them are plain bf16
 *      library GEMMs (hipBLASLt), as the reference's F.linear calls.  Replace the row-wise parts of server.py:2357-2418
 *      (_rope_tables, _rope, _attn_router, _prefill_block) and of neural/moe/gptoss_core_graphs.py:48-53 (_rms). */

/* x [T, 2880] <- embed[ids[t]] (ids int64 [T], clamped into [0, vocab)); the reference's EMB_ROWS(ids). */
int na_rows_embed(const void* emb, long long vocab, const int64_t* ids, int T, void* x, hipStream_t stream);

/* Residual + RMSNorm per row: when add is not NULL, x[t] <- bf16(x[t] + add[t]) in place; hn[t] <- bf16(w * (x[t] *
 * rsqrt(mean(x[t]^2) + eps))).  x, add, hn bf16 [T, 2880]; w bf16 [2880]; 16-byte aligned. */
int na_rows_norm(void* x, const void* add, int T, const void* w, float eps, void* hn, hipStream_t stream);

/* RoPE of qkv [T, 5120] (= F.linear(hn, Wqkv, bqkv)) at positions p0 .. p0+T-1 with cos/sin =
 * bf16(cos(inv_freq[d] pos) * att_scale) (server.py:2357-2364): q [T, 64, 64] <- rotated q heads; the rotated k
 * heads to k_dst + t kt + h kh and the v heads to v_dst + t vt + h vh (element strides: the linear cache rows at p0,
 * or [T, 8, 64] buffers of the block for a rolling cache). */
int na_rows_rope(const void* qkv, int T, long long p0, const float* inv_freq, float att_scale, void* q, void* k_dst,
                 long long kt, long long kh, void* v_dst, long long vt, long long vh, hipStream_t stream);

/* Router selection per row: logits bf16 [T, 128] (= F.linear(hn, Wr, br)) -> ids int64 [T, 4] (top 4 by repeated
 * argmax, lowest index on ties) and wts bf16 [T, 4] (softmax over the four; server.py:2400-2401). */
int na_rows_topk(const void* logits, int T, int64_t* ids, void* wts, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* NEURAL_AMD_H */
