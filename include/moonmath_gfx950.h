/*
 * C ABI of libmoonmath_gfx950.so -- MI355X (gfx950) bf16 flash-attention
 * forward and fp8-KV absorbed-MLA decode.
 *
 * Conventions (same as the reference's extern "C" launchers):
 *  - every device buffer is caller-owned; the library never allocates;
 *  - launches go on the caller's hipStream_t, passed as void*; no host sync;
 *  - return 0 on success, a positive (attention) or negative (MLA) argument
 *    code, otherwise the hipGetLastError() value of the launch;
 *  - stateless and reentrant (no host statics, no symbol uploads), except
 *    launch_mla_decode_a16w8_paged_dev_noalloc: it caches one device address
 *    per GPU and shares a library-owned device scratch array between its
 *    calls, which callers must serialise per GPU.
 *
 * Each declaration cites the reference interface it replaces
 * (moonmath-ai/amd-kernels, path:line).
 */
#ifndef MOONMATH_GFX950_H
#define MOONMATH_GFX950_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------------
 * Attention forward, head_dim 128, bf16 in/out. layout: 0 = [B,H,S,D] (bhsd),
 * 1 = [B,S,H,D] (bshd). One symbol set per bf16 round mode (rtne/rtna/rtz).
 * ------------------------------------------------------------------------- */

/* V -> V_t, the PV operand order of the forward kernel; V_t holds
 * moonmath_attention_vt_bytes(B, H, Skv) bytes (= B*H*ceil(Skv/64)*64*128 bf16,
 * the reference's V_t size). n_rows = B*H*Skv, seq_len_per_head = Skv.
 * Replaces csrc/attention_api.cpp:18-19 / csrc/attention_kernel.hip:1685-1715. */
int launch_v_transpose_rtne(const void* v, void* v_t, int n_rows, int seq_len_per_head, int heads, int layout,
                            void* stream);
int launch_v_transpose_rtna(const void* v, void* v_t, int n_rows, int seq_len_per_head, int heads, int layout,
                            void* stream);
int launch_v_transpose_rtz(const void* v, void* v_t, int n_rows, int seq_len_per_head, int heads, int layout,
                           void* stream);

/* O = softmax(Q K^T / sqrt(128)) V. workspace: tail KV-split partials of
 * tail_workspace_bytes_<mode>() bytes, or NULL (no split). Codes: 1 B/H <= 0,
 * 2 Sq <= 0, 3 head_dim != 128, 5 Skv <= 0, 7 bad layout, 8 null pointer.
 * Replaces csrc/attention_api.cpp:20-32 / csrc/attention_kernel.hip:1560-1597. */
int launch_attention_forward_rtne(const void* q, const void* k, const void* v_t, void* out, int batch, int heads,
                                  int seq_len, int seq_len_kv, int head_dim, int layout, void* workspace,
                                  void* stream);
int launch_attention_forward_rtna(const void* q, const void* k, const void* v_t, void* out, int batch, int heads,
                                  int seq_len, int seq_len_kv, int head_dim, int layout, void* workspace,
                                  void* stream);
int launch_attention_forward_rtz(const void* q, const void* k, const void* v_t, void* out, int batch, int heads,
                                 int seq_len, int seq_len_kv, int head_dim, int layout, void* workspace,
                                 void* stream);

/* Replaces csrc/attention_api.cpp:123-125 / csrc/attention_kernel.hip:1549-1551. */
size_t tail_workspace_bytes_rtne(void);
size_t tail_workspace_bytes_rtna(void);
size_t tail_workspace_bytes_rtz(void);

/* LiteAttention forward: only the K-blocks named by read_list (int16
 * [B,H,ceil(Sq/256),ceil(Skv/64)+2] run-length rows: len, then (end, start)
 * pairs read from the back, walked ascending when phase != 0, descending
 * otherwise) are computed; write_list (same shape) receives the next step's
 * rows. Each wave of 32 q rows keeps a processed block for its rows when
 * some valid row's block max came within `threshold` (log2) of the row's
 * running max over the blocks the wave kept before, or when it is the first
 * block processed; a block the wave drops adds nothing to its rows. The next
 * list keeps a block some wave kept, or one that must_do_list (int16 [len,
 * s0, e0, ...], end exclusive; nullable) holds. v_t is the output of
 * launch_v_transpose_<mode>.
 * workspace: lite_workspace_bytes_<mode>() bytes for the heaviest-first CTA
 * order, or NULL (plain order). Codes: as the dense launcher, plus 4 (NULL
 * read or write list) and 6 (more than 8192 K-blocks, Skv > 524288).
 * Replaces csrc/attention_api.cpp:67-104 / csrc/attention_kernel.hip:1604-1681. */
int launch_attention_forward_lite_rtne(const void* q, const void* k, const void* v_t, void* out, int batch,
                                       int heads, int seq_len, int seq_len_kv, int head_dim, const void* read_list,
                                       void* write_list, const void* must_do_list, float threshold, int phase,
                                       int layout, void* workspace, void* stream);
int launch_attention_forward_lite_rtna(const void* q, const void* k, const void* v_t, void* out, int batch,
                                       int heads, int seq_len, int seq_len_kv, int head_dim, const void* read_list,
                                       void* write_list, const void* must_do_list, float threshold, int phase,
                                       int layout, void* workspace, void* stream);
int launch_attention_forward_lite_rtz(const void* q, const void* k, const void* v_t, void* out, int batch,
                                      int heads, int seq_len, int seq_len_kv, int head_dim, const void* read_list,
                                      void* write_list, const void* must_do_list, float threshold, int phase,
                                      int layout, void* workspace, void* stream);

/* Bytes of the lite CTA-order workspace: per 256-row q tile and head one int
 * (the order, first) and one byte (its work bucket, after the order).
 * Replaces csrc/attention_kernel.hip:1554-1558. */
size_t lite_workspace_bytes_rtne(int batch, int heads, int seq_len);
size_t lite_workspace_bytes_rtna(int batch, int heads, int seq_len);
size_t lite_workspace_bytes_rtz(int batch, int heads, int seq_len);

/* Mode-generic forward (round_mode 0 = RTNE, 1 = RTNA, 2 = RTZ). force_split_ways
 * > 1 forces that KV split on the last round of CTAs (test hook; 0 = planner).
 * Serves the Python wrapper that replaces csrc/attention_api.cpp:152-283. */
int moonmath_attention_forward_ex(const void* q, const void* k, const void* v_t, void* out, int batch, int heads,
                                  int seq_len, int seq_len_kv, int head_dim, int layout, int round_mode,
                                  void* workspace, int force_split_ways, void* stream);

/* Tail split plan -> out4 = {prefix CTAs, tail, split ways G, parts}. Pure host.
 * Replaces plan_tail_split, csrc/attention_kernel.hip:1349-1393. */
int moonmath_attention_plan_tail(int batch, int heads, int seq_len, int seq_len_kv, int enable, int force_split_ways,
                                 int* out4);

/* out4 = {q rows per CTA, kv rows per block, CTA slots on the device, max parts}. */
int moonmath_attention_geometry(int* out4);

/* Bytes of V_t for (B, H, Skv). */
size_t moonmath_attention_vt_bytes(int batch, int heads, int seq_len_kv);

/* ---------------------------------------------------------------------------
 * Absorbed-MLA decode: bf16 q_lat [.., 512] / q_pe [.., 64], fused fp8 OCP
 * e4m3fn KV rows of 576 bytes, per-tensor kv_scale, bf16 o_lat written in
 * place. H in [1,128], q_len in [1,8]. Codes: -2 lat/rope dims, -3 H,
 * -4 q_len or B, -6 null pointer, -7 S < 1, -8 grid overflow, -9 split
 * records beyond the allocation-free entry point's array, -10 no device
 * address for that array, -11 bad block-table geometry.
 * ------------------------------------------------------------------------- */

/* Fixed split-workspace cap in bytes. Replaces csrc/mla_decode_a16w8.hip:178-181. */
size_t mla_decode_a16w8_workspace_bytes(void);

/* Exact split workspace for (B, H, parts, q_len). Replaces
 * csrc/mla_decode_a16w8_multiq_api.cpp:22-34 (workspace_for). */
size_t mla_decode_a16w8_multiq_workspace_for(int B, int H, int parts, int q_len);

/* Contiguous [B,S,576] slab, q_len 1. k_pe and scale_p are unused (ABI).
 * Replaces csrc/mla_decode_a16w8.hip:784-809. */
int launch_mla_decode_a16w8(const void* q_lat, const void* q_pe, const void* c_kv, const void* k_pe, void* o_lat,
                            int B, int H, int S, int lat_dim, int rope_dim, float scale, float kv_scale,
                            float scale_p, void* workspace, void* stream);

/* Paged pool [slots,576]; request b owns kv_indices[kv_indptr[b] ..
 * kv_indptr[b] + seq_lens[b]); rows[B] (nullable) maps request -> q/out row;
 * parts fixed by the caller. kv_bytes is accepted for ABI parity.
 * Replaces csrc/mla_decode_a16w8.hip:813-844. */
int launch_mla_decode_a16w8_paged_dev(const void* q_lat, const void* q_pe, const void* kv_pool, void* o_lat,
                                      const void* seq_lens, const void* rows, const void* kv_indices,
                                      const void* kv_indptr, int B, int H, int parts, int lat_dim, int rope_dim,
                                      float scale, float kv_scale, float scale_p, void* workspace, void* stream,
                                      size_t kv_bytes, int q_len);

/* Allocation-free variant of launch_mla_decode_a16w8_paged_dev (same arguments
 * and results, q_len 1..8, no workspace argument). No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops that forbid hipMalloc). The split records
 * live in a 64.3 MiB device array of the library (held on each GPU the library
 * runs on until the process ends); the call performs no allocation. Limit:
 * B * parts * R <= 32768 split-record rows once parts is clamped as in the
 * workspace launcher (parts 1 needs none), R = H * q_len, rounded up to a
 * multiple of 32 when 96 <= H * q_len <= 128; else returns -9 with nothing
 * launched. Calls that overlap on one GPU share the array and race: serialise
 * them (one stream, or events). */
int launch_mla_decode_a16w8_paged_dev_noalloc(const void* q_lat, const void* q_pe, const void* kv_pool, void* o_lat,
                                              const void* seq_lens, const void* rows, const void* kv_indices,
                                              const void* kv_indptr, int B, int H, int parts, int lat_dim,
                                              int rope_dim, float scale, float kv_scale, float scale_p, void* stream,
                                              size_t kv_bytes, int q_len);

/* Paged decode over 64-token block tables: kv_pool holds num_blocks pages of
 * 64 fused 576-byte rows; request b's token t lives in page
 * block_table[b * max_blocks + t / 64], row t % 64; q_len 1..8 as in
 * launch_mla_decode_a16w8_paged_dev (rows, parts, workspace likewise).
 * index_workspace: mla_decode_a16w8_blocks_index_bytes(B, max_blocks) bytes
 * into which the table is expanded to per-token slots (page ids clamped to
 * [0, num_blocks), lengths to [0, max_blocks * 64]) before the decode, on the
 * same stream. Codes: as the paged launcher, plus -11 (max_blocks or
 * num_blocks < 1, or tables beyond int32 indexing). No counterpart in the
 * reference, whose decode takes flat per-token slots only: this is the
 * block-table form a serving stack's paged KV cache keeps. */
size_t mla_decode_a16w8_blocks_index_bytes(int B, int max_blocks);
int launch_mla_decode_a16w8_paged_blocks_dev(const void* q_lat, const void* q_pe, const void* kv_pool, void* o_lat,
                                             const void* seq_lens, const void* rows, const void* block_table,
                                             int max_blocks, int num_blocks, int B, int H, int parts, int q_len,
                                             int lat_dim, int rope_dim, float scale, float kv_scale, float scale_p,
                                             void* workspace, void* index_workspace, void* stream);

/* Multi-query (draft window) contiguous decode. Replaces
 * csrc/mla_decode_a16w8_multiq.hip:955-983. */
int launch_mla_decode_a16w8_multiq(const void* q_lat, const void* q_pe, const void* kv, void* o_lat, int B, int H,
                                   int S, int q_len, int lat_dim, int rope_dim, float scale, float kv_scale,
                                   void* workspace, void* stream);

/* Multi-query paged decode. Replaces csrc/mla_decode_a16w8_multiq.hip:984-1001. */
int launch_mla_decode_a16w8_multiq_paged_dev(const void* q_lat, const void* q_pe, const void* kv_pool, void* o_lat,
                                             const void* seq_lens, const void* rows, const void* kv_indices,
                                             const void* kv_indptr, int B, int H, int parts, int q_len,
                                             int lat_dim, int rope_dim, float scale, float kv_scale,
                                             void* workspace, void* stream, size_t kv_bytes);

/* Split planners (pure host). Replace csrc/mla_decode_a16w8.hip:846-876 and
 * csrc/mla_decode_a16w8_multiq.hip:870-894. */
int mla_decode_a16w8_plan_parts(int B, int H, int max_seq_len, int lat_dim);
int mla_decode_a16w8_plan_parts_q(int B, int max_seq_len, int q_len, int H);
int mla_decode_a16w8_plan_parts_capped(int B, int H, int max_seq_len, int lat_dim);
int mla_decode_a16w8_multiq_plan_parts_q(int B, int max_seq_len, int q_len, int H);
/* Replaces csrc/mla_decode_a16w8.hip:866 (mla_decode_a16w8_max_ctas). */
int mla_decode_a16w8_max_ctas(void);

/* The parts value a launcher will use for (B, H, parts, q_len) given a
 * workspace (have_workspace != 0) or none. */
int moonmath_mla_effective_parts(int B, int H, int parts, int q_len, int have_workspace);

/* fp8 KV producer: for each token i < n_tokens with 0 <= slots[i] < num_slots,
 * writes row slots[i] of kv_pool ([num_slots, 576] bytes) as
 * e4m3fn(fl32(x / kv_scale)) of c_kv[i, 0:512] then k_pe[i, 0:64] (bf16,
 * contiguous [n, 512] and [n, 64]); round to nearest even, |x| > 464 -> NaN
 * (saturate == 0, torch's float8_e4m3fn cast) or +-448 (saturate != 0).
 * Other rows are not touched (slot -1 marks a padding token). Codes: -4
 * negative sizes, -6 null pointer, -8 grid overflow, -12 kv_scale not a
 * positive finite number. The reference has no producer; this writes its
 * cache format (moonmath_attention/mla.py:17-20,
 * csrc/mla_decode_a16w8_api.cpp:5-8) the way its tests fill it
 * (tests/test_mla_decode.py:34-38). */
int launch_mla_kv_quantize(const void* c_kv, const void* k_pe, void* kv_pool, const void* slots, long long n_tokens,
                           long long num_slots, float kv_scale, int saturate, void* stream);

/* Test hook: decode n OCP e4m3fn bytes to bf16 bits with the kernel's
 * hardware convert (v_cvt_scalef32_pk_bf16_fp8, scale 1). */
int moonmath_fp8e4m3_to_bf16(const void* in, void* out, int n, void* stream);

/* Test hook: pack n fp32 values (n even) to bf16 bits with the output packing
 * of the attention epilogue, the split-KV merge and the MLA outputs
 * (round_mode 0 RTNE, 1 RTNA, 2 RTZ; every NaN becomes 0x7FFF). The rounding
 * rules are the reference's bf16_round_one (csrc/attention_kernel.hip:110-145). */
int moonmath_pack_bf16(const void* in, void* out, int n, int round_mode, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOONMATH_GFX950_H */
