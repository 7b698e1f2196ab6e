/*
 * zonos3_gdn.h -- C ABI of the MI355X (gfx950) gated-DeltaNet kernels.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream (as void*, NULL = the default
 * stream), launches asynchronously on that stream, allocates nothing, never synchronises the host and is
 * therefore capturable into a HIP graph. Return value: ZGDN_OK, or an error code with a message available
 * from zgdn_last_error() (per calling thread).
 *
 * Layouts (all contiguous, row-major, the reference's FLA calling convention):
 *   q, k          [B, T, Hk, K]     v, o  [B, T, Hv, V]     g (log decay), beta  [B, T, Hv]
 *   state         [N, Hv, V, K] float32, value-major ("state_v_first"); N = B, or the number of packed
 *                 sequences when cu_seqlens [N+1] (int32) is given with B == 1.
 * Grouped value heads: v-head h reads k-head h / (Hv / Hk).
 */
#ifndef ZONOS3_GDN_H
#define ZONOS3_GDN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of the tensors handed over. */
enum zgdn_dtype { ZGDN_F32 = 0, ZGDN_BF16 = 1 };

/* Status codes. */
enum zgdn_status { ZGDN_OK = 0, ZGDN_EINVAL = 1, ZGDN_EHIP = 2, ZGDN_EUNSUPPORTED = 3 };

/* Message of the last failed call on this thread ("" after a success). */
const char* zgdn_last_error(void);

/* ABI version of this library (bumped on any signature change). */
int zgdn_abi_version(void);

/*
 * Token-by-token gated delta rule (recurrent form), T >= 1 tokens per sequence; T == 1 is the decode step.
 * Replaces the token loop of model/src/zonos3/reference/lm.py:574-583 (S *= a; p = S.k; d = beta (v - p);
 * S += d k^T; o = S.(q scale)), which the serving layer otherwise recomputes through a 64-row chunk window
 * (servers/sgl/src/zonos3_sgl/models/gdn.py:329-355).
 *   g, beta: dtype gb_dtype (F32 or BF16); g is the log decay (alpha = exp(g)).
 *   initial_state: NULL = zeros. final_state: NULL = not written; may equal initial_state (in place).
 *   o: dtype o_dtype. K must be 64 or 128; V >= 1; Hv % Hk == 0.
 */
int zgdn_recurrent_fwd(const void* q, const void* k, const void* v, int qkv_dtype, const void* g,
                       const void* beta, int gb_dtype, const float* initial_state, float* final_state,
                       void* o, int o_dtype, const int32_t* cu_seqlens, int n_seqs, int B, int T, int Hk,
                       int Hv, int K, int V, float scale, void* stream);

/*
 * Bytes of workspace zgdn_chunk_fwd needs for n_chunks 64-token chunks (over all sequences) and Hv value
 * heads (73,984 bytes per chunk and head).
 */
size_t zgdn_chunk_workspace_size(int n_chunks, int Hv);

/*
 * Chunked (WY/UT form, 64-token chunks) gated delta rule over whole sequences on bf16 MFMA with fp32
 * accumulation: the prefill core. Replaces FLA's chunk_gated_delta_rule_fwd as called at
 * servers/sgl/src/zonos3_sgl/models/gdn.py:418-434 (state_v_first=True, chunk_size=64, output o and the
 * final state), itself the chunked form of model/src/zonos3/reference/lm.py:574-583.
 *   q, k, v: bf16, K == V == 128. o: bf16 [B, T, Hv, V].
 *   g, beta: gb_dtype. With A_log and dt_bias (float32 [Hv], both or neither) g holds the raw gate input a
 *   and the log decay is -exp(A_log[h]) * softplus(a + dt_bias[h]) (FLA use_gate_in_kernel=True,
 *   gdn.py:430-432); otherwise g is the log decay.
 *   cu_seqlens [n_seqs+1] + chunk_indices [n_chunks, 2] (sequence, chunk within it; the table of
 *   gdn.py:49-59) for packed sequences (B == 1); otherwise n_chunks is derived from B and T.
 *   initial_state NULL = zeros; final_state NULL = not written; may equal initial_state (in place).
 *   workspace: device memory of at least zgdn_chunk_workspace_size(n_chunks, Hv) bytes.
 */
int zgdn_chunk_fwd(const void* q, const void* k, const void* v, int qkv_dtype, const void* g, const void* beta,
                   int gb_dtype, const float* A_log, const float* dt_bias, const float* initial_state,
                   float* final_state, void* o, const int32_t* cu_seqlens, const int32_t* chunk_indices,
                   int n_seqs, int n_chunks, int B, int T, int Hk, int Hv, int K, int V, float scale,
                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * One single-token step of the whole GDN block for B independent streams, fused in one launch: depthwise
 * causal conv1d (width W == 4) over the raw q|k|v channels with a rolling history, SiLU, q/k L2-norm, the
 * in-kernel gate, the gated delta-rule state update and the gated RMSNorm of the output. Replaces, for one
 * new row per stream, model/src/zonos3/reference/lm.py:563-587 (and the serving layer's decode path through
 * FLA, servers/sgl/src/zonos3_sgl/models/gdn.py:403-445).
 *   x_qkv [B, C] with C = 2 Hk K + Hv V (q | k | v channels); z [B, Hv, V]; a, b [B, Hv]; conv_weight
 *   [C, W] (tap 0 oldest); norm_weight [V]; out [B, Hv, V]: all of element type `dtype` (F32 or BF16).
 *   conv_cache [B, C, W-1] (same dtype, oldest first) and state [B, Hv, V, K] (float32) are updated in place.
 *   A_log, dt_bias: float32 [Hv]. K == V == 128, Hv / Hk in {1, 2, 4}.
 */
int zgdn_fused_decode_step(const void* x_qkv, const void* z, const void* a, const void* b, int dtype,
                           const void* conv_weight, void* conv_cache, const float* A_log, const float* dt_bias,
                           const void* norm_weight, float* state, void* out, int B, int Hk, int Hv, int K, int V,
                           int W, float eps, float scale, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ZONOS3_GDN_H */
