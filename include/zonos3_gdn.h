/*
 * zonos3_gdn.h -- C ABI of the MI355X (gfx950) gated-DeltaNet kernels.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream (as void*, NULL = the default
 * stream), launches asynchronously on that stream, allocates nothing, never synchronises the host and is
 * therefore capturable into a HIP graph. Return value: ZGDN_OK, or an error code with a message available
 * from zgdn_last_error() (per calling thread).
 *
 * Layouts (row-major, the reference's FLA calling convention; contiguous except where an entry point takes
 * row strides):
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
 *   g, beta: dtype gb_dtype (F32 or BF16). Without A_log / dt_bias g is the log decay (alpha = exp(g)); with
 *   them (float32 [Hv], both or neither) g is the raw gate input a and the log decay is
 *   -exp(A_log[h]) * softplus(a + dt_bias[h]) (lm.py:572).
 *   qk_l2norm != 0: q and k are L2-normalised in the kernel, x * rsqrt(sum x^2 + 1e-6) in fp32 (lm.py:570-571).
 *   initial_state: NULL = zeros. final_state: NULL = not written; may equal initial_state (in place).
 *   o: dtype o_dtype. K must be 64 or 128; V >= 1; Hv % Hk == 0.
 */
int zgdn_recurrent_fwd(const void* q, const void* k, const void* v, int qkv_dtype, const void* g,
                       const void* beta, int gb_dtype, const float* A_log, const float* dt_bias, int qk_l2norm,
                       const float* initial_state, float* final_state, void* o, int o_dtype,
                       const int32_t* cu_seqlens, int n_seqs, int B, int T, int Hk, int Hv, int K, int V,
                       float scale, void* stream);

/*
 * Bytes of workspace zgdn_chunk_fwd needs for n_chunks 64-token chunks (over all sequences) and Hv value
 * heads: 98,560 bytes per chunk and head, then the control block of the overlapped launch (11,520 bytes and 4
 * per chunk and head, padded to 256). zgdn_chunk_fwd runs phase 1 (per chunk) and the sequential state pass
 * as two launches; it can run them in one launch, side by side (the overlapped launch: unpacked batches, and
 * packed batches of up to 256 sequences), which measured slower on every shape tried with the present phase 1
 * and is taken only when zgdn_chunk_set_launch_form asks for it (the same results, bit for bit).
 */
size_t zgdn_chunk_workspace_size(int n_chunks, int Hv);

/*
 * Bytes of workspace zgdn_chunk_fwd needs for n_chunks chunks and Hv value heads at head sizes K == V and element
 * type qkv_dtype of q/k/v: zgdn_chunk_workspace_size's for bf16 at K == V == 128; 164,096 bytes (K == 128) or
 * 82,176 bytes (K == 64) per chunk and head on the fp32-arithmetic path (fp32 q/k/v, or K == 64); 0 for a
 * combination zgdn_chunk_fwd does not take. The library's own function, sizing FLA's internal intermediates
 * (chunk_gated_delta_rule_fwd allocates them itself).
 */
size_t zgdn_chunk_workspace_bytes(int n_chunks, int Hv, int K, int V, int qkv_dtype);

/*
 * Launch form of zgdn_chunk_fwd for this process: -1 the library's choice (two launches, above), 0 always
 * phase 1 and the state pass as two launches, 1 the overlapped launch for every eligible batch. The initial value is read once,
 * when the library is loaded, from the environment variable ZGDN_CHUNK_OVERLAP ("0" or "1"; otherwise -1); no
 * call reads the environment. The library's own control, with no counterpart in the reference (FLA picks its
 * launches itself). zgdn_chunk_get_launch_form returns the current value.
 */
int zgdn_chunk_set_launch_form(int form);
int zgdn_chunk_get_launch_form(void);

/*
 * Device status of the chunked path. The overlapped launch's state pass waits for each chunk's phase-1 results
 * with a bounded spin; a wait that runs out (which a correct launch never reaches) sets ZGDN_STATUS_WAIT_GAVE_UP
 * in a sticky per-device status word, lets every kernel end, and leaves o and the final states of that call
 * undefined. zgdn_chunk_status synchronises the current device, stores the word in *status (0 = no error since
 * it was last cleared) and clears it when `clear` is nonzero. It is not a hot-path call: launches stay
 * asynchronous and never read the word. (The reference's FLA launches have no such wait.)
 */
enum { ZGDN_STATUS_WAIT_GAVE_UP = 1 };
int zgdn_chunk_status(int* status, int clear);

/*
 * The same status word without a synchronisation: enqueues on `stream` a copy of the current device's word into
 * *host_status, which must be page-locked host memory (hipHostMalloc, torch's pin_memory=True); the value is
 * there once the stream has passed the copy (an event recorded behind it tells). Does not clear the word. For
 * callers that check their earlier launches from the host without stalling, as the serving layer does before
 * its next call (the reference raises RuntimeError on what it can detect, servers/sgl/src/zonos3_sgl/models/
 * gdn.py:241-272).
 */
int zgdn_chunk_status_async(int* host_status, void* stream);

/*
 * Queues of the overlapped launch for a device of n_cu compute units in n_xcc XCDs (accelerator complex dies,
 * each with its own L2): one queue per XCD, the queue of a workgroup being its XCC_ID register modulo the
 * count, so that a chunk's phase-1 producer and its state-pass consumers share one L2. Returns n_xcc when
 * 1 <= n_xcc <= 8 and the CUs split evenly over the XCDs, else 0 (the overlapped launch is then not taken and
 * zgdn_chunk_fwd runs its two launches). zgdn_chunk_fwd reads n_cu and n_xcc from the device
 * (hipDeviceAttributeMultiprocessorCount, hipDeviceAttributeNumberOfXccs). A host-only function.
 */
int zgdn_chunk_overlap_queues(int n_cu, int n_xcc);

/*
 * Test control of the overlapped launch's waits for this process: `spins` bounds each wait (0 = the default,
 * about a few tenths of a second), and never_ready != 0 makes every wait treat its chunk as not ready, so that
 * each wait runs out after `spins` tries -- the way tests drive the error path of zgdn_chunk_status while
 * every kernel still ends normally. No counterpart in the reference.
 */
int zgdn_chunk_set_wait_limit(int spins, int never_ready);

/*
 * Extra workspace bytes (after zgdn_chunk_workspace_size's) with which zgdn_chunk_fwd runs an unpacked batch of
 * B sequences of T tokens as segments, 0 when it would not. When the sequential state pass would hold at most
 * half the current device's CUs (few sequences and heads) and the sequences are long enough for it to pay
 * (about 48 chunks at one sequence of 4 heads), each sequence is cut into 2 .. 8 segments run at once -- from
 * zero states, and from the identity to obtain each segment's state map -- and their outputs and states are
 * combined (the same results up to rounding). A smaller workspace runs the plain pass.
 */
size_t zgdn_chunk_segment_workspace_size(int B, int T, int Hv);

/*
 * Chunked (WY/UT form, 64-token chunks) gated delta rule over whole sequences: the prefill core. Replaces FLA's
 * chunk_gated_delta_rule_fwd as called at servers/sgl/src/zonos3_sgl/models/gdn.py:418-434 (state_v_first=True,
 * chunk_size=64, output o and the final state), itself the chunked form of
 * model/src/zonos3/reference/lm.py:574-583, in the layer's dtype (lm.py:556-602 runs fp32 or bf16).
 *   q, k, v: element type qkv_dtype (BF16 or F32), K == V, 64 or 128. bf16 at 128 runs on bf16 MFMA with fp32
 *   accumulation (bf16 operands; hi + lo pairs where the state needs them); fp32 inputs, and bf16 at 64, run in
 *   fp32 arithmetic (v_mfma_f32_16x16x4_f32). Rows of [B * T] tokens q_ld / k_ld / v_ld elements apart (a
 *   token's heads contiguous; a multiple of 16 bytes of elements, bases 16-byte aligned), so that q, k, v may be
 *   column slices of one wider row such as the conv output. o: qkv_dtype [B, T, Hv, V] (dense).
 *   g, beta: gb_dtype, rows of Hv values gb_ld elements apart (column slices of the input projection read in
 *   place). With A_log and dt_bias (float32 [Hv], both or neither) g holds the raw gate input a and the log
 *   decay is -exp(A_log[h]) * softplus(a + dt_bias[h]) (FLA use_gate_in_kernel=True, gdn.py:430-432);
 *   otherwise g is the log decay. beta_sigmoid != 0: beta holds the raw input b and the kernel uses
 *   sigmoid(b) (fp32), the value zgdn_sigmoid_fwd would give (FLA fused_beta_sigmoid_fwd, gdn.py:423).
 *   qk_l2norm != 0: q and k are the raw rows and are L2-normalised in the kernel (fp32 factors; the
 *   normalised rows are never rounded to bf16), as lm.py:570-571 does before its fp32 recurrence.
 *   cu_seqlens [n_seqs+1] + chunk_indices [n_chunks, 2] (sequence, chunk within it; the table of
 *   gdn.py:49-59) for packed sequences (B == 1); otherwise n_chunks is derived from B and T.
 *   initial_state NULL = zeros; final_state NULL = not written; may equal initial_state (in place).
 *   workspace: device memory of at least zgdn_chunk_workspace_bytes(n_chunks, Hv, K, V, qkv_dtype) bytes (plus,
 *   on the bf16 path, zgdn_chunk_segment_workspace_size(B, T, Hv) for the segmented pass of unpacked batches).
 */
int zgdn_chunk_fwd(const void* q, const void* k, const void* v, int qkv_dtype, const void* g, const void* beta,
                   int gb_dtype, const float* A_log, const float* dt_bias, int qk_l2norm,
                   const float* initial_state, float* final_state, void* o, const int32_t* cu_seqlens,
                   const int32_t* chunk_indices, int n_seqs, int n_chunks, int B, int T, int Hk, int Hv, int K,
                   int V, long q_ld, long k_ld, long v_ld, long gb_ld, int beta_sigmoid, float scale,
                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * zgdn_chunk_fwd without a workspace argument, for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the reference: FLA's
 * chunk_gated_delta_rule_fwd allocates its own intermediates. Same arguments and layouts as zgdn_chunk_fwd,
 * and the same results as zgdn_chunk_fwd given a workspace of the same size (the same kernels): the
 * segmented state pass of long unpacked prompts is taken only when its extra space fits the scratch as well,
 * else the plain pass, whose results differ from the segmented one's in the last bits (its combine rounds
 * through bf16 hi / lo parts). The caller still passes every input and output. The workspace is the
 * library's own per-device scratch of zgdn_chunk_noalloc_max_bytes() bytes (64 MiB; on the bf16 path 680 chunk x
 * head items, e.g. 4 heads up to 10,880 tokens or 16 heads up to 2,720; 408 items on the fp32 path at K == 128,
 * 816 at K == 64: zgdn_chunk_workspace_bytes sizes them), a static device array held by each device the
 * library runs on until the process ends; calls needing more fail with ZGDN_EINVAL before any launch. Its
 * address is looked up once per device (hipGetSymbolAddress, with the device current), then no call
 * allocates. Every call on one device shares that device's scratch, which keeps the last call's contents (the
 * kernels clear what must start at zero with a fill kernel): calls that overlap on one device, e.g. on two
 * streams, race and must be serialised by the caller.
 */
size_t zgdn_chunk_noalloc_max_bytes(void);
int zgdn_chunk_fwd_noalloc(const void* q, const void* k, const void* v, int qkv_dtype, const void* g,
                           const void* beta, int gb_dtype, const float* A_log, const float* dt_bias, int qk_l2norm,
                           const float* initial_state, float* final_state, void* o, const int32_t* cu_seqlens,
                           const int32_t* chunk_indices, int n_seqs, int n_chunks, int B, int T, int Hk, int Hv,
                           int K, int V, long q_ld, long k_ld, long v_ld, long gb_ld, int beta_sigmoid, float scale,
                           void* stream);

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
 *   qk_round: 0 keeps the L2-normalised q, k in fp32 (lm.py:569-571); nonzero rounds them to `dtype`, as the
 *   serving layer's l2norm operator returns them (gdn.py:416-417).
 */
int zgdn_fused_decode_step(const void* x_qkv, const void* z, const void* a, const void* b, int dtype,
                           const void* conv_weight, void* conv_cache, const float* A_log, const float* dt_bias,
                           const void* norm_weight, float* state, void* out, int B, int Hk, int Hv, int K, int V,
                           int W, float eps, float scale, int qk_round, void* stream);

/*
 * The serving layer's single-row decode step for B requests in table slots, in place on its per-slot caches.
 * Replaces the static decode of servers/sgl/src/zonos3_sgl/models/gdn.py:329-355, which recomputes each
 * request's whole 64-row window through the chunked operators (gdn.py:403-445): here the new row goes
 * through the fused block (zgdn_fused_decode_step's arithmetic) from the slot's live caches.
 *   mixed [B, mixed_ld]: each request's in_proj row, q|k|v (C = 2 Hk K + Hv V) | z (Hv V) | a (Hv) | b (Hv)
 *   (the split of gdn.py:402), mixed_ld >= C + Hv V + 2 Hv; x_hidden [B, hidden]: the raw rows; out
 *   [B, Hv, V]; conv_weight [C, W]; norm_weight [V]: all of element type `dtype`.
 *   slots [B] int64: the requests' table slots (one outside [0, n_slots) is skipped: its caches are not
 *   touched and its out rows are left unwritten; a slot repeated later in the batch, as padded graph replays
 *   repeat a spare slot, is served by its first entry only, the later entries' out rows left unwritten). Per slot (n_slots = cap): conv_live, conv_commit
 *   [cap, C, W] (the last W raw inputs, oldest first, `dtype`); state_live, state_commit [cap, Hv, V, K]
 *   float32; window [cap, window_rows, hidden] (`dtype`); win_len [cap] int32, the real rows in the window.
 *   Updates conv_live and state_live; writes the row into window[slot, win_len]; when the window fills
 *   (win_len + 1 == window_rows) also writes the new conv history and state to conv_commit / state_commit;
 *   then win_len = (win_len + 1) % window_rows. qk_round as in zgdn_fused_decode_step.
 */
int zgdn_serving_decode_step(const void* mixed, long mixed_ld, const void* x_hidden, int hidden, int dtype,
                             const int64_t* slots, int n_slots, int B, int Hk, int Hv, int K, int V, int W,
                             const void* conv_weight, void* conv_live, void* conv_commit, float* state_live,
                             float* state_commit, void* window, int32_t* win_len, int window_rows,
                             const float* A_log, const float* dt_bias, const void* norm_weight, void* out,
                             float eps, float scale, int qk_round, void* stream);

/*
 * Full Attention-Residual routing of the LM's residual bank: out = sum_s softmax_s(rms_norm(x_s) . query) x_s
 * per token, the logits and softmax in fp32. Replaces full_attnres_route of
 * model/src/zonos3/reference/lm.py:384-389 (a list of sources) and of
 * servers/sgl/src/zonos3_sgl/models/zonos3.py:99-113 (a stacked [S, T, dim] bank), without stacking.
 *   sources: host array of n_sources (1..64) device pointers, each to `tokens` rows of `dim` elements spaced
 *   row_stride elements apart (dim a multiple of 8, <= 2048); query [dim]; out [tokens, dim] contiguous; all of
 *   element type `dtype`. eps: the rms_norm eps.
 */
int zgdn_attnres_route(const void* const* sources, int n_sources, int tokens, int dim, long row_stride, int dtype,
                       const void* query, float eps, void* out, void* stream);

/*
 * Depthwise causal conv1d over packed sequences with a rolling history, optional SiLU. Replaces FLA's
 * causal_conv1d_fwd as called at servers/sgl/src/zonos3_sgl/models/gdn.py:403-414, and the conv of
 * model/src/zonos3/reference/lm.py:563-568 (cross-correlation, weight tap 0 oldest).
 *   x, y [B, T, D] (packed: B == 1 with cu_seqlens [n_seqs+1] and chunk_indices [n_chunks, 2] of 64-token
 *   chunks); the rows of x are x_ld >= D elements apart (the q|k|v columns of the input projection are read in
 *   place), y is dense; weight [D, W], bias [D] or NULL; all of element type `dtype`; W <= 4.
 *   State rows [n_seqs, D, state_width], state_width in [W-1, 4]: the raw inputs before the sequence, oldest
 *   first (the last W-1 columns are the taps' history). lm.py keeps [D, W-1] (state_width W-1); the serving
 *   layer keeps [N, D, W] (state_width W). final_state receives the last state_width raw inputs of
 *   [history | x]; it may equal initial_state (in place). NULL initial_state = zeros; NULL final_state =
 *   not written.
 *   activation: 0 none, 1 SiLU. The conv is accumulated in fp32 and rounded to `dtype` before the
 *   activation, the activation's result rounded again (F.conv1d then F.silu on `dtype` tensors).
 */
int zgdn_causal_conv1d_fwd(const void* x, const void* weight, const void* bias, int dtype,
                           const void* initial_state, void* final_state, int state_width, void* y,
                           const int32_t* cu_seqlens, const int32_t* chunk_indices, int n_seqs, int n_chunks,
                           int B, int T, int D, int W, int activation, long x_ld, void* stream);

/*
 * Row-wise L2 norm y = x * rsqrt(sum x^2 + eps), D <= 1024; rstd [rows] (float32) receives the factor when
 * not NULL. Replaces FLA's l2norm_fwd (gdn.py:416-417) and lm.py:570-571 (eps 1e-6).
 *   y: dense [rows, D]. Row r of x starts at x + (r / x_group) * x_ld + (r % x_group) * D, so a token's
 *   x_group heads may sit inside a wider row (q or k of the conv output, read in place); dense x: x_group 1,
 *   x_ld D.
 */
int zgdn_l2norm_fwd(const void* x, int x_dtype, void* y, int y_dtype, float* rstd, int rows, int D, int x_group,
                    long x_ld, float eps, void* stream);

/*
 * y = sigmoid(x) * scale elementwise. Replaces FLA's fused_beta_sigmoid_fwd (gdn.py:423) and the beta of
 * lm.py:573.
 */
int zgdn_sigmoid_fwd(const void* x, int x_dtype, void* y, int y_dtype, size_t n, float scale, void* stream);

/*
 * Gated RMSNorm of the recurrent output, y = (rms_norm(x) * weight).to(dtype) * silu(g), product in fp32 then
 * cast, one row of D <= 1024 at a time; rstd [rows] receives 1/rms when not NULL. Replaces FLA's
 * layer_norm_gated_fwd(activation="swish", is_rms_norm=True) at gdn.py:435-445 and lm.py:584-587.
 *   x, y: dense [rows, D]. Row r's gate starts at g + (r / g_group) * g_ld + (r % g_group) * D, so a token's
 *   g_group per-head gates may sit inside a wider row (z of the input projection, read in place); dense g:
 *   g_group 1, g_ld D.
 */
int zgdn_gated_rmsnorm_fwd(const void* x, const void* g, const void* weight, int dtype, void* y, float* rstd,
                           int rows, int D, int g_group, long g_ld, float eps, void* stream);

/*
 * Bytes of workspace zgdn_accent_shift needs: rows x K rounded up to 32, of bf16 elements (bf16) or floats
 * (fp32).
 */
size_t zgdn_accent_workspace_size(int rows, int out, int K, int dtype);

/*
 * Accent adapter shift of a projection output, y_out = y_in + ((x . down^T) * mask) . up per row: replaces
 * accent_shift / apply_accent of servers/sgl/src/zonos3_sgl/layers/accent.py:25-62 as the GDN mixer applies
 * them to in_proj and wo (servers/sgl/src/zonos3_sgl/models/gdn.py:400-401, 448-449).
 *   x [rows, in] (rows x_ld elements apart), down [K, in], up [K, out], mask [rows, K] (rows mask_ld apart),
 *   y_in / y_out [rows, out] (rows y_in_ld / y_out_ld apart; y_out may equal y_in; y_in NULL = zeros, i.e.
 *   the shift alone): all of element type `dtype`. K <= 256 (the summed ranks of the loaded adapters).
 *   bf16: the reference's rounding points (x . down^T, times mask, . up, the sum with y each rounded to bf16,
 *   products accumulated in fp32); in, out and x_ld multiples of 8, x, down, up 16-byte aligned. fp32: fp32.
 *   Each row is computed independently in a fixed order: a row's bits do not depend on the rest of the call
 *   (the batch invariance accent.py gets from fixed-size row blocks). A zero mask row leaves y exact.
 *   workspace: device memory (16-byte aligned) of at least zgdn_accent_workspace_size(rows, out, K, dtype)
 *   bytes.
 */
int zgdn_accent_shift(const void* x, long x_ld, const void* down, const void* up, const void* mask, long mask_ld,
                      const void* y_in, long y_in_ld, void* y_out, long y_out_ld, int rows, int in, int out, int K,
                      int dtype, void* workspace, size_t workspace_bytes, void* stream);

/*
 * y = x . w^T on bf16 MFMA with fp32 accumulation, rounded to bf16: the GDN layer's projections, in_proj
 * (model/src/zonos3/reference/lm.py:561, servers/sgl/src/zonos3_sgl/models/gdn.py:399) and wo (lm.py:602,
 * gdn.py:447), F.linear without bias.
 *   x [M, K] (rows x_ld elements apart), w [N, K] (dense, the weight as stored), y [M, N] (rows y_ld apart):
 *   bf16 (dtype BF16); K a multiple of 128, N, x_ld and y_ld multiples of 8, 16-byte aligned bases.
 */
int zgdn_gemm_nt(const void* x, long x_ld, const void* w, void* y, long y_ld, int M, int N, int K, int dtype,
                 void* stream);

/*
 * The GDN layer's in_proj with its depthwise causal conv + SiLU fused into the GEMM's epilogue, for one sequence
 * of M rows: y[:, :C] = silu(conv(x . w[:C]^T)) (the conv output the chunked prefill reads q, k, v from), and
 * y[:, C:] = x . w[C:]^T (z | a | b, raw). Replaces F.linear + the conv of model/src/zonos3/reference/lm.py:561-568
 * (and, on the serving path, gdn.py:399 + causal_conv1d_fwd at gdn.py:403-414 for a single request), with
 * lm.py's rounding points: the projection rounded to bf16, the conv accumulated in fp32 and rounded, the SiLU
 * rounded again; the projection's raw q|k|v is never written.
 *   x, w, y, x_ld, y_ld, M, N, K as zgdn_gemm_nt (bf16). C: conv channels (q|k|v), a multiple of 128, <= N.
 *   conv_weight [C, 4] (tap 0 oldest, 8-byte aligned). hist_in [C, 3]: the raw inputs before row 0, oldest
 *   first (NULL = zeros); hist_out [C, 3] receives the last 3 raw inputs of [history | rows] (NULL = not
 *   written; must not be hist_in).
 */
int zgdn_in_proj_conv(const void* x, long x_ld, const void* w, void* y, long y_ld, int M, int N, int K,
                      const void* conv_weight, int C, const void* hist_in, void* hist_out, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ZONOS3_GDN_H */
