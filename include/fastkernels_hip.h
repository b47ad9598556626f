/*
 * fastkernels_hip.h - C ABI of libfastkernels_hip.so, the MI355X (gfx950)
 * kernels behind fastkernels_amd.kernels.hip.
 *
 * Conventions shared by every entry point:
 *   - All tensor arguments are device pointers to contiguous, row-major
 *     storage.  Rows that the kernels stream with vector loads (weights,
 *     hidden rows) must start on a 16-byte boundary and hold a multiple of 8
 *     elements; violations return FK_ERR_ALIGNMENT before any launch.
 *   - `*_dtype` arguments take FK_DTYPE_* codes.  Arithmetic is fp32.
 *   - `stream` is a hipStream_t passed as void*; NULL means the legacy
 *     default stream.  Calls only enqueue work: no host synchronisation, no
 *     device allocation.  Outputs and workspaces are caller-owned.
 *   - Workspaces hold self-resetting counters and must be zero-filled once
 *     when first allocated; after that they can be reused by consecutive calls
 *     on one stream.  Calls that overlap on different streams need separate
 *     workspaces.
 *   - Every function returns FK_OK (0) or an FK_ERR_* status;
 *     fk_last_error_detail() gives a human-readable reason for the calling
 *     thread's last failure.
 *
 * Each declaration cites the reference operator it replaces
 * (suryavanshi/fastkernels, src/fastkernels/kernels/triton/...).
 */
#ifndef FASTKERNELS_HIP_H
#define FASTKERNELS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FK_ABI_VERSION 1

enum {
  FK_DTYPE_F32 = 0,
  FK_DTYPE_BF16 = 1,
  FK_DTYPE_I32 = 2,
  FK_DTYPE_I64 = 3
};

enum {
  FK_OK = 0,
  FK_ERR_INVALID = 1,     /* bad rank/shape/size argument */
  FK_ERR_DTYPE = 2,       /* unsupported dtype code */
  FK_ERR_WORKSPACE = 3,   /* workspace missing or too small */
  FK_ERR_LAUNCH = 4,      /* hipLaunchKernel / runtime error */
  FK_ERR_UNSUPPORTED = 5, /* shape outside the kernels' limits */
  FK_ERR_ALIGNMENT = 6,   /* pointer or row length breaks 16-byte vector loads */
  FK_ERR_DEVICE = 7       /* a bounded wait inside a kernel ran out (fk_workspace_status) */
};

int fk_abi_version(void);
const char* fk_status_string(int status);
const char* fk_last_error_detail(void);

/* Device error word of a workspace of fk_moe_router / fk_moe_align /
 * fk_moe_experts / fk_moe_layer, fk_deltanet_step or fk_attention_decode.
 * Those kernels hand values between workgroups and assume that every
 * workgroup of a launch is resident at once (the host caps their grids at
 * the device's co-resident capacity); each wait is bounded.  A wait that
 * runs out (another process or stream holding CUs for long) sets the error
 * word, the kernel ends normally and the outputs its workgroups produced
 * from incomplete inputs are NaN (routing weights, MoE outputs, DeltaNet
 * update and recurrent state, attention update and the step's cache rows).
 * While the word stays set, every later call on the workspace gives NaN
 * outputs.  fk_attention_decode also sets it (another bit) when a
 * device-held position would take the step past the cache: the update is
 * NaN, the caches are untouched and the position is not advanced.  This
 * call synchronises `stream`, then returns FK_OK or FK_ERR_DEVICE (with the
 * flags in fk_last_error_detail); `clear` != 0 also resets the word
 * (stream-ordered), after which calls give valid outputs again.
 * No counterpart in the reference: its Triton kernels never wait on another
 * program.  For callers that validate a run (tests, benchmarks). */
int fk_workspace_status(const void* workspace, size_t workspace_bytes, int clear, void* stream);

/* Bound on every in-kernel wait of the calls on `workspace` (same
 * workspaces as fk_workspace_status), stream-ordered: `limit` poll rounds,
 * each one coherent read of the words not yet in (roughly 0.1-1 us), at
 * most FK_MAX_POLL_LIMIT (FK_ERR_INVALID above it: a wait that fails still
 * ends within seconds); 0: each wait gives up at once, so every such call
 * flags FK_ERR_DEVICE and gives NaN outputs, and every kernel still ends; a
 * negative `limit` restores the built-in bound (2^16 rounds).  No
 * counterpart in the reference: a test hook for the failure path, and a
 * knob for callers that prefer an early flagged failure to a long wait. */
#define FK_MAX_POLL_LIMIT (1ll << 22)
int fk_workspace_set_poll_limit(void* workspace, size_t workspace_bytes, long long limit, void* stream);

/* ------------------------------------------------------------------------ */
/* MoE decode layer                                                          */
/* ------------------------------------------------------------------------ */

/* Bytes of workspace needed by fk_moe_router / fk_moe_align / fk_moe_experts
 * / fk_moe_layer for this problem size (routing tables, counters, and the
 * fp32 SwiGLU activations and down-projection outputs of every routed
 * (token, slot) pair and shared-expert token). */
size_t fk_moe_workspace_bytes(int tokens, int top_k, int num_experts, int intermediate, int hidden_size);

/* Router: n = RMSNorm(x) * (norm_offset + w); logits = n . W^T (+ bias);
 * softmax; top-k ordered by (probability desc, expert id asc); weights
 * renormalised to sum 1.  Also writes the routing tables consumed by
 * fk_moe_experts into `workspace`.
 * Replaces triton_qwen36_moe_router_decode (qwen36_router.py:193-257) and
 * triton_qwen36_batched_moe_router_decode (qwen36_router.py:260-319).
 * `router_bias` (nullable, length num_experts) has no reference counterpart:
 * it is added to the logits (and so appears in `logits`). */
int fk_moe_router(const void* hidden, int hidden_dtype,
                  const void* norm_weight, int norm_dtype,
                  const void* router_weight, int router_dtype,
                  const void* router_bias, int bias_dtype,
                  int tokens, int hidden_size, int num_experts, int top_k,
                  float eps, float norm_offset,
                  float* logits, int64_t* topk_ids, float* topk_weights,
                  void* workspace, size_t workspace_bytes, void* stream);

/* Routing tables from caller-supplied ids/weights: expert histogram,
 * exclusive offsets, the stable permutation of (token, slot) pairs sorted by
 * (expert, token, slot), and its inverse.  Out-of-range ids are clamped to
 * [0, num_experts-1] as the reference expert kernels do
 * (qwen36_expert.py:146).  The four outputs are optional copies of the tables
 * kept in `workspace`.  `topk_weights` may be NULL (histogram-only use).
 * Replaces triton_expert_histogram (moe.py:87-102); the permutation has no
 * reference counterpart (the reference re-streams weights per pair,
 * qwen36_expert.py:456-537). */
int fk_moe_align(const void* topk_ids, int ids_dtype,
                 const void* topk_weights, int weights_dtype,
                 int tokens, int top_k, int num_experts,
                 void* workspace, size_t workspace_bytes,
                 int32_t* counts_out, int32_t* offsets_out,
                 int32_t* perm_out, int32_t* inverse_out, void* stream);

/* Expert stage for the routing tables in `workspace`: per routed pair
 * a = silu(W_gu[e,:I] x) * (W_gu[e,I:] x), y += w * (W_d[e] a); optional
 * shared expert (same shapes, un-indexed) scaled by sigmoid(w_g . x) when
 * `shared_gate` is non-NULL.  Experts read the un-normalised hidden x.
 * out (f32[T,H]) = moe update; layer_out (nullable) = x + out.
 * shared_gate_up == NULL && shared_down == NULL selects routed-only.
 * Replaces triton_qwen36_routed_experts_decode (qwen36_expert.py:889-966),
 * triton_qwen36_routed_shared_experts_decode (:969-1093),
 * triton_qwen36_batched_routed_experts_decode (:1096-1178),
 * triton_qwen36_batched_routed_shared_experts_decode (:1181-1309) and
 * triton_qwen36_single_expert_mlp_decode (:817-886, one expert, K=1). */
int fk_moe_experts(const void* hidden, int hidden_dtype,
                   const void* gate_up, const void* down, int expert_dtype,
                   const void* shared_gate_up, const void* shared_down,
                   const void* shared_gate, int shared_gate_dtype,
                   int tokens, int hidden_size, int intermediate,
                   int num_experts, int top_k,
                   float* out, float* layer_out,
                   void* workspace, size_t workspace_bytes, void* stream);

/* Router + expert stage in one call (the full MoE block plus residual).
 * Replaces triton_qwen36_moe_decode (qwen36_expert.py:1312-1350),
 * triton_qwen36_batched_moe_decode (:1353-1387) and
 * triton_qwen36_batched_moe_layer_decode (qwen36_layer.py:55-106). */
int fk_moe_layer(const void* hidden, int hidden_dtype,
                 const void* norm_weight, int norm_dtype,
                 const void* router_weight, int router_dtype,
                 const void* router_bias, int bias_dtype,
                 const void* gate_up, const void* down, int expert_dtype,
                 const void* shared_gate_up, const void* shared_down,
                 const void* shared_gate, int shared_gate_dtype,
                 int tokens, int hidden_size, int intermediate,
                 int num_experts, int top_k, float eps, float norm_offset,
                 float* logits, int64_t* topk_ids, float* topk_weights,
                 float* moe_out, float* layer_out,
                 void* workspace, size_t workspace_bytes, void* stream);

/* fk_moe_layer without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No counterpart in the reference.
 * The workspace is a file-scope device array of FK_MOE_NOALLOC_SCRATCH_BYTES
 * (16 MiB) that each GPU holds from the moment a process loads this library
 * until the process ends, whether or not it ever calls this function;
 * a problem whose fk_moe_workspace_bytes exceeds it returns
 * FK_ERR_UNSUPPORTED (at the model's shape: up to 174 tokens).  The call
 * allocates nothing.  The first call on a device zero-fills the array on
 * `stream` and waits for that fill (so a first call from another stream or
 * thread cannot see an uncleared array); it must not be under graph capture,
 * later calls may be.  Every call on a GPU shares that GPU's array, so calls
 * that overlap on one GPU (on different streams, or from several threads)
 * race and give wrong results; serialise them.  A bounded in-kernel wait
 * that runs out gives NaN outputs for this call and every later one on the
 * GPU until the array's error word is cleared: fk_moe_noalloc_workspace
 * gives the array's device address, for fk_workspace_status and
 * fk_workspace_set_poll_limit. */
#define FK_MOE_NOALLOC_SCRATCH_BYTES (16u << 20)
int fk_moe_layer_noalloc(const void* hidden, int hidden_dtype,
                         const void* norm_weight, int norm_dtype,
                         const void* router_weight, int router_dtype,
                         const void* router_bias, int bias_dtype,
                         const void* gate_up, const void* down, int expert_dtype,
                         const void* shared_gate_up, const void* shared_down,
                         const void* shared_gate, int shared_gate_dtype,
                         int tokens, int hidden_size, int intermediate,
                         int num_experts, int top_k, float eps, float norm_offset,
                         float* logits, int64_t* topk_ids, float* topk_weights,
                         float* moe_out, float* layer_out, void* stream);

/* The current device's fk_moe_layer_noalloc array: its device address and
 * size, for fk_workspace_status (read and clear its error word) and
 * fk_workspace_set_poll_limit.  Allocates nothing; the first use on a device
 * clears the array as fk_moe_layer_noalloc's first call does (same rules). */
int fk_moe_noalloc_workspace(void** workspace, size_t* workspace_bytes, void* stream);

/* counts[e] = #{i : ids[i] == e} over n ids (int32 or int64); ids outside
 * [0, num_experts) are ignored.  counts is overwritten.
 * Replaces triton_expert_histogram (moe.py:87-102) as a standalone op. */
int fk_expert_histogram(const void* ids, int ids_dtype, int64_t n,
                        int num_experts, int32_t* counts, void* stream);

/* out[r, i] = silu(gu[r, i]) * gu[r, I + i]; out has the dtype of gu.
 * Replaces triton_fused_swiglu (moe.py:67-84). */
int fk_fused_swiglu(const void* gate_up, int dtype, int64_t rows,
                    int intermediate, void* out, void* stream);

/* out = float(hidden) + update over n elements.
 * Replaces the residual-add kernel of qwen36_layer.py:37-52. */
int fk_residual_add(const void* hidden, int hidden_dtype, const float* update,
                    int64_t n, float* out, void* stream);

/* Reads `bytes` (a multiple of 16) at `src` once, as the weight streams do
 * (16-byte non-temporal loads, one-shot 16 KiB per workgroup), and writes
 * nothing (`sink`, one word, is only a guard).  A bandwidth probe: the read
 * ceiling bench.py reports the kernels' fractions against, beside the
 * published peak.  No counterpart in the reference. */
int fk_stream_read(const void* src, size_t bytes, uint32_t* sink, void* stream);

/* ------------------------------------------------------------------------ */
/* Gated full attention (the mixer of every fourth layer)                    */
/* ------------------------------------------------------------------------ */

/* xn = RMSNorm(x) * (norm_offset + w); q = xn Wq^T (q_rows: query/gate pairs
 * per head), k = xn Wk^T, v = xn Wv^T (kv_rows each); f32 outputs.
 * Replaces triton_qwen36_batched_attention_project (qwen36_attention.py:168-211). */
int fk_attention_project(const void* hidden, int hidden_dtype,
                         const void* norm_weight, int norm_dtype,
                         const void* q_proj, const void* k_proj, const void* v_proj,
                         int weight_dtype, int tokens, int hidden_size, int q_rows,
                         int kv_rows, float eps, float norm_offset,
                         float* q_out, float* k_out, float* v_out, void* stream);

/* Bytes of workspace for fk_attention_decode. */
size_t fk_attention_workspace_bytes(int tokens, int heads, int kv_heads, int head_dim);

/* Gated attention decode of `tokens` (<= 32) rows at positions
 * start_position ..: projections, per-head RMSNorm(1 + w) of q and k, RoPE
 * of the first rope_dim dims (rope_interleaved: pairs (2i, 2i+1); else
 * halves (i, i + rope_dim/2)), the new k/v rows written into the caches
 * [max_positions, kv_heads, head_dim] (f32 or bf16) in place, causal
 * softmax attention (GQA: heads / kv_heads query heads per kv head),
 * o * sigmoid(gate), update = . Wo^T (f32 [T, hidden]) and, when hidden_out
 * is not NULL, hidden_out = hidden + update.  head_dim <= 256,
 * heads * head_dim <= 4096, heads / kv_heads <= 8.  start_position_device
 * (nullable, no reference counterpart): a device int32 read at run time in
 * place of start_position and advanced by `tokens` at the end of the step,
 * so one captured HIP graph decodes successive positions; a value with
 * start + tokens past max_positions gives NaN updates and leaves the caches
 * untouched.  For tokens <= 4 with bf16 weights, hidden_size a multiple of
 * 512 up to 2048, head_dim a power of two in [64, 256], heads / kv_heads <=
 * 8 (a multiple of 4 above 4) and heads * head_dim a multiple of 512 (the
 * model's shapes) this is one launch whose workgroups hand values to each
 * other (the workspace then also carries the error word of
 * fk_workspace_status); other calls run four launches.
 * Replaces triton_qwen36_batched_attention_decode (qwen36_attention.py:448-577)
 * and the residual add of triton_qwen36_batched_attention_moe_layer_decode
 * (qwen36_layer.py:109-201). */
int fk_attention_decode(const void* hidden, int hidden_dtype,
                        const void* norm_weight, int norm_dtype,
                        const void* q_proj, const void* k_proj, const void* v_proj,
                        const void* o_proj, int weight_dtype,
                        const void* q_norm_weight, const void* k_norm_weight, int qk_norm_dtype,
                        void* key_cache, void* value_cache, int cache_dtype,
                        int max_positions, int start_position,
                        const int32_t* start_position_device, int tokens, int hidden_size,
                        int heads, int kv_heads, int head_dim, int rope_dim, float rope_theta,
                        int rope_interleaved, float eps, float qk_eps,
                        float* update, float* hidden_out,
                        void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Gated DeltaNet decode step                                                */
/* ------------------------------------------------------------------------ */

/* xn = RMSNorm(x) * (norm_offset + w); mixed_qkv = xn W_qkv^T, z = xn W_z^T,
 * a = xn W_a^T, b = xn W_b^T (all f32 outputs).
 * Replaces triton_qwen36_batched_deltanet_project (qwen36_deltanet.py:403-457). */
int fk_deltanet_project(const void* hidden, int hidden_dtype,
                        const void* norm_weight, int norm_dtype,
                        const void* w_qkv, const void* w_z,
                        const void* w_a, const void* w_b, int weight_dtype,
                        int tokens, int hidden_size, int qkv_rows, int z_rows,
                        int ab_rows, float eps, float norm_offset,
                        float* mixed_qkv, float* z, float* a_logits,
                        float* b_logits, void* stream);

/* Causal depthwise conv over [conv_state | mixed^T] per channel, SiLU, and
 * the rolled state (last kernel_size columns, stored in state_dtype).
 * Replaces triton_qwen36_batched_deltanet_conv (qwen36_deltanet.py:534-584). */
int fk_deltanet_conv(const void* mixed, int mixed_dtype,
                     const void* conv_state, int state_dtype,
                     const void* conv_weight, int weight_dtype,
                     int tokens, int channels, int kernel_size,
                     float* conv_out, void* next_state, void* stream);

/* Bytes of workspace for fk_deltanet_recurrent_output. */
size_t fk_deltanet_workspace_bytes(int tokens, int value_heads, int head_dim);

/* Gated delta rule over `tokens` consecutive rows through one recurrent
 * state, per-head gated RMSNorm (plain weight) and the output projection.
 * update (f32[T,hidden]) = core W_out^T; next_state has state_dtype.
 * residual/residual_out (both nullable) add: residual_out = residual + update.
 * `tensor_dtypes` holds the dtypes of, in order: mixed_qkv, z, a_logits,
 * b_logits, recurrent_state, out_proj_weight, linear_norm_weight, a_log,
 * dt_bias, residual.
 * Replaces triton_qwen36_batched_deltanet_recurrent_output
 * (qwen36_deltanet.py:744-863). */
int fk_deltanet_recurrent_output(const void* mixed_qkv, const void* z,
                                 const void* a_logits, const void* b_logits,
                                 const void* recurrent_state,
                                 const void* out_proj_weight,
                                 const void* linear_norm_weight,
                                 const void* a_log, const void* dt_bias,
                                 const void* residual,
                                 const int32_t* tensor_dtypes,
                                 int tokens, int qk_heads, int value_heads,
                                 int head_dim, int hidden_size, float eps,
                                 float* update, void* next_state,
                                 float* residual_out,
                                 void* workspace, size_t workspace_bytes,
                                 void* stream);

/* Bytes of workspace for fk_deltanet_step. */
size_t fk_deltanet_step_workspace_bytes(int tokens, int qk_heads, int value_heads, int head_dim);

/* The whole Gated DeltaNet step with the residual: RMSNorm(1+w) +
 * projections with the causal conv, the recurrent rule with the per-head
 * gated RMSNorm, and the output projection.  At the model's shapes and
 * dtypes (tokens <= 8, head_dim 128, bf16 weights, fp32 recurrent state)
 * this is one launch (deltanet_step_kernel); other shapes run three staged
 * launches (projection + conv, recurrent + gated norm, output projection).
 * update = core W_out^T; hidden_out (nullable) =
 * hidden + update; next_conv_state / next_recurrent_state keep the dtypes of
 * their inputs.  `dtypes` holds, in order: hidden, input_norm_weight,
 * projection weights (qkv/z/a/b share one), conv_state, conv1d_weight,
 * recurrent_state, out_proj_weight, linear_norm_weight, a_log, dt_bias.
 * Limits: tokens <= 64, kernel_size <= 8.
 * Replaces the project -> conv -> recurrent/output -> residual sequence of
 * triton_qwen36_batched_deltanet_moe_layer_decode (qwen36_layer.py:238-282). */
int fk_deltanet_step(const void* hidden, const void* input_norm_weight,
                     const void* w_qkv, const void* w_z, const void* w_a, const void* w_b,
                     const void* conv_state, const void* conv_weight,
                     const void* recurrent_state, const void* out_proj_weight,
                     const void* linear_norm_weight, const void* a_log, const void* dt_bias,
                     const int32_t* dtypes, int tokens, int hidden_size,
                     int qk_heads, int value_heads, int head_dim, int kernel_size, float eps,
                     float* update, float* hidden_out, void* next_conv_state,
                     void* next_recurrent_state, void* workspace, size_t workspace_bytes,
                     void* stream);

/* ------------------------------------------------------------------------ */
/* Synthetic (tiny-spec) decode blocks behind the --moe-impl/--deltanet-impl  */
/* switch of bench/qwen36_decode_reference.py                                */
/* ------------------------------------------------------------------------ */

/* One-token MoE with plain-weight RMSNorm router, softmax top-k (ties to the
 * lower id) with renormalisation, routed + ungated shared expert, residual;
 * output in out_dtype.  Limits: hidden, intermediate <= 1024, experts <= 1024.
 * Replaces triton_synthetic_qwen36_moe_decode (qwen36_moe.py:362-444). */
int fk_synthetic_moe(const void* hidden, int hidden_dtype,
                     const void* norm_weight, const void* router_weight,
                     const void* gate_up, const void* down,
                     const void* shared_gate_up, const void* shared_down,
                     int weight_dtype, int hidden_size, int num_experts,
                     int intermediate, int top_k, float eps,
                     void* out, int out_dtype, void* stream);

/* One-token toy DeltaNet: S' = 0.95 S + k (x) v per qk head,
 * out = x + W_o ((q . S') * sigmoid(W_g xn)), xn = RMSNorm(x) * w.
 * hidden_out has hidden_dtype, state_out has state_dtype.
 * Replaces triton_synthetic_qwen36_deltanet_decode (qwen36_deltanet.py:966-1041). */
int fk_synthetic_deltanet(const void* hidden, int hidden_dtype,
                          const void* state, int state_dtype,
                          const void* norm_weight, const void* q_weight,
                          const void* k_weight, const void* v_weight,
                          const void* gate_weight, const void* out_weight,
                          int weight_dtype, int hidden_size, int qk_heads,
                          int head_dim, int value_dim_per_head, float eps,
                          void* hidden_out, void* state_out, void* stream);

/* One-token synthetic grouped-query attention: xn = RMSNorm(x) * w;
 * q, k, v = W xn (held in hidden_dtype); RoPE on q and k (interleaved pairs,
 * angle position / 10000^(2i / r), r = min(rope_dim, head_dim) rounded down
 * to even); k and v written to row `position` of the caches ([max_positions,
 * kv_heads, head_dim], cache_dtype, updated in place); each query head
 * attends over rows 0..position of its kv head; out = x + W_o attended, in
 * hidden_dtype.  Limits: widths and max_positions <= 128.
 * Replaces triton_synthetic_qwen36_attention_decode
 * (qwen36_attention.py:852-998; the caller copies the caches first when it
 * wants them untouched, as the reference's copy_cache=True does). */
int fk_synthetic_attention(const void* hidden, int hidden_dtype,
                           void* key_cache, void* value_cache, int cache_dtype,
                           const void* norm_weight, const void* q_weight,
                           const void* k_weight, const void* v_weight,
                           const void* out_weight, int weight_dtype,
                           int hidden_size, int attention_heads, int kv_heads,
                           int head_dim, int rope_dim, int position,
                           int max_positions, float eps, void* out,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FASTKERNELS_HIP_H */
