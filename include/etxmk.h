/*
 * etxmk — C ABI of the MI355X (gfx950) batch-small decode megakernel.
 *
 * One handle drives one decoder model on one GPU.  The caller owns every buffer (weights, KV cache,
 * workspace) and hands the library device pointers; the library never allocates device memory and
 * never frees what it is given.  Calls are asynchronous on the HIP stream passed in; one handle is not
 * thread-safe; errors are integer status codes with a message in etxmk_last_error() (no exit()).
 *
 * Each entry point names the reference interface it replaces (paths relative to the reference checkout).
 */
#ifndef ETXMK_H
#define ETXMK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ETXMK_ABI_VERSION 3

/* status codes */
#define ETXMK_OK 0
#define ETXMK_EINVAL 1          /* bad argument or unsupported shape */
#define ETXMK_EHIP 2            /* a HIP runtime call failed */
#define ETXMK_ABORTED 3         /* the device spin limit fired or the host set the abort word */
#define ETXMK_EUNBOUND 4        /* buffers not bound yet */
#define ETXMK_TIMEOUT 5         /* etxmk_sync_timeout: the stream outlived the limit (the step was asked to stop) */

/* tensor kinds (also the seeded generator's stream kinds: stream = kind << 48 | (layer + 1) << 24 | expert) */
#define ETXMK_T_EMBED 1
#define ETXMK_T_LMHEAD 2
#define ETXMK_T_WQKV 3
#define ETXMK_T_WO 4
#define ETXMK_T_ROUTER 5
#define ETXMK_T_W13 6
#define ETXMK_T_W2 7
#define ETXMK_T_WGU 8
#define ETXMK_T_WD 9
/* DeepSeek-V2: kv_b_proj [NH*(qk_nope + v_head)][kv_lora] (stored split: W_UK^T [NH][kv_lora][qk_nope], then W_UV
 * [NH*v_head][kv_lora]), shared experts' gate/up [2*n_shared*MI][H] (gate and up rows interleaved) and down
 * [H][n_shared*MI]; ETXMK_T_WQKV holds q_proj then kv_a_proj_with_mqa, ETXMK_T_KNORM the kv_a_layernorm weight */
#define ETXMK_T_WKVB 14
#define ETXMK_T_WSGU 15
#define ETXMK_T_WSD 16
#define ETXMK_T_LN1 20
#define ETXMK_T_LN2 21
#define ETXMK_T_QNORM 22
#define ETXMK_T_KNORM 23
#define ETXMK_T_FINAL_NORM 24

/* Model dimensions: the POD copy of examples/llm/model.py:45-93 Dims (load_dims, :95-140) that the
 * reference's llm_params.h (__constant__ LlmParams, examples/llm/llm_params.h:1-73) carries.
 * batch: sequences decoded together (1..16; the reference's ETX_VL_REQUESTS requests,
 * examples/vllm_llm/vl_tiles.hip:24-28).  Each sequence owns up to ceil(max_ctx / block_size) blocks of
 * one paged-KV pool, its own token row and its own position; a batched step equals one single-sequence step
 * per sequence, bit for bit. */
typedef struct etxmk_config {
  int32_t H, NH, NKV, HD, I, E, TOPK, MI, L, V;
  int32_t moe, qk_norm, norm_topk, block_size, max_ctx, batch;
  float eps, theta;
  int32_t wdtype;               /* ETXMK_W_BF16, or ETXMK_W_FP8 */
  /* ETXMK_ARCH_DSV2 (DeepSeek-V2): multi-head latent attention (kv_lora, qk_nope, qk_rope,
   * v_head; HD = qk_nope + qk_rope; NKV unused), n_shared shared experts of width MI, first_dense leading dense
   * layers of width dense_I, routing weights times routed_scale, yarn RoPE (theta, rope_* and beta_*) */
  int32_t arch;
  int32_t kv_lora, qk_nope, qk_rope, v_head;
  int32_t n_shared, first_dense, dense_I;
  float routed_scale, rope_factor, rope_mscale, rope_mscale_all, beta_fast, beta_slow;
  int32_t rope_orig_max;
  /* rows of etxmk_prefill launches (0..16; DeepSeek-V2 0..4): the workspace holds max(batch, prefill) rows of
   * activations */
  int32_t prefill;
} etxmk_config;

/* Weight types.  ETXMK_W_FP8: the QKV, O, expert (gate/up, down) and dense MLP matrices are stored as OCP e4m3
 * (round to nearest even, saturated at +-448) with one fp32 scale per output row, s = amax(row) / 448, quantised
 * from bf16 by the library; a matvec row is (sum_k e4m3_k * x_k) * s in the bf16 path's fixed order and rounding
 * points.  Embedding, router, norms and lm_head stay bf16.  Reference: the fp8 fixture quantisation of
 * examples/glm53/cpu_check.py:93-98 (per tensor there; per output channel here). */
#define ETXMK_W_BF16 0
#define ETXMK_W_FP8 1

/* Architectures: Qwen3 (GQA, QK-norm) and DeepSeek-V2 (MLA) */
#define ETXMK_ARCH_QWEN3 0
#define ETXMK_ARCH_DSV2 1

typedef struct etxmk_handle etxmk_handle;

/* Library identity; no reference counterpart (the reference links its runtime statically). */
int etxmk_abi_version(void);
/* Message of the last failing call on this thread (reference: ETX_CHECK's stderr text, etx/runtime/include/etx/host.h:18). */
const char* etxmk_last_error(void);

/* Buffer sizes for a configuration (reference: the allocations of examples/llm/host.hip:122-160 and
 * examples/vllm_llm/host.hip:274-317; here the caller allocates). */
int etxmk_weight_bytes(const etxmk_config* cfg, uint64_t* bytes);
int etxmk_kv_bytes(const etxmk_config* cfg, uint64_t* bytes);
int etxmk_workspace_bytes(const etxmk_config* cfg, uint64_t* bytes);

/* Create / destroy a handle (reference: etx_host::setup, etx/runtime/include/etx/host.h:79-210). */
int etxmk_create(const etxmk_config* cfg, etxmk_handle** out);
int etxmk_destroy(etxmk_handle* h);

/* Bind caller-owned device buffers (reference: the tensor table etx_params.args, etx/runtime/include/etx/abi.h:80-84,
 * filled by the host from its allocations).  Computes and uploads the bf16 RoPE tables
 * (examples/llm/host.hip:164-178) into the workspace and the identity block table. */
int etxmk_bind(etxmk_handle* h, void* weights, void* kv, void* workspace);

/* Where a tensor lives in the weight arena: byte offset, rows, cols, and whether its rows are stored
 * lane-permuted (1) or natural (0).  Reference: the `t name offset count` manifest lines of
 * etx/models/llm/prep.py:243-258. */
int etxmk_tensor_info(etxmk_handle* h, int kind, int layer, int expert, uint64_t* offset, int32_t* rows,
                      int32_t* cols, int32_t* permuted);

/* Storage of a tensor kind: ETXMK_W_BF16 rows (2 * cols bytes, lane-permuted in blocks of 512 when permuted) or
 * ETXMK_W_FP8 rows (cols e4m3 codes lane-permuted in blocks of 1024, then the row's fp32 scale and 12 zero
 * bytes: cols + 16 bytes).  Reference: the per-tensor dtype kind and scale offset of examples/glm53/stage.py:100-124
 * (block scales there; one scale per row here). */
int etxmk_tensor_format(etxmk_handle* h, int kind, int layer, int32_t* wdtype, uint64_t* row_bytes);

/* Fill every weight from the seeded generator (bf16(scale * N(0,1)); norm weights 1.0).
 * Reference: random-init weights have no counterpart; the shapes are those of prep.py:88-146. */
int etxmk_init_weights_seeded(etxmk_handle* h, uint64_t seed, float scale, void* stream);

/* Copy one tensor in natural row-major bf16 layout (device pointer) into the arena, permuting its rows (and
 * quantising them when the tensor is held as fp8).  Reference: the weight load of examples/llm/host.hip:70-121. */
int etxmk_load_tensor(etxmk_handle* h, int kind, int layer, int expert, const void* src, void* stream);

/* Paged-KV block tables, [batch][ceil(max_ctx / block_size)] flattened: entry b * nbps + i is the physical
 * block of sequence b's logical block i; the first n entries are replaced.  No physical block may serve two
 * entries.  Default: the identity.  Reference: block_tables upload, examples/vllm_llm/host.hip:279-282. */
int etxmk_set_block_table(etxmk_handle* h, const int32_t* table, int32_t n, void* stream);

/* Fill KV positions [0, npos) of sequence `seq` (every layer) with bf16 N(0,1) from the seeded generator (the
 * single-layer configuration's cache, the batched workloads' contexts; stream kinds 10 and 11, expert field =
 * seq).  No reference counterpart (the reference prefills by decoding).  etxmk_fill_kv_seeded = sequence 0. */
int etxmk_fill_kv_seeded_seq(etxmk_handle* h, uint64_t seed, int32_t seq, int32_t npos, void* stream);
int etxmk_fill_kv_seeded(etxmk_handle* h, uint64_t seed, int32_t npos, void* stream);

/* Token rows, one per sequence: tokens[0..n) are the prompt; a step at position s reads tokens[s] and writes
 * out_tokens[s] (reference: P.token_in / token_out, examples/llm/tiles.hip:77-82; per request,
 * examples/vllm_llm/vl_tiles.hip:12-22).  The unsuffixed forms address sequence 0. */
int etxmk_set_tokens_seq(etxmk_handle* h, int32_t seq, const int32_t* tokens, int32_t n, void* stream);
int etxmk_read_tokens_seq(etxmk_handle* h, int32_t seq, int32_t* out_tokens, int32_t n, void* stream);
int etxmk_set_tokens(etxmk_handle* h, const int32_t* tokens, int32_t n, void* stream);
int etxmk_read_tokens(etxmk_handle* h, int32_t* out_tokens, int32_t n, void* stream);

/* One decode step at position pos for sequence step `pos` (token tokens[pos]); the greedy token goes to
 * out_tokens[pos] and, when write_next != 0, to tokens[pos + 1].  Asynchronous on `stream`.
 * Reference: etx_host::run (etx/runtime/include/etx/host.h:518-544) = reset_step + launch of
 * etx_megakernel_d0 (etx/codegen/kernel.py:471-605), after llm_set_params (examples/llm/tiles.hip:16-19). */
int etxmk_step(etxmk_handle* h, int32_t pos, int32_t write_next, void* stream);

/* etxmk_step without the workspace's scratch: no counterpart in the reference; for callers that cannot allocate or
 * cannot hand the library a workspace's worth of scratch per handle (code under HIP graph capture, tight serving
 * loops).  The step's scratch (activations, attention chunk partials and arrival counters, the argmax key, the
 * grid-barrier words) lives in a static device array of at most 4 MiB per GPU, held until the process ends; the
 * handle's bound buffers still provide the weights, the KV cache, the token rows (inputs and outputs), block table,
 * RoPE tables and abort word.  Every call clears the array's counters with a fill kernel on `stream` first and calls no
 * allocator.  Calls on one GPU share the array: calls that overlap on one GPU (other streams, other handles) race and
 * must be ordered by the caller.  Single-sequence Qwen3 handles in fused mode; a shape whose scratch exceeds the
 * array is refused with ETXMK_EINVAL.  Results are those of etxmk_step, bit for bit. */
int etxmk_step_static(etxmk_handle* h, int32_t pos, int32_t write_next, void* stream);

/* One decode step of every sequence of a batched handle, sequence b at position positions[b] (host array of
 * `batch` entries), in one persistent launch (fused mode only).  Bit b of write_next_mask: sequence b's greedy
 * token also goes to its tokens[positions[b] + 1] (clear while the sequence is still reading its prompt).
 * Reference: vl_set_params with one VlParams per request (examples/vllm_llm/vl_tiles.hip:92-95) + etx_host::run. */
int etxmk_step_batch(etxmk_handle* h, const int32_t* positions, int32_t write_next_mask, void* stream);

/* Batched prefill: positions pos0 .. pos0 + n - 1 of sequence seq (their tokens set beforehand) in one launch of
 * the batched persistent kernel, one row per position (fused mode, n <= max(batch, prefill)).  Each row
 * computes what etxmk_step computes at its position, bit for bit: its K/V row goes to the cache, its greedy token
 * to out_tokens[pos], and, when write_next != 0, the last row's also to tokens[pos0 + n].  The rows attend to the
 * cache below pos0 and to the launch's own K/V rows (taken from their QKV outputs inside the launch).  Other
 * sequences are untouched.  Prefill launches write no per-layer dumps (etxmk_set_dump buffers hold batch rows) and
 * no trace stamps (the stamp buffer is sized for the handle's step kernel).  Reference: the prompt loop of
 * examples/llm/host.hip:203-213 (one decode step per prompt token), which this replaces by ceil(prompt / n)
 * launches. */
int etxmk_prefill(etxmk_handle* h, int32_t seq, int32_t pos0, int32_t n, int32_t write_next, void* stream);

/* Layers [l0, l1) only, on the residual already in the workspace (etxmk_set_residual), no embedding and
 * no head: the single-layer configuration (single-sequence handles).  Reference: a graph of one layer
 * (examples/llm/model.py:220-273). */
int etxmk_step_layers(etxmk_handle* h, int32_t pos, int32_t l0, int32_t l1, void* stream);
int etxmk_set_residual(etxmk_handle* h, const float* x, void* stream);
int etxmk_read_residual(etxmk_handle* h, float* x, void* stream);

/* Wait for the stream and check the abort word (reference: etx_host::wait + after_wait,
 * etx/runtime/include/etx/host.h:351-417).  Returns ETXMK_ABORTED if the device gave up; after an abort the
 * barrier and attention counters are reset, so the next step runs normally (re-run the aborted position). */
int etxmk_sync(etxmk_handle* h, void* stream);

/* The host watchdog (reference: etx_host::wait_stream's poll loop, which writes ctrl_abort on timeout,
 * etx/runtime/include/etx/host.h:351-376): polls the stream for up to timeout_ms (< 0: no limit); past the limit it
 * sets the handle's stop word, which every grid-barrier wait of a running step reads (see etxmk_set_spin_limit), waits
 * for the stream to drain and returns ETXMK_TIMEOUT (the stopped step's outputs are void; counters are reset as after
 * an abort).  A step that is not stuck finishes before its waits look at the stop word: its results then stand, and
 * the call still reports ETXMK_TIMEOUT for the missed limit.  Otherwise as etxmk_sync. */
int etxmk_sync_timeout(etxmk_handle* h, void* stream, int64_t timeout_ms);

/* Ask the running (or next) step of this handle to stop: sets the stop word in pinned host memory that its waits
 * read; the step ends with ETXMK_ABORTED at the next etxmk_sync, which clears the word.  Reference: the host's write of
 * ctrl_abort (etx/runtime/include/etx/host.h:366). */
int etxmk_abort(etxmk_handle* h);

/* Bounds of every grid-barrier wait (reference: etx_params.spin_limit, etx/runtime/include/etx/abi.h:102, set at
 * etx/runtime/include/etx/host.h:199): a wait gives up after `ticks` of the 100 MHz clock (0: the default 2 s) and sets
 * the abort word; it checks the clock, the abort word and the stop word once every `check_every` polls (a power of two
 * up to 256; 0: 256).  Small values force the abort path on purpose (tests of the error handling). */
int etxmk_set_spin_limit(etxmk_handle* h, uint64_t ticks, int32_t check_every);

/* Execution mode: 1 = one persistent cooperative launch per step (the fused megakernel), 0 = one launch per
 * phase with the same device functions (reference: run_unfused, etx/runtime/include/etx/host.h:418-457). */
int etxmk_set_fused(etxmk_handle* h, int32_t fused);

/* Per-layer dumps of the next steps (device pointers, may be NULL): residual after each layer [L][batch][H] fp32,
 * top-k ids [L][batch][TOPK] int32, weights [L][batch][TOPK] fp32, router logits [L][batch][E] fp32.
 * Reference: ref_numpy.py --dump (examples/llm/ref_numpy.py:199-201) and host --check-dsl
 * (examples/vllm_llm/host.hip:954-1141). */
int etxmk_set_dump(etxmk_handle* h, float* x_layers, int32_t* topk_ids, float* topk_w, float* router_logits);

/* Phase timeline of the next fused steps (device pointer, may be NULL): uint64 [barriers_per_step + 1][workgroups][3];
 * every workgroup writes the 100 MHz s_memrealtime clock when its wait for phase k's inputs returns ([k][wg][0];
 * phase 0: the launch), when it arrives after phase k ([k][wg][1]) and, in GEMV phases, when its first weight
 * loads are issued ([k][wg][2]; attention: when its chunk partials are issued).  Overwritten by each step.
 * Reference: ETX_TRACE stamps (etx/codegen/kernel.py:346-347, etx/runtime/include/etx/host.h:143-145). */
int etxmk_set_trace(etxmk_handle* h, uint64_t* stamps);

/* Workgroups of the persistent launch (0 = one per CU). */
int etxmk_set_grid(etxmk_handle* h, int32_t workgroups);
/* Grid barriers executed by one step (diagnostics). */
int etxmk_barriers_per_step(etxmk_handle* h, int32_t* n);

/* The plan of a configuration, without a GPU: the persistent kernel a step launches (its symbol, or "unfused" for
 * the per-phase kernels), the grid barriers of one step, threads per workgroup, the batch capacity of the kernel and
 * the three buffer sizes.  Reference: the planned-workload record of etx.api.plan (docs/core/API.md:47-49) and the
 * `types` / grid data of the build's plan.json (etx/codegen/plan_header.py). */
typedef struct etxmk_plan_info {
  char kernel[96];
  int32_t barriers_per_step;
  int32_t threads;
  int32_t batch_capacity;
  int32_t matrix_cores;  // 1: the batched projections and experts run on the matrix cores (phases per layer: qkv,
                         // attn, attn_merge, oproj, router, expert_up, expert_down, combine)
  uint64_t weight_bytes, kv_bytes, workspace_bytes;
} etxmk_plan_info;
int etxmk_plan(const etxmk_config* cfg, int32_t fused, etxmk_plan_info* out);

#ifdef __cplusplus
}
#endif
#endif
