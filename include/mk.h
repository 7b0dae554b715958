/*
 * mk.h — C ABI of libmk.so, the MI355X (gfx950) Llama-3.2-1B decode megakernel.
 *
 * One call runs one token-generation step of all requested decoder layers in a
 * single persistent kernel launch, optionally followed by the final RMSNorm,
 * the tied lm_head GEMV and a greedy argmax, on the caller's HIP stream.
 *
 * Every pointer in mk_weights / mk_step_args is a device pointer owned by the
 * caller (PyTorch tensors in this repository), except k_cache / v_cache, which
 * are host arrays holding one device pointer per layer. The library never
 * allocates, frees or synchronises inside mk_decode_step.
 *
 * Reference interfaces this ABI replaces (keaganchern/llama1B-megakernel):
 *   - transformer_llama_megakernel_16layers(X, Wq_all, Wk_all, Wv_all, Wo_all,
 *       gpre_all, Wgu_all, Wd_all, gpost_all, K_00..K_15, V_00..V_15, cos, sin,
 *       position_ids) -> (Y, K_00..K_15, V_00..V_15)
 *       transformer_llama.py:196-241 (body 90-144)       -> mk_decode_step
 *   - transformer_llama_megakernel_1layer(...)  transformer_llama.py:154-191
 *                                                          -> mk_layer_step
 *   - the lm_head / sampling of NxDI's token-generation graph
 *       (llama.py:1208-1227, main.py:57, 291)              -> mk_decode_step
 *         with logits / next_token set
 *
 * Error convention: 0 on success, a negative MK_ERR_* code otherwise, with a
 * message from mk_last_error(). Arguments are validated before any HIP call.
 * Faults the device detects while running (a position out of range, a wait
 * for another workgroup's results that timed out) set bits in the workspace;
 * mk_read_device_error() returns and clears them.
 */
#ifndef MK_H_
#define MK_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MK_ABI_VERSION 1

#define MK_OK                0
#define MK_ERR_NULL         -1   /* a required pointer is NULL                  */
#define MK_ERR_SHAPE        -2   /* layer count, batch, s_max, rope_rows        */
#define MK_ERR_WORKSPACE    -3   /* workspace too small or misaligned           */
#define MK_ERR_UNSUPPORTED  -4   /* a valid request this build does not run     */
#define MK_ERR_HIP          -5   /* a HIP runtime call failed                   */
#define MK_ERR_DEVICE       -6   /* device cannot co-schedule the persistent grid */
#define MK_ERR_ALIGN        -7   /* a pointer is not 16-byte aligned            */

/* Device-side error bits (mk_read_device_error). */
#define MK_DEVERR_POS        0x1u  /* pos[b] < 0 or >= s_max or >= rope_rows: step skipped */
#define MK_DEVERR_SYNC       0x2u  /* a wait for another workgroup's results exceeded its time limit */
#define MK_DEVERR_BARRIER    MK_DEVERR_SYNC   /* earlier name of the same bit */

/* mk_step_args.flags */
#define MK_FLAG_ADVANCE      0x1u  /* after the step: pos[b] += 1 (device side)   */
#define MK_FLAG_COOPERATIVE  0x2u  /* launch cooperatively: co-residency of the
                                      one-workgroup-per-CU grid guaranteed by the
                                      runtime (default: a plain launch, which
                                      leaves ~20 us less between steps)          */
#define MK_FLAG_PREFILL      0x4u  /* context encoding: the batch's tokens are
                                      consecutive tokens of ONE sequence, token b
                                      at position pos[b] = pos[0] + b, all using
                                      sequence 0 of the caches (k_cache[l] may be
                                      [1][8][s_max][64]); token b attends to rows
                                      [0, pos[b]], including the rows the other
                                      tokens of the step write. Needs a batched
                                      workspace (mk_workspace_bytes(batch >= 2)). */
#define MK_DEVERR_PREFILL    0x4u  /* MK_FLAG_PREFILL with pos[b] != pos[0] + b: step skipped */

/* Model constants the kernel is built for (Llama-3.2-1B). */
#define MK_HIDDEN      2048
#define MK_N_Q_HEADS   32
#define MK_N_KV_HEADS  8
#define MK_HEAD_DIM    64
#define MK_INTER       8192
#define MK_VOCAB       128256
#define MK_MAX_LAYERS  16
#define MK_QKV_ROWS    3072

/*
 * Packed, layer-stacked weights (all bf16, row-major [out][in]).
 * Counterpart of the eight mk_*_stack parameters built by
 * NeuronLlamaForCausalLMMK.convert_hf_to_neuron_state_dict
 * (llama_with_megakernel.py:281-351), in this build's own layout:
 *   w_qkv     [L][3072][2048]  Q,K,V rows in RoPE pairs (d, d+32) of a head:
 *                              Q heads, then K heads, then V heads; the
 *                              input_layernorm gamma folded in.
 *   w_o       [L][2048][2048]  o_proj.weight
 *   w_gu      [L][16384][2048] rows (gate_i, up_i) interleaved; the
 *                              post_attention_layernorm gamma folded in.
 *   w_down    [L][2048][8192]  down_proj.weight
 *   embed     [128256][2048]   token embedding, also the tied lm_head
 *   norm_final[2048]           final RMSNorm gamma
 *   rope      [rope_rows][128] bf16 cos(64) | sin(64) per position
 *                              (replaces the per-step cos/sin kernel inputs)
 */
typedef struct mk_weights {
    const void *w_qkv;
    const void *w_o;
    const void *w_gu;
    const void *w_down;
    const void *embed;
    const void *norm_final;
    const void *rope;
    int32_t n_layers;    /* layers present in the stacks (1..16)       */
    int32_t rope_rows;   /* rows of the rope table (>= s_max)          */
    /*
     * Optional second copies of w_qkv, w_o, w_gu, w_down and embed in MFMA
     * tile order, read by the batched kernel (batch > 1 and prefill steps)
     * when all five are set; NULL: it reads the row-major stacks above. For
     * a matrix [N][K] (N a multiple of 16, K of 32) the 1 KiB block
     * (n16, ks) = (row / 16, column / 32) sits at block index n16*(K/32) + ks,
     * and in it the 16 bytes at ((column % 32) / 8 * 16 + row % 16) * 16 hold
     * columns 8*j .. 8*j+7 of the k-step: one block is one MFMA B operand
     * (16 rows x 32 columns), so each load instruction reads 1 KiB
     * contiguous instead of 64 bytes from each of 16 rows. Stacked per layer
     * like the row-major copies (same sizes). No counterpart in the reference
     * (its NKI kernel has one layout per weight).
     */
    const void *t_qkv;
    const void *t_o;
    const void *t_gu;
    const void *t_down;
    const void *t_embed;
} mk_weights;

/*
 * One decode step.
 *   layers [first_layer, first_layer + n_layers) run, in order.
 *   Input: tokens[b] (embedding gather) or hidden_in[b][2048] (bf16);
 *          exactly one of the two is non-NULL.
 *   k_cache[i], v_cache[i]: layer first_layer+i, bf16 [batch][8][s_max][64].
 *          The fresh K (after RoPE) and V rows are written in place at row
 *          pos[b]; attention reads rows [0, pos[b]] (the fresh row included).
 *          Nothing else in the caches is read or written.
 *   pos[b]: device int32, 0 <= pos[b] < s_max.
 *   hidden_out: bf16 [batch][2048] hidden state after the last layer (before
 *          the final norm), or NULL.
 *   logits: fp32 [batch][128256] or NULL; next_token: int32 [batch] greedy
 *          argmax (lowest index on ties) or NULL. If both are NULL the final
 *          norm and lm_head are skipped (the layer-stack seam of
 *          transformer_llama.py). next_token may alias tokens.
 *   workspace: device memory of at least mk_workspace_bytes(batch, s_max)
 *          bytes, 256-byte aligned, initialised once with mk_workspace_init
 *          before first use; every step leaves it ready for the next.
 *   stream: hipStream_t (NULL = default stream).
 * Calls on one workspace must not overlap in time (same stream, or ordered).
 */
typedef struct mk_step_args {
    int32_t first_layer;
    int32_t n_layers;
    int32_t batch;
    int32_t s_max;
    void *const *k_cache;
    void *const *v_cache;
    const int32_t *tokens;
    const void *hidden_in;
    int32_t *pos;
    void *hidden_out;
    float *logits;
    int32_t *next_token;
    uint32_t flags;
    void *workspace;
    size_t workspace_bytes;
    void *stream;
    /* Optional phase trace (NULL = off): device uint64 [grid][MK_TRACE_SLOTS].
     * Workgroup w records the device wall clock (mk_wall_clock_hz ticks/s) in
     * slot 0 at start, 2k-1 when it starts waiting for the input of hand-over
     * k and 2k when that input has arrived, and MK_TRACE_SLOTS-1 at exit.
     * Hand-over k = 5*i + j is phase j of run-layer i (1 QKV input, 2
     * attention inputs, recorded by workgroups with attention work only, 3
     * attention output, 4 h1, 5 gate/up output); k = 5*n_layers + 1 is the
     * lm_head input. Slot MK_TRACE_DONE0 + 5*i + j (below MK_TRACE_SLOTS-8)
     * is recorded when phase j (0 QKV, 1 attention, 2 O, 3 gate/up, 4 down)
     * of run-layer i has issued its result stores; slots MK_TRACE_SLOTS-8 ..
     * MK_TRACE_SLOTS-2 hold kernel-specific diagnostic values (in a decode
     * loop, whose trace keeps the marks of its last step: MK_TRACE_SLOTS-4 the
     * previous step's arrival at the step barrier, -3 the barrier seen, -2
     * the token read). */
    void *trace;
} mk_step_args;

#define MK_TRACE_SLOTS 256
#define MK_TRACE_DONE0 166

/*
 * On-device sampling of the next token from fp32 logits (after a decode step
 * that wrote `logits`). Counterpart of NxDI's on-device sampler configured by
 * --top-k / --top-p / --temperature / --global-topk / --on-device-sampling
 * (main.py:57-61, 85, 129-130) with per-sequence sampling parameters as built
 * by prepare_sampling_params (main.py:195-206).
 *   params: device fp32 [batch][3] = (top_k, top_p, temperature) per row.
 *     top_k == 1 or temperature <= 0: greedy argmax (lowest index on ties);
 *     top_k <= 0 or > MK_SAMPLE_MAX_TOPK: the global cap MK_SAMPLE_MAX_TOPK;
 *     tokens with logit/temperature >= the top_k-th largest are kept (ties
 *     included, at most MK_SAMPLE_CAND of them), then top_p in (0, 1) keeps,
 *     in descending order, each token whose preceding softmax mass is < top_p;
 *     one draw from the renormalised kept distribution (inverse CDF in
 *     descending order) with u = Philox4x32-10(key = seed, counter =
 *     (counter[row], row, 0, 0)) first word >> 8, times 2^-24.
 *   counter: device int32 [batch] (e.g. the sequences' positions) or NULL (0).
 *   tokens_out: device int32 [batch]; uniforms_out: device fp32 [batch] (the u
 *     each row used, -1 for greedy rows) or NULL.
 * Asynchronous on `stream`; allocates nothing.
 */
#define MK_SAMPLE_MAX_TOPK 1024
#define MK_SAMPLE_CAND     2048
typedef struct mk_sample_args {
    const float *logits;
    int32_t batch;
    int32_t vocab;
    int32_t vocab_stride;      /* floats between rows of logits (>= vocab) */
    const float *params;
    uint64_t seed;
    const int32_t *counter;
    int32_t *tokens_out;
    float *uniforms_out;
    void *stream;
} mk_sample_args;
int mk_sample(const mk_sample_args *a);
const char *mk_sample_last_error(void);

/* Library / device information. */
int mk_abi_version(void);
const char *mk_last_error(void);
/* Grid size (workgroups, one per CU) the kernel uses on `device`; <0 on error. */
int mk_grid_size(int device);
/*
 * Launch the kernels of `device` on `workgroups` workgroups, one per CU, in
 * [32, CU count] (0: back to one per CU). Any other count runs the kernels'
 * generic-grid variants (MI355X's 256 gets variants with the grid size fixed
 * at compile time), and leaves the other CUs to other work. Applies to the
 * steps launched after the call; make it with no step of the device in
 * flight. MK_ERR_SHAPE for a count out of range. No counterpart in the
 * reference (its NKI kernel runs on one NeuronCore).
 */
int mk_set_grid_size(int device, int workgroups);
/* Frequency of the device wall clock used by the trace (ticks per second). */
long long mk_wall_clock_hz(int device);

/* Workspace bytes for `batch` sequences with `s_max` cache rows; 0 if unsupported. */
size_t mk_workspace_bytes(int32_t batch, int32_t s_max);
/*
 * Initialise the workspace on `stream` with fill kernels. The first call for
 * a workspace address on a device also ALLOCATES its exchange area (the
 * per-layer hand-over buffers the kernel's workgroups pass results through):
 * 3.2 MB of uncached device memory for a batch-1 workspace, or
 * BatchLayout(batch) bytes (about 100 MB at batch 32) of ordinary device
 * memory for a batched one. So this call must not be made under stream
 * capture; later calls for the same workspace only launch the fills. At most
 * 256 exchange areas exist at once per process (MK_ERR_WORKSPACE beyond).
 * No counterpart in the reference (its NKI kernel keeps its state on chip).
 */
int mk_workspace_init(void *workspace, size_t workspace_bytes, void *stream);
/*
 * Return the exchange area of a workspace initialised on the current device:
 * synchronises the device (every step that used it has finished), then frees
 * a batched area, or keeps a batch-1 (uncached) area as a spare that the next
 * mk_workspace_init reuses (uncached memory a kernel has read is never freed
 * while the process runs). The workspace must be initialised again before its
 * next step. A HIP graph that captured steps on the workspace holds the
 * area's address in its kernel arguments and a replay does not check it, so
 * release a workspace only after every such graph is destroyed, and never
 * during a stream capture (the device synchronisation fails there:
 * MK_ERR_HIP). Lifecycle counterpart of mk_workspace_init; no counterpart in
 * the reference.
 */
int mk_workspace_release(void *workspace);
/*
 * Synchronise `stream`, return the device error bits of `workspace` and clear
 * them. workspace == NULL: the sticky error bits of the current device's
 * allocation-free scratch (every faulted mk_decode_step_noalloc step since the
 * last such read; 0 before its first use), read and cleared with two small
 * copies (no allocation by this library).
 */
int mk_read_device_error(void *workspace, void *stream, uint32_t *bits_out);

/* The decode step (see mk_step_args). Asynchronous on the stream. */
int mk_decode_step(const mk_weights *w, const mk_step_args *a);

/*
 * Greedy decode loop: n_steps consecutive batch-1 decode steps in ONE
 * persistent launch, each step's token the previous step's argmax. No
 * counterpart in the reference, whose generation loop (NxDI, main.py:178-271)
 * launches one token-generation step per token; mk_decode_step is that seam.
 * Between steps the workgroups meet at an on-device barrier instead of a
 * kernel boundary, so the next step's layer-0 weights stream while the
 * slowest workgroups finish the lm_head, and no launch gap separates the
 * steps. Each step is the mk_decode_step computation (bitwise: same kernel
 * code, rows, order and rounding).
 *   a: as for mk_decode_step with batch 1, tokens[0] the first step's token
 *     (hidden_in must be NULL), a batch-1 workspace; positions pos[0] ..
 *     pos[0] + n_steps - 1 must lie below s_max and rope_rows; logits (if
 *     given) receive the last step's, next_token (if given) the last step's
 *     token; MK_FLAG_ADVANCE advances pos by n_steps.
 *   tokens_out: device int32 [n_steps], the token each step produced, or NULL.
 *   step_clock: device uint64 [n_steps + 1], or NULL: the device wall clock
 *     (mk_wall_clock_hz) at the launch's start, when step n's token was known
 *     to workgroup 0 (entry n + 1, n < n_steps - 1), and when the launch
 *     ended (entry n_steps): entry differences are per-step latencies.
 *   MK_ERR_UNSUPPORTED for batch > 1, hidden_in, MK_FLAG_PREFILL or a batched
 *   workspace; MK_ERR_NULL without w->norm_final (every step runs the lm_head).
 *   Asynchronous on the stream; allocates nothing.
 */
int mk_decode_loop(const mk_weights *w, const mk_step_args *a, int32_t n_steps, int32_t *tokens_out,
                   uint64_t *step_clock);

/*
 * Allocation-free variant of mk_decode_step. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc), so it takes
 * no workspace and needs no mk_workspace_init.
 *   The kernel's scratch (the control block and both sets of per-layer
 *   exchange buffers of the batch-1 kernel) is a static device array inside
 *   the library, MK_NOALLOC_SCRATCH_BYTES per device, held until the process
 *   ends. The library looks its address up on its first call on a device and
 *   fills it there (a fill kernel on `stream`; repeated on the next call if
 *   that first call was under stream capture). Nothing is allocated or freed.
 *   Same arguments and results as mk_decode_step, except:
 *     - batch must be 1 (MK_ERR_SHAPE otherwise) and MK_FLAG_PREFILL is
 *       refused (MK_ERR_UNSUPPORTED): the scratch holds batch-1 buffers only;
 *     - workspace must be NULL and workspace_bytes 0 (MK_ERR_WORKSPACE);
 *     - device-detected faults (MK_DEVERR_*): a faulted step writes
 *       next_token[0] = -1 (if next_token is given), does not advance pos,
 *       and ORs its bits into a sticky word of the scratch that
 *       mk_read_device_error(NULL, stream, &bits) returns and clears, so a
 *       step without next_token (the layer-stack seam) reports its faults too.
 *   Every call of this entry point on one device shares that device's
 *   scratch, and each call leaves it ready for the next: calls that overlap
 *   in time on one device (e.g. on two unordered streams) race and give
 *   wrong results. Order them (one stream, or events).
 */
#define MK_NOALLOC_SCRATCH_BYTES 3277056
int mk_decode_step_noalloc(const mk_weights *w, const mk_step_args *a);

/*
 * Context encoding (prefill) of one sequence: the K/V rows of n_tokens
 * consecutive prompt tokens at positions start_pos .. start_pos + n_tokens - 1,
 * written into every requested layer's cache, each token attending causally
 * to rows [0, its position] (rows below start_pos must hold the sequence's
 * earlier K/V). Counterpart of the reference's context-encoding pass, which
 * runs its baseline decoder layers over the prompt (llama_with_megakernel.py:
 * 194-204; the layer at llama.py:1039-1139), and of mk_decode_step's
 * MK_FLAG_PREFILL path, which runs at most 32 tokens per launch of the decode
 * megakernel: this entry point runs layer by layer (RMSNorm, QKV GEMM with
 * RoPE, causal attention, O GEMM, RMSNorm, gate/up GEMM with SwiGLU, down GEMM)
 * on the matrix cores, in chunks as large as the workspace holds, so each
 * layer's weights stream once per chunk. Same rounding points as the decode
 * step; the attention keeps p = exp(s - running max) rounded to bf16 for the
 * PV product.
 *   tokens: device int32 [n_tokens]; k_cache[i] / v_cache[i]: layer
 *     first_layer + i of ONE sequence, bf16 [8][s_max][64];
 *     0 <= start_pos, start_pos + n_tokens <= s_max <= rope_rows.
 *   hidden_out: bf16 [n_tokens][2048], the hidden state after the last layer
 *     (before the final norm), or NULL (the last layer then runs its QKV
 *     GEMM only).
 *   workspace: device memory of at least mk_prefill_workspace_bytes(c)
 *     bytes, 256-byte aligned, for chunks of c tokens (the entry point takes
 *     the largest multiple of 16 the given size holds, up to 16384): one
 *     layer's activations of a chunk (36,864 bytes per token) and a fixed
 *     16 MiB of fp32 split-K partials; no initialisation, contents not kept
 *     between calls.
 *   Uses the MFMA-tiled weight copies when all of t_qkv, t_o, t_gu, t_down
 *   are set, else the row-major stacks. Asynchronous on `stream`; no
 *   allocation; every launch is an ordinary kernel (capturable).
 */
typedef struct mk_prefill_args {
    int32_t first_layer;
    int32_t n_layers;
    int32_t n_tokens;
    int32_t start_pos;
    int32_t s_max;
    const int32_t *tokens;
    void *const *k_cache;
    void *const *v_cache;
    void *hidden_out;
    void *workspace;
    size_t workspace_bytes;
    void *stream;
} mk_prefill_args;
size_t mk_prefill_workspace_bytes(int32_t chunk_tokens);
int mk_prefill(const mk_weights *w, const mk_prefill_args *a);

/*
 * Single-layer step (transformer_llama_megakernel_1layer,
 * transformer_llama.py:154-191): layer `layer` of the stacks applied to
 * hidden_in, result in hidden_out, K/V row pos[b] written in place.
 */
int mk_layer_step(const mk_weights *w, int32_t layer, int32_t batch, int32_t s_max,
                  void *k_cache, void *v_cache, const void *hidden_in, int32_t *pos,
                  void *hidden_out, void *workspace, size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* MK_H_ */
