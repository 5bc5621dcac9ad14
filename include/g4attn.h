/*
 * g4attn.h — C ABI of the MI355X (gfx950) Gemma-4 attention library.
 *
 * Drop-in replacement for gemma4-webgpu's attention kernels: the six WGSL
 * shaders registered in src/shaders.ts:43-74 and dispatched from
 * src/engine.ts:2056-2095, plus the fused decode and prefill paths that the
 * WGSL engine does not have. All signatures use plain pointers, sizes and POD
 * structs; device buffers are opaque `void*` device addresses owned by the
 * caller (the engine), as GPUBuffers are owned by GemmaEngineImpl
 * (src/engine.ts:1347-1426) and only borrowed by the kernels.
 *
 * Conventions
 *   - Every entry point returns 0 (G4_OK) or a negative status. The message of
 *     the last failure on the calling thread is returned by g4_last_error().
 *     WebGPU validation errors are asynchronous and silent; here a bad argument
 *     is rejected before anything is enqueued.
 *   - `stream` is a hipStream_t (NULL = the null stream). Kernel entry points
 *     only enqueue; they never synchronise the host. Prepare calls upload
 *     their tables through pinned staging slots, copied to the workspace by
 *     a kernel on `stream`; a slot is reused only once the copy reading it has
 *     completed, and a thread's ring grows instead of waiting, up to 4096
 *     uploads in flight.
 *   - Per-token fields (position, slot, seq_len) are passed by value and
 *     captured at enqueue time. This gives the ordering WebGPU provides with
 *     queue.writeBuffer before a later submit (src/engine.ts:1967-1987) without
 *     mutable device uniforms, so two forwards may be in flight at once.
 *   - Work vectors q/k/v/out are f32 [heads][head_dim] (src/engine.ts:1369-1371).
 *     KV caches are f16 (IEEE binary16, round-to-nearest-even on store),
 *     slot-major [max_seq][num_kv_heads][head_dim] (kv_cache_store.wgsl:15);
 *     the WGSL caches hold the same layout in f32.
 *   - Weights (q_norm / k_norm) and the rope_freqs table are f16, as the
 *     reference binds them (fused_per_head_norm_rope.wgsl:15,17).
 */
#ifndef G4ATTN_H
#define G4ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status ----------------------------------------------------------- */
#define G4_OK 0
#define G4_EINVAL (-1)  /* bad argument, rejected before enqueue */
#define G4_EHIP (-2)    /* HIP runtime error */
#define G4_ENOSPC (-3)  /* caller-provided workspace too small */
#define G4_ENODEV (-4)  /* no usable gfx950 device */
#define G4_ERANGE (-5)  /* a prepared plan was advanced past its limit: prepare it again */

/* Message for the last non-zero status returned on this thread. */
const char* g4_last_error(void);
/* Library version string. */
const char* g4_version(void);

/* ---- device, streams, buffers ----------------------------------------- *
 * Replace initWebGPU / device.createBuffer / queue.writeBuffer / mapAsync
 * (src/engine.ts:350-353, 402-437, 1347-1426, 2309).                       */
int g4_device_count(int* count);
int g4_set_device(int device);
int g4_stream_create(void** stream);
int g4_stream_destroy(void* stream);
int g4_stream_synchronize(void* stream);
int g4_malloc(void** dev_ptr, size_t bytes);
int g4_free(void* dev_ptr);
/* queue.writeBuffer(buffer, offset, data): host -> device, ordered on stream. */
int g4_upload(void* dev_dst, size_t offset, const void* host_src, size_t bytes, void* stream);
/* copyBufferToBuffer + mapAsync: device -> host; returns after the copy is done. */
int g4_download(void* host_dst, const void* dev_src, size_t offset, size_t bytes, void* stream);
/* The same readback in two halves, for callers that wait off their issuing
 * thread (mapAsync's promise): begin enqueues the copy into pinned staging
 * memory on `stream`, ordered after the work already enqueued there, and
 * returns a handle; finish, from any thread, waits for that copy, writes the
 * bytes to host_dst (NULL: discard them) and releases the handle. Every
 * begun readback must be finished exactly once. */
typedef struct g4_readback g4_readback;
int g4_readback_begin(const void* dev_src, size_t offset, size_t bytes, void* stream, g4_readback** handle);
int g4_readback_finish(g4_readback* handle, void* host_dst);
/* Timestamp queries for labelled passes: the engine's GPUQuerySet of type
 * 'timestamp' (created in enableProfile, src/engine.ts:3089-3110), written at
 * each pass's beginning and end (timestampWrites, :3208-3227) and resolved
 * after submit (resolveQuerySet + mapAsync, :3253-3288). A set holds `count`
 * slots (1 .. 65536); a pass uses a pair (slot, slot+1).
 * begin_pass opens a pass on the calling thread (one at a time): every kernel
 * the library launches from this thread until end_pass carries the pair on its
 * own dispatch, the first kernel's start in `slot` and the last one's end in
 * slot+1 (no packet is added between kernels); keep passes closed around code
 * under HIP graph capture. write instead records a marker
 * for one slot on `stream`, in stream order (a few microseconds of GPU time
 * each). resolve waits, from any thread, for n_pairs pairs from slot `first`
 * and writes ns_out[i] = the time from slot first+2i to slot first+2i+1 in
 * nanoseconds, or NaN where either slot was not written since the last resolve
 * of it (a pass that launched nothing); the resolved slots may then be written
 * again. A set has at most one open pass, on any thread. Each call sees the
 * others, whatever their threads: resolve refuses the slots of the open pass,
 * begin_pass and write refuse slots being resolved, and destroy refuses a set
 * with a pass open on another thread or a resolve under way (G4_EINVAL). */
typedef struct g4_query_set g4_query_set;
int g4_query_set_create(uint32_t count, g4_query_set** out);
int g4_query_begin_pass(g4_query_set* set, uint32_t slot);
int g4_query_end_pass(void);
int g4_query_write(g4_query_set* set, uint32_t slot, void* stream);
int g4_query_resolve(g4_query_set* set, uint32_t first, uint32_t n_pairs, double* ns_out);
int g4_query_set_destroy(g4_query_set* set);
/* Measurement hook (no counterpart in the reference): the device's read-stream
 * ceiling. Streams `bytes` of buf with nontemporal 16-byte loads (the decode
 * kernels' load form) and writes nothing (sink is only a guard against the
 * loads being dropped); the two events, when given (created with timing),
 * record the kernel's own start and end. bytes / elapsed is the ceiling that
 * a kernel's achieved bandwidth is compared with, next to the spec sheet. */
int g4_read_ceiling(const void* buf, size_t bytes, uint32_t* sink, void* stream, void* start_event, void* stop_event);
/* Zero `bytes` at dev_dst with a fill kernel (safe inside HIP graph capture). */
int g4_zero(void* dev_dst, size_t bytes, void* stream);

/* ---- Params: the reference's uniform structs, field for field -------- */

/* fused_per_head_norm_rope.wgsl:13; built at src/engine.ts:583-588 */
typedef struct g4_norm_rope_params {
    uint32_t num_heads;
    uint32_t head_dim;
    float eps;
    uint32_t position;
    float theta;
    uint32_t apply_divisor;
} g4_norm_rope_params;

/* per_head_rms_norm_no_weight.wgsl:8; built at src/engine.ts:539-541 */
typedef struct g4_norm_params {
    uint32_t num_heads;
    uint32_t head_dim;
    float eps;
    uint32_t pad;
} g4_norm_params;

/* kv_cache_store.wgsl:1; built at src/engine.ts:548-550 */
typedef struct g4_kv_store_params {
    uint32_t num_kv_heads;
    uint32_t head_dim;
    uint32_t position; /* cache slot */
    uint32_t max_seq_len;
} g4_kv_store_params;

/* attn_score.wgsl:9; built at src/engine.ts:562-567 */
typedef struct g4_attn_score_params {
    uint32_t num_q_heads;
    uint32_t num_kv_heads;
    uint32_t head_dim;
    uint32_t seq_len;
    float scale;
    uint32_t sliding_window; /* 0 = full attention */
} g4_attn_score_params;

/* softmax.wgsl:1; built at src/engine.ts:493 */
typedef struct g4_softmax_params {
    uint32_t num_heads;
    uint32_t seq_len;
} g4_softmax_params;

/* attn_output.wgsl:1; built at src/engine.ts:568-570 */
typedef struct g4_attn_output_params {
    uint32_t num_q_heads;
    uint32_t num_kv_heads;
    uint32_t head_dim;
    uint32_t seq_len;
} g4_attn_output_params;

/* ---- the six reference kernels (registry names in src/shaders.ts:43-74) - *
 * Same semantics, grids and reduction order as the WGSL; f16 caches.      */

/* SHADERS.fusedPerHeadNormRope — fused_per_head_norm_rope.wgsl:20-64,
 * dispatched at src/engine.ts:2078-2085. In place on data[num_heads*head_dim]. */
int g4_fused_per_head_norm_rope(float* data, const uint16_t* weight, const uint16_t* rope_freqs,
                                g4_norm_rope_params p, void* stream);

/* SHADERS.perHeadRmsNormNoWeight — per_head_rms_norm_no_weight.wgsl:13-38,
 * dispatched at src/engine.ts:2060-2066. In place. */
int g4_per_head_rms_norm_no_weight(float* data, g4_norm_params p, void* stream);

/* SHADERS.kvCacheStore — kv_cache_store.wgsl:8-18, dispatched at
 * src/engine.ts:2089-2091. Writes row p.position of the f16 caches. */
int g4_kv_cache_store(const float* k_in, const float* v_in, uint16_t* k_cache, uint16_t* v_cache,
                      g4_kv_store_params p, void* stream);

/* SHADERS.attnScore — attn_score.wgsl:15-40, dispatched at src/engine.ts:2092.
 * scores[num_q_heads][seq_len] (head stride = seq_len). */
int g4_attn_score(const float* q, const uint16_t* k_cache, float* scores, g4_attn_score_params p,
                  void* stream);

/* SHADERS.softmax — softmax.wgsl:7-46, dispatched at src/engine.ts:2093. In place. */
int g4_softmax(float* scores, g4_softmax_params p, void* stream);

/* SHADERS.attnOutput — attn_output.wgsl:7-23, dispatched at src/engine.ts:2094. */
int g4_attn_output(const float* probs, const uint16_t* v_cache, float* out, g4_attn_output_params p,
                   void* stream);

/* ---- fused producer-side prep ----------------------------------------- *
 * One launch for the vNorm -> fusedNormRope(Q, K) -> kvCacheStore sequence
 * of src/engine.ts:2056-2091. Results are bit-identical to running the four
 * reference kernels in that order. On KV-consumer layers (store_kv = 0, the
 * layers that read a producer's cache, src/engine.ts:1518-1522) only Q is
 * normalised and rotated and k/v/caches may be NULL.                        */
typedef struct g4_prep_params {
    uint32_t num_q_heads;
    uint32_t num_kv_heads;
    uint32_t head_dim;
    float eps;
    uint32_t position;      /* RoPE position */
    float theta;
    uint32_t apply_divisor; /* 1 on global layers: divide by rope_freqs[i] */
    uint32_t slot;          /* cache row written (== position without a ring) */
    uint32_t max_seq_len;
    uint32_t store_kv;      /* 1 on producer layers */
} g4_prep_params;

int g4_attn_prep(float* q, float* k, float* v, const uint16_t* q_weight, const uint16_t* k_weight,
                 const uint16_t* rope_freqs, uint16_t* k_cache, uint16_t* v_cache, g4_prep_params p,
                 void* stream);

/* Many layers' prep in one launch. `layers` is a DEVICE array of n_layers
 * entries, built once by the engine (as bind groups are built once at init,
 * src/engine.ts:1428-1923); position and slot are the per-token values.
 * Grid: (num_q_heads + 2*num_kv_heads) x n_layers workgroups. The table is
 * trusted: head_dim must be even and every pointer valid for its layer. A
 * layer whose max_seq_len <= slot skips the store.                         */
typedef struct g4_prep_layer {
    float* q;
    float* k;
    float* v;
    const uint16_t* q_weight;
    const uint16_t* k_weight;
    const uint16_t* rope_freqs;
    uint16_t* k_cache;
    uint16_t* v_cache;
    uint32_t head_dim;
    float theta;
    uint32_t apply_divisor;
    uint32_t store_kv;
    uint32_t max_seq_len;
    uint32_t reserved[3];
} g4_prep_layer;

int g4_attn_prep_many(const g4_prep_layer* layers, uint32_t n_layers, uint32_t num_q_heads,
                      uint32_t num_kv_heads, float eps, uint32_t position, uint32_t slot, void* stream);

/* ---- fused decode attention (attnScore -> softmax -> attnOutput) ------- *
 * Flash-decoding on MFMA: one pass over the K/V rows of the attended range
 * (the whole cache on global layers, the last sliding_window rows on local
 * layers), split across workgroups, merged with a fixed-order log-sum-exp.
 * out[num_q_heads][head_dim] equals the reference chain's attnOut within
 * floating-point rounding. Requires head_dim 256 or 512 and
 * num_q_heads / num_kv_heads <= 8; out 16-byte aligned. The workspace holds the split partials;
 * g4_attn_decode_workspace_size gives the bytes needed for seq_len up to
 * max_seq_len (allocate once, like attnScores at src/engine.ts:1375).      */
int g4_attn_decode_workspace_size(uint32_t num_q_heads, uint32_t num_kv_heads, uint32_t head_dim,
                                  uint32_t max_seq_len, size_t* bytes);
int g4_attn_decode(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out,
                   g4_attn_score_params p, void* workspace, size_t workspace_bytes, void* stream);

/* The same decode with no workspace argument and no allocation (no hipMalloc,
 * hipFree or allocating library call), for callers that cannot allocate:
 * code under HIP graph capture, tight serving loops. No counterpart in the
 * reference. The split partials live in a fixed device array of the library
 * (8.03 MiB per GPU, held until the process ends): num_q_heads <= 8, and at
 * most 512 splits (the split size grows for longer ranges). Every call on a
 * GPU uses that GPU's one array, so calls that overlap on one GPU (on
 * different streams, or from different threads) race; calls ordered on one
 * stream do not. Same results as g4_attn_decode where both pick the same
 * split size. */
int g4_attn_decode_noalloc(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out,
                           g4_attn_score_params p, void* stream);

/* ---- many independent decode problems in one launch ------------------- *
 * Each entry is one (query block, KV cache, length) problem: the layers of
 * one token's attention stack when their queries are available together, or
 * the sequences of a ragged batch (each with its own cache and length; the
 * engine has one sequence, src/engine.ts:116, so batching is new here).
 * Splits are sized so the whole set fills the GPU; ragged lengths get
 * proportional numbers of workgroups.                                       */
typedef struct g4_decode_entry {
    const float* q;          /* [num_q_heads][head_dim] f32 */
    const uint16_t* k_cache; /* f16 [rows][num_kv_heads][head_dim] */
    const uint16_t* v_cache;
    float* out;              /* [num_q_heads][head_dim] f32, 16-byte aligned */
    uint32_t seq_len;        /* valid rows */
    uint32_t sliding_window; /* 0 = full */
    float scale;
    uint32_t reserved;
} g4_decode_entry;

/* Workspace for up to n_entries problems attending total_rows rows in all. */
int g4_attn_decode_many_workspace_size(uint32_t n_entries, uint32_t num_q_heads, uint32_t num_kv_heads,
                                       uint32_t head_dim, uint64_t total_rows, size_t* bytes);

/* A prepared launch: the split table lives in the workspace. Prepare when the
 * entries change (each token, as the engine rewrites seq_len uniforms each
 * token, src/engine.ts:1980-1987); run as often as wanted. Running a plan
 * while another prepare on the same workspace is pending is a race. */
typedef struct g4_decode_plan {
    uint64_t opaque[8];
} g4_decode_plan;

int g4_attn_decode_many_prepare(const g4_decode_entry* entries, uint32_t n_entries, uint32_t num_q_heads,
                                uint32_t num_kv_heads, uint32_t head_dim, void* workspace, size_t workspace_bytes,
                                g4_decode_plan* plan, void* stream);
int g4_attn_decode_many_run(const g4_decode_plan* plan, void* stream);
/* The two launches of g4_attn_decode_many_run, separately: the split pass,
 * then the log-sum-exp merge of entries with more than one split. */
int g4_attn_decode_many_run_split(const g4_decode_plan* plan, void* stream);
int g4_attn_decode_many_run_merge(const g4_decode_plan* plan, void* stream);
/* prepare + run. */
int g4_attn_decode_many(const g4_decode_entry* entries, uint32_t n_entries, uint32_t num_q_heads,
                        uint32_t num_kv_heads, uint32_t head_dim, void* workspace, size_t workspace_bytes,
                        void* stream);

/* ---- RoPE inverse frequencies ---------------------------------------------
 * inv_freq[i] = f32(1 / pow(theta, 2i/head_dim)) (divided by rope_freqs[i]
 * when apply_divisor), i < head_dim/2: the position-independent factor of
 * the angle in fused_per_head_norm_rope.wgsl:50-54, bit-identical to what
 * g4_fused_per_head_norm_rope evaluates. A model has one table per RoPE
 * configuration (Gemma 4: local theta 1e4; global theta 1e6 with the
 * proportional divisor); compute them once and pass them in g4_step_entry. */
int g4_rope_inv_freq(float theta, uint32_t head_dim, uint32_t apply_divisor, const uint16_t* rope_freqs,
                     float* inv_freq, void* stream);
/* The same table computed on the host from host copies of the divisor table
 * (what g4_step_entry.rope_inv_freq_host takes). Bit-identical to the device
 * version. */
int g4_rope_inv_freq_host(float theta, uint32_t head_dim, uint32_t apply_divisor, const uint16_t* rope_freqs_host,
                          float* inv_freq_host);

/* ---- one-launch decode step ---------------------------------------------
 * The whole attention block of one token for many layers or sequences in one
 * launch: per entry, q RMSNorm + RoPE, the current row's k (norm + RoPE) and v
 * (weightless norm), the f16 store of that row (store_kv = 1, KV-producer
 * layers), and split-K attention over the attended rows with the current row
 * taken from registers. KV-consumer layers (src/engine.ts:1518-1522) read
 * their producer's cache with store_kv = 0, in one of two ways: with their
 * producer's raw k/v and k_weight, when the producer's entry runs in the same
 * launch (the current row is recomputed, bit-identical to the stored one); or
 * with k, v and k_weight NULL, when the producer's step already stored the
 * row (the engine's layer-by-layer order, where consumers project only q):
 * the current row is then read from the cache like the others. It replaces the dispatch sequence
 * vNorm, fusedNormRopeQK, kvCacheStore, attnScore, softmax, attnOutput of
 * src/engine.ts:2056-2094. Unlike the reference kernels, q/k/v are read
 * only (the raw projections stay in their buffers); attnOut is written.
 * Work is split evenly over the GPU across all entries. head_dim 256 or
 * 512 (one per call), up to 8 query heads per kv head. Prepare when the entries change (each
 * token); run as often as wanted. */
typedef struct g4_step_entry {
    const float* q;            /* raw projection [num_q_heads][head_dim] f32 */
    const float* k;            /* raw projection [num_kv_heads][head_dim] f32; NULL: the current row is */
    const float* v;            /* already in the cache (k, v, k_weight all NULL, store_kv 0) */
    const uint16_t* q_weight;  /* attn_q_norm, f16 [head_dim] */
    const uint16_t* k_weight;  /* attn_k_norm, f16 [head_dim] */
    const uint16_t* rope_freqs; /* f16 divisor table, read when apply_divisor */
    const float* rope_inv_freq_host; /* optional HOST [head_dim/2] table from g4_rope_inv_freq_host for
                                        this entry's theta/divisor (computed once, at load): prepare then
                                        evaluates the RoPE factors on the host; NULL: in the kernel */
    uint16_t* k_cache;         /* f16 [rows][num_kv_heads][head_dim]; rows < seq_len - 1 hold earlier tokens */
    uint16_t* v_cache;
    float* out;                /* attnOut [num_q_heads][head_dim] f32, 16-byte aligned */
    uint32_t seq_len;          /* rows including the current token's (its row is seq_len - 1) */
    uint32_t position;         /* RoPE position of the current token */
    uint32_t sliding_window;   /* 0 = full */
    uint32_t store_kv;         /* 1: write the current row to the caches */
    float theta;
    uint32_t apply_divisor;
    float scale;               /* attention scale (1.0 for Gemma 4) */
    float eps;
    uint32_t q_ready;          /* 1: q already holds the post-norm, post-RoPE query (what
                                  fused_per_head_norm_rope.wgsl leaves in it; g4_linear_qkv_prep's output):
                                  the step reads it as is; q_weight is then not read */
} g4_step_entry;

int g4_attn_step_workspace_size(uint32_t n_entries, uint32_t num_q_heads, uint32_t num_kv_heads, uint32_t head_dim,
                                size_t* bytes);
int g4_attn_step_prepare(const g4_step_entry* entries, uint32_t n_entries, uint32_t num_q_heads,
                         uint32_t num_kv_heads, uint32_t head_dim, void* workspace, size_t workspace_bytes,
                         g4_decode_plan* plan, void* stream);
int g4_attn_step_run(const g4_decode_plan* plan, void* stream);
/* The next token without a new prepare: every entry of the plan (every
 * layer of the stack, every sequence of the batch) moves `tokens` decode steps
 * ahead, seq_len and position both growing by `tokens`, the current row being
 * the new last one, as the engine rewrites the position, slot and seq_len
 * uniforms every token (src/engine.ts:1967-1987). Host-only: it changes the
 * plan and enqueues nothing, so a decode loop's per-token host work is this
 * call and the launches. The plan keeps its partition: the part holding the
 * last row takes the new rows of a full-attention entry, and a windowed
 * entry's parts slide with its window. The RoPE factors of later positions
 * are evaluated in the kernel from the inverse frequencies of the entry's
 * rope_inv_freq_host table (uploaded by the prepare), in f64 rounded to f32,
 * as the prepare evaluates the prepared position's; entries without a host
 * table evaluate theirs in the kernel at every position anyway. The caches
 * must hold the new rows, as for a prepare. At most 4096 tokens per prepare
 * (G4_ERANGE beyond; prepare again to rebalance the parts: every 32 tokens
 * add one 32-row tile to the part holding the last row of a full-attention
 * entry). Works on plans of g4_attn_step_prepare and of
 * g4_attn_step_prepare_layers (advance each layer's plan). */
int g4_attn_step_advance(g4_decode_plan* plan, uint32_t tokens);
/* The two launches of g4_attn_step_run, separately: the attention pass (one
 * kernel for all entries), then the log-sum-exp merge of entries spread over
 * more than one workgroup (nothing when there are none). */
int g4_attn_step_run_attention(const g4_decode_plan* plan, void* stream);
int g4_attn_step_run_merge(const g4_decode_plan* plan, void* stream);
/* Measurement hook (the reference times passes with WebGPU timestamp
 * queries, src/engine.ts:131-135, 411-414): the attention launch of
 * g4_attn_step_run_attention with two hipEvent_t (created with timing enabled)
 * that record the kernel's own start and end. */
int g4_attn_step_run_attention_timed(const g4_decode_plan* plan, void* stream, void* start_event, void* stop_event);
/* A token of a model with two head_dims (E2B: 512 on the global layers, 256
 * on the local ones) has one plan per head_dim. These run both plans' attention
 * passes as one launch: the head_dim-512 plan's workgroups first, then the
 * head_dim-256 plan's, which take the CUs the first ones leave (one launch and
 * its start-up instead of two, and the short local layers in the long global
 * ones' tail). The plans (either order) come from separate prepares with
 * separate workspaces. Each plan's merge then runs as usual
 * (g4_attn_step_run_merge); g4_attn_step_run_pair does all three. The
 * head_dim-256 entries are computed by 4-wave workgroups whatever the plan's
 * own form, so their results agree with g4_attn_step_run's to rounding, not
 * bit for bit, when that plan took 8-wave workgroups. No counterpart in the
 * reference (one dispatch per kernel per layer, src/engine.ts:2056-2095). */
int g4_attn_step_run_attention_pair(const g4_decode_plan* plan_1, const g4_decode_plan* plan_2, void* stream);
int g4_attn_step_run_attention_pair_timed(const g4_decode_plan* plan_1, const g4_decode_plan* plan_2, void* stream,
                                          void* start_event, void* stop_event);
int g4_attn_step_run_pair(const g4_decode_plan* plan_1, const g4_decode_plan* plan_2, void* stream);
/* prepare + run. */
int g4_attn_step(const g4_step_entry* entries, uint32_t n_entries, uint32_t num_q_heads, uint32_t num_kv_heads,
                 uint32_t head_dim, void* workspace, size_t workspace_bytes, void* stream);
/* One token's layers in the engine's order (src/engine.ts:2029-2156: per
 * layer q/k/v projection, attention block, output projection, each layer's
 * input the previous layer's output), prepared together: the engine patches
 * every layer's position, slot and seq_len uniforms once per token
 * (src/engine.ts:1967-1987) and then runs the layers one by one. Layer i is
 * entries[i * entries_per_layer .. (i + 1) * entries_per_layer) (one entry
 * per layer for the engine's single sequence; a batch of sequences per layer
 * for a batched decode) and becomes plans[i], a plan of that layer alone
 * (partitioned as g4_attn_step_prepare would partition it, so that each layer
 * fills the GPU when it runs); every layer's tables go up in one upload, and
 * layers at one (inverse-frequency table, position) pair share one set of
 * RoPE factors. Each plan is run with g4_attn_step_run_attention followed by
 * g4_attn_step_run_merge or g4_attn_step_run_out (or g4_attn_step_run), in
 * layer order, as often as wanted until the next prepare into the same
 * workspace; the layers' partial records are separate. One head_dim per call
 * (E2B: one call per head_dim group). A failed call leaves every plan
 * unprepared. Workspace: g4_attn_step_layers_workspace_size (enough for any
 * smaller entries_per_layer too). */
int g4_attn_step_layers_workspace_size(uint32_t n_layers, uint32_t entries_per_layer, uint32_t num_q_heads,
                                       uint32_t num_kv_heads, uint32_t head_dim, size_t* bytes);
int g4_attn_step_prepare_layers(const g4_step_entry* entries, uint32_t n_layers, uint32_t entries_per_layer,
                                uint32_t num_q_heads, uint32_t num_kv_heads, uint32_t head_dim, void* workspace,
                                size_t workspace_bytes, g4_decode_plan* plans, void* stream);

/* ---- causal prefill on MFMA ---------------------------------------------
 * The reference runs a prompt as one decode step per token (src/engine.ts:
 * 2469-2475); this computes the same attention for a chunk of tokens at once.
 * Token t of an entry sits at position start + t and attends cache rows
 * [lo, start + t], lo = start + t + 1 - sliding_window on local layers
 * (0 when that is negative or the window is 0): out[t] equals the decode step
 * at that position (attn_score.wgsl -> softmax.wgsl -> attn_output.wgsl)
 * within f32/f16 rounding. q is the post norm + RoPE query in f16; the
 * caches already hold the chunk's own K/V rows. Several entries (chunks,
 * layers, sequences) go in one launch. head_dim 256 or 512 (one per call),
 * 32 % (num_q_heads / num_kv_heads) == 0. The prepare splits long query tiles'
 * key ranges into parts and spreads the work over one workgroup per CU;
 * parts of a tile are merged by a second launch. A plan runs as often as
 * wanted; runs on one workspace must not overlap. */
typedef struct g4_prefill_entry {
    const uint16_t* q;        /* f16 [n_tokens][num_q_heads][head_dim] */
    const uint16_t* k_cache;  /* f16 [rows][num_kv_heads][head_dim], rows >= start + n_tokens */
    const uint16_t* v_cache;
    float* out;               /* f32 [n_tokens][num_q_heads][head_dim], 16-byte aligned */
    uint32_t n_tokens;
    uint32_t start;           /* position of token 0 */
    uint32_t sliding_window;  /* 0 = full */
    float scale;              /* attention scale (1.0 for Gemma 4) */
    const uint16_t* vt_cache; /* optional: v_cache's rows as V^T blocks [num_kv_heads][ceil(vt_rows / 32)]
                                 [head_dim][32] f16, written by g4_attn_prompt_prep_vt; every row the entry
                                 attends must have been stored there (rows a decode step stores are not).
                                 NULL: every prefill call transposes the attended rows into its workspace */
    uint32_t vt_rows;         /* rows the V^T cache was sized for (the prompt prep's max_seq_len) */
} g4_prefill_entry;

int g4_attn_prefill_workspace_size(const g4_prefill_entry* entries, uint32_t n_entries, uint32_t num_q_heads,
                                   uint32_t num_kv_heads, uint32_t head_dim, size_t* bytes);
int g4_attn_prefill_prepare(const g4_prefill_entry* entries, uint32_t n_entries, uint32_t num_q_heads,
                            uint32_t num_kv_heads, uint32_t head_dim, void* workspace, size_t workspace_bytes,
                            g4_decode_plan* plan, void* stream);
int g4_attn_prefill_run(const g4_decode_plan* plan, void* stream);
/* Measurement hook: g4_attn_prefill_run with two hipEvent_t (timing enabled)
 * that record the attention kernel's own start and end (the merge, when the
 * plan has one, follows untimed). */
int g4_attn_prefill_run_timed(const g4_decode_plan* plan, void* stream, void* start_event, void* stop_event);
/* prepare + run. */
int g4_attn_prefill(const g4_prefill_entry* entries, uint32_t n_entries, uint32_t num_q_heads, uint32_t num_kv_heads,
                    uint32_t head_dim, void* workspace, size_t workspace_bytes, void* stream);

/* ---- chunked prompt prep ----------------------------------------------------
 * The producer-side prep of every token of a prompt chunk in one launch: the
 * engine runs vNorm -> fusedNormRope(Q, K) -> kvCacheStore once per prompt
 * token (src/engine.ts:2460-2479, each through 2056-2091). Token t sits at
 * position (and cache row) start + t. Per token: q (norm with q_weight +
 * RoPE) written to q_out as f16 (the query g4_attn_prefill takes); on
 * producer layers (store_kv) k (norm with k_weight + RoPE) and v (weightless
 * norm) stored as f16 rows start + t of the caches. Every value is the f16
 * rounding of what fused_per_head_norm_rope.wgsl / per_head_rms_norm_no_weight
 * .wgsl compute for that token, bit for bit. q, k, v are read only.        */
typedef struct g4_prompt_prep_params {
    uint32_t num_q_heads;
    uint32_t num_kv_heads;
    uint32_t head_dim;       /* 256 or 512 */
    uint32_t n_tokens;
    uint32_t start;          /* position of token 0 */
    float eps;
    float theta;
    uint32_t apply_divisor;  /* 1 on global layers: divide by rope_freqs[i] */
    uint32_t store_kv;       /* 1 on producer layers */
    uint32_t max_seq_len;    /* cache rows (start + n_tokens <= max_seq_len when store_kv) */
} g4_prompt_prep_params;

/* q: f32 [n_tokens][num_q_heads][head_dim]; k, v: f32 [n_tokens][num_kv_heads][head_dim]
 * (NULL with store_kv 0); q_out: f16 [n_tokens][num_q_heads][head_dim].
 * rope_inv_freq: optional device [head_dim/2] table from g4_rope_inv_freq for
 * this layer's theta / divisor (computed once, at load; the same bits as the
 * kernel's own evaluation); NULL: every workgroup evaluates the reference's
 * f64 pow itself. */
int g4_attn_prompt_prep(const float* q, const float* k, const float* v, const uint16_t* q_weight,
                        const uint16_t* k_weight, const uint16_t* rope_freqs, const float* rope_inv_freq,
                        uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache, g4_prompt_prep_params p,
                        void* stream);
/* The same, also writing the stored V rows into vt_cache, V^T in 32-row blocks
 * [num_kv_heads][ceil(max_seq_len / 32)][head_dim][32] f16 (row r, element d
 * at [h][r / 32][d][r % 32]): the layout g4_attn_prefill reads V in
 * (g4_prefill_entry.vt_cache), kept beside the cache so that a prompt run as
 * chunks transposes each row once rather than at every chunk's prefill. The
 * rows of the chunk's last block past its end are written as 0 (the next
 * chunk's prep overwrites them). No counterpart in the reference, whose
 * attn_output.wgsl reads V row by row (src/engine.ts:2094). store_kv 1. */
int g4_attn_prompt_prep_vt(const float* q, const float* k, const float* v, const uint16_t* q_weight,
                           const uint16_t* k_weight, const uint16_t* rope_freqs, const float* rope_inv_freq,
                           uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache, uint16_t* vt_cache,
                           g4_prompt_prep_params p, void* stream);
/* Several chunks' preps in one launch: chunks of several sequences in a
 * batched prefill (or several layers whose inputs are all ready), one
 * head_dim for all. Entry i is exactly the call g4_attn_prompt_prep (vt_cache
 * NULL) or g4_attn_prompt_prep_vt (vt_cache set) with its arguments, and gives
 * the same bits; the entries' outputs must not overlap. At most 8 entries.
 * No counterpart in the reference (one token per dispatch, src/engine.ts:
 * 2460-2479). */
typedef struct g4_prompt_prep_entry {
    const float* q;
    const float* k;
    const float* v;
    const uint16_t* q_weight;
    const uint16_t* k_weight;
    const uint16_t* rope_freqs;
    const float* rope_inv_freq;
    uint16_t* q_out;
    uint16_t* k_cache;
    uint16_t* v_cache;
    uint16_t* vt_cache;
    g4_prompt_prep_params p;
} g4_prompt_prep_entry;
int g4_attn_prompt_prep_many(const g4_prompt_prep_entry* entries, uint32_t n_entries, void* stream);

/* ---- the f16 projections either side of the block ------------------------
 * attn.linearQKV (src/engine.ts:2045-2051) and attn.linearOut (:2096):
 * matmulQuant / matmulQuantMR4 over f16 weights. One call runs up to four
 * weight matrices that read the same input (q, k and v in one launch);
 * out[r] of each segment is bit-identical to matmul_quant.wgsl's row r.
 * n (input length) a multiple of 256 in [1024, 4096]; input and weights
 * 16-byte aligned. */
typedef struct g4_linear_seg {
    const uint16_t* weight;  /* f16 [rows][n] */
    float* out;              /* f32 [rows] */
    uint32_t rows;
} g4_linear_seg;

int g4_linear_f16(const float* input, uint32_t n, const g4_linear_seg* segs, uint32_t n_segs, void* stream);

/* attn.linearOut after a prepared decode step (src/engine.ts:2096, after the
 * attention block of :2056-2094), with the step's log-sum-exp merge folded
 * into the projection's launch. Call after g4_attn_step_run_attention, in
 * place of g4_attn_step_run_merge: for every entry i of the plan, attnOut
 * (the entry's `out`) is merged and written exactly as g4_attn_step_run_merge
 * writes it, and o_proj[i].out receives o_proj[i].weight (f16
 * [rows][num_q_heads * head_dim]) times attnOut, each row bit-identical to
 * g4_linear_f16 over that attnOut. One launch when no entry spans more than 8
 * workgroups of the attention pass and the step has one kv head of 4 or 8
 * query heads; otherwise the merge launch, then the projection launch.
 * n_segs: the plan's entry count (at most 64); num_q_heads * head_dim a
 * multiple of 256 in [1024, 4096]; weights 16-byte aligned. */
int g4_attn_step_run_out(const g4_decode_plan* plan, const g4_linear_seg* o_proj, uint32_t n_segs, void* stream);

/* The same for the engine's in-shader quantized weights (weightQuant 'q8' /
 * 'q4k', src/engine.ts:2040-2043): each row bit-identical to matmulQ8 /
 * matmulQ4K. weight: int8 [rows][n] (q8) or u32 [rows][n/8] (q4k); meta: the
 * f16 scales [rows][n/32] (q8) or scale/min table [rows][n/256][16] (q4k).
 * Same limits as g4_linear_f16; weight 16-byte aligned. */
#define G4_WEIGHT_F16 0
#define G4_WEIGHT_Q8 1
#define G4_WEIGHT_Q4K 2
typedef struct g4_linear_qseg {
    const void* weight;
    const uint16_t* meta;
    float* out;               /* f32 [rows] */
    uint32_t rows;
} g4_linear_qseg;

int g4_linear_quant(const float* input, uint32_t n, uint32_t format, const g4_linear_qseg* segs, uint32_t n_segs,
                    void* stream);

/* attn.linearQKV with the attention block's producer-side prep as its
 * epilogue, in one launch: the dispatches linearQKV, vNorm, fusedNormRope(Q),
 * fusedNormRope(K), kvCacheStore of src/engine.ts:2045-2091. segs: q
 * (num_q_heads * head_dim rows), then k and v (num_kv_heads * head_dim rows
 * each) on KV-producer layers (store_kv 1), q alone on consumer layers; weights
 * in `format` (G4_WEIGHT_F16: meta NULL; G4_WEIGHT_Q8 / G4_WEIGHT_Q4K as for
 * g4_linear_quant). Afterwards each segment's out holds what the reference
 * leaves in its q / k / v buffers: the projection (rows bit-identical to
 * matmulQuant / matmulQ8 / matmulQ4K) normalised per head in place, q and k
 * with RoPE at `position` (bit-identical to fused_per_head_norm_rope.wgsl /
 * per_head_rms_norm_no_weight.wgsl), and on producer layers row `slot` of the
 * f16 caches [rows][num_kv_heads][head_dim] holds k and v (kv_cache_store.wgsl,
 * f16 RNE). rope_inv_freq: optional device [head_dim / 2] table from
 * g4_rope_inv_freq; NULL: evaluated from theta / rope_freqs. workspace:
 * g4_linear_qkv_prep_workspace_size bytes of per-head arrival counters,
 * zeroed once after allocation (every call leaves them zero); calls sharing a
 * workspace must not overlap. head_dim 256 or 512; n as g4_linear_f16. */
typedef struct g4_qkv_prep_params {
    uint32_t num_q_heads;
    uint32_t num_kv_heads;
    uint32_t head_dim;       /* 256 or 512 */
    uint32_t position;       /* RoPE position of the token */
    uint32_t slot;           /* cache row the k and v rows go to */
    uint32_t max_seq_len;    /* cache rows (slot < max_seq_len) */
    float eps;
    float theta;
    uint32_t apply_divisor;  /* 1 on global layers: divide by rope_freqs[i] */
    uint32_t store_kv;       /* 1 on KV-producer layers */
} g4_qkv_prep_params;

int g4_linear_qkv_prep_workspace_size(uint32_t num_q_heads, uint32_t num_kv_heads, size_t* bytes);
int g4_linear_qkv_prep(const float* input, uint32_t n, uint32_t format, const g4_linear_qseg* segs, uint32_t n_segs,
                       const uint16_t* q_weight, const uint16_t* k_weight, const uint16_t* rope_freqs,
                       const float* rope_inv_freq, uint16_t* k_cache, uint16_t* v_cache, g4_qkv_prep_params p,
                       void* workspace, void* stream);

/* ---- lm head -> logit softcap -> argmax (greedy top-1) ------------------
 * src/engine.ts:2223-2255: lmHead (matmulQuant over the f16 tied embedding
 * [vocab][hidden]), logitSoftcap (when final_logit_softcapping > 0), then
 * sample.argmax (one workgroup). */

/* matmul_quant.wgsl:12; built for lmHead as {M: vocab, N: hidden} */
typedef struct g4_matmul_params {
    uint32_t M;
    uint32_t N;
} g4_matmul_params;

/* logit_softcap.wgsl:5 */
typedef struct g4_softcap_params {
    uint32_t size;
    float cap;
} g4_softcap_params;

/* SHADERS.matmulQuant — matmul_quant.wgsl:20-52, dispatched by dispatchMatmul
 * (src/engine.ts:363-377): output[m] = sum_k f16 weight[m][k] * input[k], in
 * the shader's order (invocation tid sums k = tid mod 256 in order, then the
 * 128 -> 1 tree): bit-identical to it. */
int g4_matmul_quant_f16(const float* input, const uint16_t* weight, float* output, g4_matmul_params p, void* stream);
/* shaders/matmul_q8.wgsl (matmulQ8; matmulQ8Mr, src/engine.ts:2040, has the
 * same per-row arithmetic): int8 weights [M][N], one f16 scale per
 * 32-element block [M][N/32]. N a multiple of 32. */
int g4_matmul_q8(const float* input, const int8_t* qweight, const uint16_t* qscale, float* output, g4_matmul_params p,
                 void* stream);
/* shaders/matmul_q4k.wgsl (matmulQ4K; matmulQ4KMr likewise): 4-bit weights
 * packed 8 per u32, low nibble first, over the flat [M][N] array; per row and
 * 256-element super-block 16 f16 values, the 8 sub-block scales then the 8
 * mins. N a multiple of 256. */
int g4_matmul_q4k(const float* input, const uint32_t* qweight, const uint16_t* qmeta, float* output,
                  g4_matmul_params p, void* stream);

/* SHADERS.logitSoftcap — logit_softcap.wgsl:9-16 (src/engine.ts:2230-2236). In place. */
int g4_logit_softcap(float* logits, g4_softcap_params p, void* stream);

/* SHADERS.argmax — argmax.wgsl:7-34 (src/engine.ts:2247-2250): result[0] =
 * the index the shader's one workgroup picks, ties included. */
int g4_argmax(const float* logits, uint32_t* result, uint32_t size, void* stream);

/* The three passes above fused for the whole chip (new): one streaming pass
 * over the weight computes each logit with matmul_quant.wgsl's summation
 * order and logit_softcap.wgsl's expression (cap 0 = no softcap), so logits
 * are bit-identical to the three-kernel chain; the top-1 is chosen by
 * argmax.wgsl's rule (first maximum per index residue mod 256, residues
 * compared through its 128 -> 1 tree), so result[0] equals the chain's
 * argmax, ties included. logits may be NULL (not written). hidden % 256 == 0,
 * 1024 <= hidden <= 2560; hidden and weight 16-byte aligned. The workspace (g4_lm_head_workspace_size bytes)
 * holds per-workgroup candidates; nothing in it persists between calls. */
typedef struct g4_lm_head_params {
    uint32_t vocab;   /* rows of the weight */
    uint32_t hidden;  /* columns; length of the input */
    float cap;        /* final_logit_softcapping; 0 = none */
} g4_lm_head_params;

int g4_lm_head_workspace_size(g4_lm_head_params p, size_t* bytes);
int g4_lm_head_argmax(const float* hidden, const uint16_t* weight, float* logits, uint32_t* result, void* workspace,
                      size_t workspace_bytes, g4_lm_head_params p, void* stream);
/* Measurement hook: g4_lm_head_argmax with two hipEvent_t (timing enabled)
 * recorded around the streaming kernel (the small pick kernel follows). */
int g4_lm_head_argmax_timed(const float* hidden, const uint16_t* weight, float* logits, uint32_t* result,
                            void* workspace, size_t workspace_bytes, g4_lm_head_params p, void* stream,
                            void* start_event, void* stop_event);

#ifdef __cplusplus
}
#endif
#endif /* G4ATTN_H */
