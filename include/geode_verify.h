/* geode_verify.h - libgeode_verify.so: Geode's speculative-decoding verify step on one MI355X (gfx950).
 *
 * A C ABI with no HIP or torch type in it: plain pointers, sizes, int status (0 = done, nonzero = failed, the
 * reason in gv_last_error()). It stands where the reference engine calls its accelerator backends: the NPU
 * plugin's C ABI (npu/host/npu_api.h), which the engine dlopen()s and binds into Model::Npu's function table
 * (engine/src/model.cpp:2255-2394, engine/src/model.hpp:682-797), and the Adreno backend's decode calls
 * (engine/src/gpu8.hpp:116-192) under Model::verify_n / verify_keep (engine/src/model.cpp:1483-1634).
 *
 * Threading: one host thread drives the library at a time (engine/include/geode/geode.h:6-8). Every call is
 * enqueued on the library's stream; calls that return host data wait for it.
 *
 * q4 matrices come in the pack's row layout (engine/src/kernels.hpp:22-26; npu/host/npu_api.h:31-34): per row
 * cols/2 code bytes (value 2j in the low nibble of byte j; levels 1 3 .. 15 for codes 0..7, -1 .. -15 for 8..15)
 * then cols/16 E4M3 scale bytes; value = level x E4M3(scale) x global.
 */
#ifndef GEODE_VERIFY_H
#define GEODE_VERIFY_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ run time
 * (no reference counterpart: the device, its memory and stream; the reference's OpenCL/FastRPC equivalents are
 * engine/src/opencl.cpp and npu/host/npu_api.h's gnpu_open) */
const char *gv_last_error(void);
/* Makes the device current and creates the library's stream (idempotent). 0 when done. */
int gv_init(int device);
int gv_device_count(void);
void *gv_malloc(size_t bytes); /* device memory, NULL on failure */
int gv_free(void *p);
int gv_memcpy_h2d(void *dst, const void *src, size_t bytes);
int gv_memcpy_d2h(void *dst, const void *src, size_t bytes);
int gv_memcpy_d2d(void *dst, const void *src, size_t bytes);
int gv_memset(void *dst, int value, size_t bytes);
int gv_synchronize(void);
/* milliseconds between two points of the library's stream: gv_event_record returns an id */
int gv_event_record(void);
float gv_event_elapsed_ms(int start, int stop);

/* ------------------------------------------------------------------ the q4 format on the device */
typedef struct gv_q4 {
    const uint8_t *codes;  /* device: affine nibbles in the step-major tile layout */
    const uint8_t *scales; /* device: E4M3 bytes grouped per lane */
    int64_t rows, cols;
    int32_t lanes, steps;
    float global;
} gv_q4;

/* Device bytes a rows x cols q4 matrix takes (the same 4.5 bits a weight as the pack). */
size_t gv_q4_device_bytes(int64_t rows, int64_t cols);
/* The pack layout at pack_dev (device) into the device layout at dst (gv_q4_device_bytes of device memory):
 * a lossless permutation of the same bytes. Replaces the reference's load-time re-layouts to_quad / to_tile8
 * (engine/src/kernels.cpp:946-991). */
int gv_q4_from_pack(const uint8_t *pack_dev, int64_t rows, int64_t cols, float global, void *dst, gv_q4 *out);
/* out[rows][cols] fp32 (device) = the dequantized weights, bit for bit dequant_row's (engine/src/kernels.cpp:1214) */
int gv_q4_dequant(const gv_q4 *w, float *out);
/* The RTN packer on the device: w[rows][cols] fp32 -> pack layout, global = max|w| x 1.25 / (15 x 448); bit for
 * bit q4_block / e4m3_byte (engine/src/yue2_q4.cpp:72-114, :332-358). global_out: device float. */
int gv_q4_pack(const float *w_dev, int64_t rows, int64_t cols, uint8_t *pack_out_dev, float *global_out_dev);

/* ------------------------------------------------------------------ activations and products (device pointers) */
/* Bytes of one token's int8 activations for cols inputs. */
size_t gv_act_bytes(int64_t cols);
/* act[t] = quantize_activation(x[t]) (engine/src/kernels.cpp:1254-1295) for M tokens (x rows ldx floats apart);
 * with norm_w, x is first RMSNorm'ed with weight (1 + w) (engine/src/kernels.cpp:1520-1529) and the normalized
 * rows go to h_out when it is not NULL. */
int gv_quantize(const float *x, int64_t ldx, int M, int cols, const float *norm_w, float eps, uint8_t *act,
                float *h_out);
/* y[t][r] (= or +=) W act[t] for M <= 32 tokens: the int8 path of matvec_rows_q_multi (engine/src/kernels.cpp:
 * 1304-1420; the integer block sums bit for bit, the fp32 sum in another order). */
int gv_gemv_q4(const gv_q4 *w, const uint8_t *act, int M, float *y, int64_t ldy, int accumulate);
/* C1: y[t] = down(silu(gate x[t]) * up x[t]) for M fp16 rows x (device), the dense MLP of Model::moe
 * (engine/src/model.cpp:4126-4146) on the int8 path. ws: device scratch of gv_ffn_workspace_bytes. */
size_t gv_ffn_workspace_bytes(int64_t hidden, int64_t ff, int M);
int gv_ffn_swiglu(const gv_q4 *gate, const gv_q4 *up, const gv_q4 *down, int M, const uint16_t *x_f16, float *y,
                  void *ws);
/* gv_ffn_swiglu without a workspace argument and without allocating: no reference counterpart. For callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The workspace is the library's own 4 MiB device array, one per GPU (its address looked up by gv_init), so
 * gv_ffn_workspace_bytes(hidden, ff, M) must be at most 4 MiB (C1's 2048 -> 6144 -> 2048 takes up to 32 rows) or the
 * call fails with a message. Calls on one GPU share that array: calls that overlap on one GPU (other threads,
 * other streams) race. Same results as gv_ffn_swiglu, bit for bit. */
int gv_ffn_swiglu_noalloc(const gv_q4 *gate, const gv_q4 *up, const gv_q4 *down, int M, const uint16_t *x_f16,
                          float *y);

/* ------------------------------------------------------------------ the NPU plugin's calls, on this GPU
 * The same names' meaning as npu/host/npu_api.h (gnpu_open / gnpu_adopt_q4 / gnpu_gemm / gnpu_mlp): a handle,
 * matrices adopted in the pack layout (copied to the device), products on host rows. */
typedef struct gv_ctx gv_ctx;
gv_ctx *gv_open(int device, char *err, int err_len);                                    /* npu_api.h:16 */
void gv_close(gv_ctx *g);                                                                /* npu_api.h:30 */
int gv_adopt_q4(gv_ctx *g, const uint8_t *data, int64_t rows, int64_t cols, size_t row_bytes, float global); /* :34 */
int gv_gemm(gv_ctx *g, int id, int n, const float *const *xs, float *const *ys);       /* npu_api.h:44 */
int gv_mlp(gv_ctx *g, int gate, int up, int n_down, const int *downs, int act, int n, const float *const *xs,
           float *const *ys);                                                            /* npu_api.h:66 */

/* ------------------------------------------------------------------ the verify step
 * A whole model resident on the device and the reference's verify contract (engine/src/model.hpp:189-205):
 * gv_verify = Model::verify_n (engine/src/model.cpp:1483-1592), gv_verify_keep = Model::verify_keep
 * (engine/src/model.cpp:1594-1634). Per layer: RMSNorm, gated attention with q/k RMSNorm and partial RoPE over an
 * fp16 KV cache (engine/src/model.cpp:3690-4019), RMSNorm, the MoE block (router, top-k, experts, sigmoid-gated
 * shared expert, combine; engine/src/model.cpp:4123-4587); then the final norm and lm_head. Products on the
 * reference's int8 path (quantize_activation + matvec_rows_q). */
typedef struct gv_model_config {
    int32_t hidden, vocab, n_layers, n_experts, top_k, moe_ff, shared_ff;
    int32_t n_heads, n_kv_heads, head_dim, rope_dim;
    float rope_theta, eps;
    int32_t max_ctx;  /* KV positions the cache holds */
    int32_t max_rows; /* rows a verify takes at most (<= 32) */
    int32_t kv_int8;  /* 1: the KV cache in int8 with a float scale a (position, KV head), ModelOptions::kv_int8
                         (engine/src/model.cpp:360-363, :3756-3792); 0: fp16 (attend<_Float16>) */
    /* Gated DeltaNet layers (ModelConfig::gdn_*, engine/src/pack.hpp:36-38; gdn_v_heads = 0: none): layer l is one
     * iff gdn_layers[l] != 0 (ModelConfig::attention[l] false, pack.hpp:43: layer_types "linear_attention"). Key heads nk of dk, value heads nv of dv
     * (nv a multiple of nk; dk in {32, 64, 128, 256}; dv a multiple of 16 with dv / 8 a power of two, at most 256;
     * nv x dv a multiple of 128), causal conv of conv_kernel taps (2 .. 8). */
    int32_t gdn_k_heads, gdn_v_heads, gdn_k_dim, gdn_v_dim, conv_kernel;
    uint8_t gdn_layers[256];
    /* 1: an MTP draft layer (ModelConfig::mtp_layers, engine/src/model.cpp:175-191): a full-attention layer at index
     * n_layers (its tensors adopted with the per-layer kinds at that index, its KV after the main layers') behind
     * mtp.fc, with its own norms (GV_MTP_*); hidden at most 8192 */
    int32_t mtp;
    /* 1: the exact path (ModelOptions::exact, GEODE_EXACT=1; engine/src/model.cpp:3337-3361): every product takes
     * the fp32 activations instead of the int8 path's quantized ones (kv_int8 must be 0; the cache stays fp16, where
     * the reference's exact path keeps fp32) */
    int32_t exact;
} gv_model_config;

/* tensor kinds for gv_model_adopt (numbered as the CPU oracle's) */
enum {
    GV_EMBED = 0,         /* q4 [vocab x hidden], globals[0] */
    GV_LM_HEAD = 1,       /* q4 [vocab x hidden], globals[0] */
    GV_FINAL_NORM = 2,    /* f32 [hidden] */
    GV_IN_NORM = 3,       /* f32 [hidden] */
    GV_POST_NORM = 4,     /* f32 [hidden] */
    GV_QKV = 5,           /* q4 rows of q [n_heads x (query hd | gate hd)], then k, then v; globals[3] */
    GV_O = 8,             /* q4 [hidden x n_heads*hd], globals[0] */
    GV_Q_NORM = 9,        /* f32 [hd] */
    GV_K_NORM = 10,       /* f32 [hd] */
    GV_ROUTER = 11,       /* bf16 [n_experts x hidden] */
    GV_SHARED_GATE = 12,  /* bf16 [hidden] */
    GV_EXPERT = 13,       /* the pack's expert block: q4 gate_up [2ff x hidden] then down [hidden x ff];
                             globals[0] gate_up, globals[1] down (engine/src/pack.cpp:329-333) */
    GV_SHARED_EXPERT = 14,/* q4 gate [ff x hidden], up [ff x hidden], down [hidden x ff]; globals[3] */
    GV_KV = 17,           /* fp16 [2][n_positions][n_kv_heads*hd]: K then V of positions 0.. (an int8 cache
                             quantizes each (position, KV head) row as quant_kv_row does, model.cpp:3766-3774) */
    GV_KV_I8 = 18,        /* int8 cache only: int8 [2][n_positions][n_kv_heads*hd] then float [2][n_positions]
                             [n_kv_heads] scales, the reference's int8 chunk layout (model.cpp:3756-3763) */
    /* a Gated DeltaNet layer's tensors (Model::bind_layer, engine/src/model.cpp:129-138; kd = nk dk, vd = nv dv) */
    GV_GDN_QKV = 20,      /* q4 in_proj_qkv [2 kd + vd x hidden], globals[0] */
    GV_GDN_Z = 21,        /* q4 in_proj_z [vd x hidden], globals[0] */
    GV_GDN_OUT = 22,      /* q4 out_proj [hidden x vd], globals[0] */
    GV_GDN_A = 23,        /* bf16 in_proj_a [nv x hidden] */
    GV_GDN_B = 24,        /* bf16 in_proj_b [nv x hidden] */
    GV_GDN_ALOG = 25,     /* f32 A_log [nv] */
    GV_GDN_DTB = 26,      /* f32 dt_bias [nv] */
    GV_GDN_CONV = 27,     /* f32 conv1d [2 kd + vd][conv_kernel] */
    GV_GDN_NORM = 28,     /* f32 norm [dv] (the gated RMSNorm's weight as it is: no 1 + w) */
    GV_GDN_CONV_ST = 29,  /* f32 the conv's state [2 kd + vd][conv_kernel - 1], the last inputs oldest first */
    GV_GDN_S = 30,        /* f32 the recurrent state [nv][dk][dv] */
    /* the MTP layer's own tensors (engine/src/model.cpp:178-190; layer ignored) */
    GV_MTP_FC = 31,       /* q4 mtp.fc.weight [hidden x 2 hidden], globals[0] */
    GV_MTP_NORM = 32,     /* f32 mtp.norm.weight [hidden] */
    GV_MTP_PRE_E = 33,    /* f32 mtp.pre_fc_norm_embedding.weight [hidden] */
    GV_MTP_PRE_H = 34     /* f32 mtp.pre_fc_norm_hidden.weight [hidden] */
};

typedef struct gv_model gv_model;
gv_model *gv_model_create(const gv_model_config *cfg, char *err, int err_len);
void gv_model_free(gv_model *m);
/* A tensor from host memory (bytes: its size, checked). */
int gv_model_adopt(gv_model *m, int kind, int layer, int expert, const void *data, int64_t bytes,
                   const float *globals);
/* Every tensor seeded on the device: N(0, sigma) weights through the RTN packer, the router N(0, router_sigma) in
 * bf16, norms N(0, 0.02), the KV cache's first ctx positions N(0, 1) in fp16; the position becomes ctx. */
int gv_model_randomize(gv_model *m, uint64_t seed, float sigma, float router_sigma, int ctx);
int gv_model_set_position(gv_model *m, int pos);
int gv_model_position(const gv_model *m);
/* verify_n: n rows at KV slots pos.. . parents NULL: a chain (row i sees rows 0..i); else a draft tree in BFS
 * order, parents[0] = -1, parents[i] < i (row i sees the context, its ancestors and itself; rotary position
 * pos + depth). logits (host, [n][vocab]) may be NULL: they stay on the device (gv_model_logits). The position
 * advances by n. */
int gv_verify(gv_model *m, const int32_t *tokens, int n, const int32_t *parents, float *logits);
/* verify_keep: the first kept rows stay (a tree: path[0..kept) of row indices, path[0] = 0, ascending; their
 * keys and values move to slots pos..pos+kept-1); the position becomes the verify's start plus kept. */
int gv_verify_keep(gv_model *m, int kept, const int32_t *path);
const float *gv_model_logits(const gv_model *m); /* device [max_rows][vocab] of the last verify */
/* the last verify's routed experts, host [n_layers][n][top_k] */
int gv_model_route_ids(const gv_model *m, int32_t *out);

/* kernel classes of a verify step, for gv_model_time_kernel */
enum {
    GV_K_EMBED = 0, GV_K_QUANT = 1, GV_K_QKV = 2, GV_K_ROPE = 3, GV_K_ATTN = 4, GV_K_MERGE = 5, GV_K_O = 6,
    GV_K_ROUTER = 7, GV_K_ROUTE = 8, GV_K_MOE_UP = 9, GV_K_SWIGLU = 10, GV_K_MOE_DOWN = 11, GV_K_COMBINE = 12,
    GV_K_LM_HEAD = 13,
    /* a Gated DeltaNet layer's own (its projections are GV_K_QKV's and GV_K_O's launches): the bf16 a / b rows, the
     * causal conv, the delta rule, the gated RMSNorm with the output projection's operands */
    GV_K_GDN_AB = 14, GV_K_GDN_CONV = 15, GV_K_GDN_CORE = 16, GV_K_GDN_NORM = 17, GV_K_COUNT = 18
};
/* From now on, every launch of kernel class cls is bracketed by events on the library's stream (cls < 0: off);
 * gv_model_kernel_time waits and returns their summed milliseconds and launches since (no reference counterpart:
 * the reference's per-kernel timing is GEODE_GPU8_PROF, engine/src/gpu8.cpp:195). */
/* The verify step runs as one HIP graph per row count (captured on the second step of that count and replayed
 * after; every step parameter lives in device memory). on = 0: plain launches (no reference counterpart). */
int gv_model_set_graphs(gv_model *m, int on);
/* on (the default): dependent phases of a layer chained within one launch where the shapes fit (the output
 * projection, the post-attention RMSNorm + router and the route: workgroups of each phase wait for the previous
 * phase's counter instead of a kernel boundary), and the experts' up launch routing the rows itself (no route
 * launch or hand-off between the router and the experts); 2: the same but with the route as the last phase of the
 * output projection's launch (a measurement aid); 0: one launch a phase. The same results bit for bit (no reference
 * counterpart). */
int gv_model_set_fused(gv_model *m, int on);
/* A measurement aid with no reference counterpart: with on = 1, thread 0 of every workgroup of the traced kernels
 * stamps its clock (s_memrealtime, 100 MHz) at a few points of its work; each launch overwrites its kernel class's
 * stamps. gv_model_trace_read copies them, [GV_K_COUNT][8192 workgroups][8 slots] (0: none), and returns the count
 * copied (negative on error). */
int gv_model_trace(gv_model *m, int on);
int64_t gv_model_trace_read(gv_model *m, uint64_t *out, int64_t n);
int gv_model_time_kernel(gv_model *m, int cls);
int gv_model_kernel_time(gv_model *m, float *total_ms, int *launches);
/* Launch kernel class cls reps times back to back on the last verify's rows, launch i on the i-th layer from `layer`
 * on (cycled) that has the class (ignored for GV_K_EMBED / GV_K_LM_HEAD; a GV_K_GDN_* class: the Gated DeltaNet
 * layers; GV_K_ROPE / _ATTN / _MERGE: the attention layers), so that consecutive launches read different weights, and return
 * the mean milliseconds a launch; a measurement aid with no reference counterpart.
 * The kernels run on the state the last verify left; classes that accumulate (GV_K_O, GV_K_COMBINE) change it, so
 * verify again before trusting the model's state. */
int gv_model_replay(gv_model *m, int cls, int layer, int reps, float *ms_per_launch);

/* C3 / C5: one MoE block of layer `layer` (Model::moe, engine/src/model.cpp:4123-4587; route_topk :4021-4065,
 * combine :4554-4585; the prefill's expert-grouped products :4484-4543) on M rows h [M][hidden] fp32 (host), the
 * routed logits given [M][n_experts] or NULL (the layer's bf16 router; only for M <= max_rows); the shared
 * expert's gate from the layer's shared_gate row. M <= max_rows runs the verify step's kernels, more rows (up to
 * 16384) the prefill path: the picks grouped by expert in runs of at most 32 rows. out [M][hidden] = the block's
 * output without the residual; ids / weights [M][top_k] (may be NULL). The int8 path. Leaves no verify to keep. */
int gv_model_moe(gv_model *m, int layer, const float *h, int M, const float *router_logits, float *out,
                 int32_t *ids, float *weights);
/* One layer of the verify step (the loop body of forward_batch, engine/src/model.cpp:5324-5366) on a given residual
 * stream: x_in [n][hidden] (host) at the model's position (a chain, or the tree of parents as gv_verify takes it);
 * x_mid = after the attention's residual add, x_out = after the MoE's, ids [n][top_k] the routed experts (each may be
 * NULL). The rows' keys and values go to the cache at slots pos.. ; the position does not move and there is nothing
 * to keep. A checking aid: the layers of a step compared one at a time, each fed the same input. */
int gv_model_layer(gv_model *m, int layer, const float *x_in, int n, const int32_t *parents, float *x_mid,
                   float *x_out, int32_t *ids);
/* A Gated DeltaNet layer's states as the last verify or keep left them (a chain: after its last row; after a keep:
 * after the last kept row, model.cpp:1617-1633): conv [2 kd + vd][conv_kernel - 1] and S [nv][dk][dv], host (either
 * may be NULL). gv_model_layer reads the states and leaves them as they were. */
int gv_model_gdn_state(const gv_model *m, int layer, float *conv, float *S);

/* ---- the MTP draft layer on the GPU (a model made with mtp = 1) ----
 * Model::draft (engine/src/model.cpp:1295-1432): the MTP pass (Model::forward_mtp, :4965-5039) over n rows at MTP
 * positions pos..pos+n-1, row t the pair (hidden row t, toks[t]: the token after it), the layer's keys and values to
 * its own cache at those positions; *draft = the first maximum of the last row's logits (through the draft
 * vocabulary when one is set), *prob = its softmax probability, 1 / sum exp(double(l - max)) (softmax_at, :1286-1292).
 * hidden: host [n][hidden], or NULL for the last verify's rows after the final norm (rows 0..n-1; after a keep with a
 * path, the path's rows). 1 <= n <= max_rows. */
int gv_model_draft(gv_model *m, const int32_t *toks, int n, int pos, const float *hidden, int32_t *draft, float *prob);
/* Model::draft_next (model.cpp:1434-1479): one MTP row at position pos from the last MTP pass's output after mtp.norm
 * (its last row) and tok (the draft it made) */
int gv_model_draft_next(gv_model *m, int32_t tok, int pos, int32_t *draft, float *prob);
/* The generate loop's drafting (engine/src/geode.cpp:301-317) in one call: gv_model_draft, then chained drafts
 * while the last one's probability is at least pmin, at most kmax - 1 drafts in all and while the verify batch (the
 * token and the drafts) still fits the context after the model's position. drafts / probs [kmax - 1]. */
int gv_model_draft_chain(gv_model *m, const int32_t *toks, int n, int pos, const float *hidden, int kmax, float pmin,
                         int32_t *drafts, float *probs, int *count);
/* forward_mtp without logits (a prompt's pass, model.cpp:4985: only the layer's keys and values); n rows, in chunks
 * of max_rows; hidden NULL only for n within the last verify's rows */
int gv_model_mtp_fill(gv_model *m, const int32_t *toks, int n, int pos, const float *hidden);
/* The draft head (model.cpp:803-827, draft_vocab.bin): lm_head's rows of ids[0..n), a draft is one of them; n = 0:
 * the whole vocabulary again */
int gv_model_set_draft_vocab(gv_model *m, const int32_t *ids, int n);
/* The last verify's rows after the final norm (the MTP layer's input), host [rows][hidden]; returns the rows copied */
int gv_model_hidden(const gv_model *m, float *out, int max_rows);
/* The last MTP pass's logits (its last row, over the draft head's rows), host; returns their count */
int gv_model_draft_logits(const gv_model *m, float *out);
/* Re-run the last gv_model_moe call's block on its device-staged rows and logits reps times back to back, run i on
 * layer (layer + i) mod n_layers (so that a model of several layers rotates through distinct expert weights), and
 * return the mean milliseconds a block (device work only); a measurement aid with no reference counterpart. */
int gv_model_moe_replay(gv_model *m, int reps, float *ms_per_block);

/* ------------------------------------------------------------------ a geode-pack (F3)
 * Pack::open (engine/src/pack.cpp:39-308): the manifest geode.json (format "geode-pack" v1, its files and their
 * sizes, the config, the tensor table, the expert table) checked as the reference checks it, nothing read yet; the
 * tensors are read from their files by gv_model_load_pack. Host calls (no device work) except that one. */
typedef struct gv_pack gv_pack;
gv_pack *gv_pack_open(const char *dir, char *err, int err_len);
void gv_pack_close(gv_pack *p);
/* FNV-1a 64 of geode.json's bytes (Model::fingerprint's pack print, engine/src/state.cpp:227-238): the pack_print a
 * state file of this pack carries (gv_state_info) */
uint64_t gv_pack_print(const gv_pack *p);
/* The GPU model's config from the pack's (and the caller's context, rows and KV format): the layers that are not
 * "full_attention" Gated DeltaNet layers with the pack's linear_* shape. Fails for what the GPU model does not run:
 * another architecture than qwen35moe, a shared expert of another width (gv_model_create refuses the shapes it does
 * not take). */
int gv_pack_model_config(const gv_pack *p, int max_ctx, int max_rows, int kv_int8, gv_model_config *out);
typedef struct gv_pack_tensor_info {
    int32_t type;      /* the reference's DType: 0 f32, 1 bf16, 2 q2, 3 q3, 4 nvfp4, 5 q8, 6 q4, 8 q4i (kernels.hpp:16) */
    int64_t rows, cols;/* shape[0] and the product of the rest (one dimension: 1 x n) */
    int32_t file;      /* index among the pack's files present */
    uint64_t offset, bytes;
    float global;
} gv_pack_tensor_info;
int gv_pack_tensor(const gv_pack *p, const char *name, gv_pack_tensor_info *out);
/* Pack::expert (pack.cpp:317-328): where expert e of a layer (n_layers: the MTP layer's) is and its format */
int gv_pack_expert(const gv_pack *p, int layer, int expert, int *file, uint64_t *offset, int *type);
/* 1 when the pack's q4 experts are in the tile8 layout (geode.json formats.q4.layout) */
int gv_pack_tile8(const gv_pack *p);
/* tile8 (to_tile8, engine/src/kernels.cpp:971-991) back to the pack's rows, host memory, rows % 32, cols % 64 */
int gv_q4_untile8(int64_t rows, int64_t cols, const uint8_t *src, uint8_t *dst);
/* Every tensor of the pack adopted by a model created with gv_pack_model_config's config (Model::bind,
 * engine/src/model.cpp:95-202: the norms, q | k | v, o, q / k norms, the router and shared gate, the shared expert,
 * the routed experts with their scales, embed_tokens, norm, lm_head); the position becomes 0. */
int gv_model_load_pack(gv_model *m, const gv_pack *p);

/* ------------------------------------------------------------------ a conversation's state in a file (F4)
 * The reference's state file (engine/src/state.cpp:1-20): a 4096-byte header with an FNV-1a checksum, the fixed part
 * (gen at both ends), the KV cache in blocks of 256 positions [K, V][layer][256][n_kv_heads * hd] (fp16 or int8, then
 * the int8 cache's float scales [K, V][layer][256][n_kv_heads]). A state saved by the reference's CPU or GPU path
 * loads here and the other way round, for a model of the same pack and KV format; this model is attention-only
 * (no Gated DeltaNet states) and takes no images. */
typedef struct gv_state_info {
    uint64_t pack_print; /* FNV-1a 64 of the pack's geode.json bytes (Model::fingerprint, engine/src/state.cpp:227-245;
                            0: none, taken as 1); a load refuses a file of another pack */
    uint64_t conv_id;    /* the conversation (save: written, an append goes only to a file of the same one; load: read) */
    int32_t extra;       /* the caller's value kept with the state (geode.cpp: the token passed on, not computed yet) */
    int32_t rope_delta;
    int32_t has_mtp;     /* the fingerprint's flags (state.cpp:240-242): the model that exchanges the state has an MTP */
    int32_t has_vision;  /* layer / a vision encoder */
    float *hidden;       /* host [hidden] or NULL: the last hidden state an MTP layer drafts from (save: written when
                            has_mtp and the position > 0; load: filled when the file holds one) */
    int32_t has_hidden;  /* load: 1 when the file held a hidden state and `hidden` received it */
} gv_state_info;
/* error classes of the two calls (geode_state_save / geode_state_load's GEODE_E_*, engine/src/geode.cpp:490-518) */
enum { GV_STATE_E_IO = -1, GV_STATE_E_FORMAT = -2, GV_STATE_E_ARG = -3, GV_STATE_E_MEMORY = -4 };
/* Model::save_state (engine/src/state.cpp:251-371): the conversation (the model's position, its attention layers' KV
 * rows and its Gated DeltaNet layers' states as the last verify or keep left them) to path.
 * append: path holds an earlier state of the same conversation (fingerprint and conv_id): the fixed part and the
 * blocks from the one holding its last position are written in place, the header last; anything else is written
 * whole to path.tmp and renamed over path. Between verify steps only. */
int gv_model_save_state(gv_model *m, const char *path, int append, const gv_state_info *info);
/* Model::load_state (engine/src/state.cpp:373-463): the saved conversation replaces the model's (the position becomes
 * the saved one, nothing to keep); conv_id, extra, rope_delta and has_hidden come back in *info, which also names
 * the pack and flags to check the fingerprint against. On failure the position is 0 and the Gated DeltaNet states
 * zero (Model::reset). */
int gv_model_load_state(gv_model *m, const char *path, gv_state_info *info);

/* ------------------------------------------------------------------ sampling and acceptance (C2)
 * Rows of logits in device memory (ld floats apart, e.g. gv_model_logits'), uniforms and results on the host.
 * The double sums of the sampler run as parallel scans and expf is the device's: a sampled index can differ from
 * the reference's only when a uniform or top_p falls within ~1e-15 (relative) of a boundary. */

/* Sampler::sample (engine/src/sampler.cpp:16-50) of each row with its injected uniform u[r] in [0, 1) standing for
 * uniform_real_distribution<double>(0, kept): T <= 0 the first argmax; else the top_k candidates (else the top
 * `cap`, 1024 in the reference; top_k and cap at most 16384; both 0: the whole vocabulary, any top_p), ties to the lower
 * index. rows <= 64, V <= 262,144. */
int gv_sample_rows(const float *logits, int64_t ld, int rows, int V, float temperature, float top_p, int top_k,
                   int cap, const double *u, int32_t *out);
/* Sample-and-match over a verified chain (engine/src/geode.cpp:318-374): batch = [tok, d1..d_{n-1}]; row i sampled
 * with u[i]; a draft stands while row i samples exactly it. out: the stood drafts then the first sampled token that
 * is no draft; returns their count (or -1), *kept = the rows that stay (verify_keep's argument). n <= 32. */
int gv_accept_match(const float *logits, int64_t ld, int V, const int32_t *batch, int n, float temperature,
                    float top_p, int top_k, int cap, const double *u, int32_t *out, int *kept);
/* gv_accept_match with the generate loop's presence penalty and stop tokens (engine/src/geode.cpp:236-255, :331-350):
 * seen[0..n_seen) are the answer's tokens so far (distinct); before row i is sampled, presence_penalty is subtracted
 * (in place, as the reference's loop does) from its logits at every seen token and at each draft batch[1..i] new to
 * the answer (the tokens rows 0..i-1 sampled when their drafts stood); a draft stands only if the row before samples
 * exactly it and it is none of stop[0..n_stop). The caller adds the emitted tokens to its seen list. */
int gv_accept_match_ex(float *logits, int64_t ld, int V, const int32_t *batch, int n, float temperature, float top_p,
                       int top_k, int cap, const double *u, const int32_t *seen, int n_seen, float presence_penalty,
                       const int32_t *stop, int n_stop, int32_t *out, int *kept);
/* The textbook rule (Leviathan et al. 2023, Alg. 1; no reference counterpart: the reference accepts by
 * sample-and-match). p_i, q_i = the full-vocabulary top-p nucleus of target row i / draft row i at temperature T.
 * Draft i: greedy: argmax q_i, accepted iff argmax p_i equals it; else d_i ~ q_i by u_draft[i], accepted iff
 * u_acc[i] q_i(d_i) < p_i(d_i). At the first rejection a token from max(0, p_i - q_i) by inverse CDF in index order
 * (u_res); when all k stand, a bonus token from p_k (u_res). target [k+1][ld], draft [k][ld]; k <= 31. out: the
 * accepted drafts then the extra token; returns their count (or -1). */
int gv_accept_textbook(const float *target, const float *draft, int64_t ld, int V, int k, float temperature,
                       float top_p, int greedy, const float *u_draft, const float *u_acc, float u_res, int32_t *out);
/* How many sampling calls of the acceptance rules (gv_accept_textbook; gv_accept_match(_ex) at T > 0) the candidate
 * path decided (each row's nucleus found among the elements above one logit: a top_p < 1 prefix of the full
 * vocabulary, or the top_k / cap candidates) and how many ran the full walks, since the library loaded. No reference
 * counterpart: for tests and measurement, to tell which path served a call. */
int gv_sampler_paths(int64_t *candidate, int64_t *walks);

#ifdef __cplusplus
}
#endif

#endif /* GEODE_VERIFY_H */
