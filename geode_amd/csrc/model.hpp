// model.hpp - the verify step's device state: weights in the kernels' layout, the fp16 KV cache, per-step
// parameters and scratch. The C ABI (gv_model_*, gv_verify*) is in model.hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/geode_verify.h"
#include "common.hpp"
#include "kernels.hpp"

namespace gv {

// Per verify: the rows' tokens, their KV slots (pos + i) and rotary positions (pos + depth), and which earlier rows
// each row sees (bit j of vis[i]: row j is row i or one of its ancestors; a chain sees every earlier row).
struct StepParams {
    int pos;
    int M;
    int tokens[kMaxRows];
    int depth[kMaxRows];
    uint32_t vis[kMaxRows];
    int gdn_base;   // the Gated DeltaNet layers' slot holding the states the rows start from
    int gdn_wset;   // the first slot of the set the rows' states go to (the set without gdn_base)
    int hrow[kMaxRows];   // an MTP pass: row t's hidden row in Model::hbuf
};

// Routing of one layer, written by the route kernel: slots are runs of at most kSlotRows picks (token, rank) of one
// expert, the distinct experts picked ascending (the shared expert last, index E), an expert with more picks taking
// consecutive slots; picks ordered by (expert, token, rank).
constexpr int kSlotRows = 8;
constexpr int kRouteSlots = kMaxRows * 16 + 1;   // >= E + 1 + picks / kSlotRows for every shape the model takes
struct RouteState {
    int n_slots;
    int n_picks;
    int slot_expert[kRouteSlots];
    int slot_start[kRouteSlots];
    int slot_count[kRouteSlots];
    int slot_token[kRouteSlots * kSlotRows];   // [slot][j]: the row of the slot's pick j (past the count: the first's)
    int slot_dst[kRouteSlots * kSlotRows];     // [slot][j]: t (K + 1) + k of the slot's pick j (its output row)
    int pick_token[kMaxRows * 17];
    int pick_of[kMaxRows * 17];   // [t][k] for k < K the routed pick, [t][K] the shared expert's
    float weight[kMaxRows * 16];  // [t][k]
    float gate[kMaxRows];         // sigmoid of the shared expert's gate
};

// Expert slots in device memory: slot u is expert[u]'s run of count[u] picks from start[u]; pick p's row is
// pick_token[p]. The decode step's come from its RouteState, the prefill's from its own buffers.
struct Slots {
    const int *n_slots, *expert, *start, *count, *pick_token, *n_picks;
    const int *token;   // [slot][kSlotRows] the rows of a slot's picks (the decode step's; null for the prefill's)
    const int *dst;     // [slot][kSlotRows] their output rows t (K + 1) + k (the decode step's; null for the prefill's)
};
inline Slots route_slots(const RouteState *rs) {   // member addresses of a device struct (no host access)
    return Slots{&rs->n_slots, rs->slot_expert, rs->slot_start, rs->slot_count, rs->pick_token, &rs->n_picks,
                 rs->slot_token, rs->slot_dst};
}
// What the combine reads: the shared gate [M], the routed weights [M][K], the output row of each pick of each row
// [M][K + 1] (null: row t (K + 1) + k, the decode MoE kernels' layout)
struct MixView {
    const float *gate, *weight;
    const int *pick_of;
};
inline MixView route_mix(const RouteState *rs, bool direct) {
    return MixView{rs->gate, rs->weight, direct ? nullptr : rs->pick_of};
}

struct LayerW {
    Q4 qkv;   // [nh*2*hd (q | gate per head) + nkv*hd (k) + nkv*hd (v)] x H, three globals
    float g_q = 1, g_k = 1, g_v = 1;
    Q4 o;     // H x nh*hd
    float *in_norm = nullptr, *post_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
    uint16_t *router = nullptr;   // bf16 [E + 1][H]: the router's rows, then the shared expert's gate
    uint8_t *gu_codes = nullptr, *gu_scales = nullptr;   // [E + 1] experts' gate_up (the shared one last)
    uint8_t *dn_codes = nullptr, *dn_scales = nullptr;   // [E + 1] experts' down
    float *expert_globals = nullptr;                     // [E + 1][3]: gate half, up half, down
    _Float16 *kv = nullptr;   // K [nkv][slots][hd], then V [nkv][slots / 64][hd][64] (model.hip: k_index, v_index)
    int8_t *kv8 = nullptr;    // the int8 cache: the same layout in int8,
    float *kvs = nullptr;     // then the scales: K [nkv][slots], V [nkv][slots]
    // a Gated DeltaNet layer (gdn.hip): qkv holds in_proj_qkv then in_proj_z (globals g_q, g_k), o out_proj [H x vd]
    bool gdn = false;
    uint16_t *gdn_ab = nullptr;   // bf16 [2 nv][H]: in_proj_a then in_proj_b
    float *A_log = nullptr, *dt_bias = nullptr, *conv_w = nullptr, *gnorm = nullptr;   // [nv], [nv], [conv_dim][K], [dv]
    float *s_slots = nullptr;     // [2 max_rows] recurrent states in the core kernel's layout (gdn.hip: s_index)
    float *c_slots = nullptr;     // [2 max_rows][K - 1][conv_dim] conv states
};

// The prefill MoE's buffers (C5: many rows), allocated for `cap` rows on first use
struct Prefill {
    int cap = 0, M = 0, layer = 0;   // M, layer: the last gv_model_moe call's (for the replay)
    bool given = false;
    float *h = nullptr, *logits = nullptr, *gate = nullptr, *w = nullptr, *gu = nullptr, *y = nullptr, *out = nullptr;
    int *ids = nullptr, *cnt = nullptr, *start = nullptr, *n_slots = nullptr, *n_picks = nullptr;
    int *slot_expert = nullptr, *slot_start = nullptr, *slot_count = nullptr, *pick_token = nullptr, *pick_of = nullptr;
    _Float16 *act = nullptr, *act_m = nullptr;
    int max_slots = 0, max_picks = 0;
    std::vector<void *> allocs;
};

struct Model {
    gv_model_config c{};
    int E1 = 0;   // experts + the shared one
    size_t gu_code_stride = 0, gu_scale_stride = 0, dn_code_stride = 0, dn_scale_stride = 0;
    Q4 embed, lm_head;
    float *final_norm = nullptr;
    std::vector<LayerW> layers;
    std::vector<void *> allocs;
    float *rope_cos = nullptr, *rope_sin = nullptr;   // [max_ctx + kMaxRows][rope_dim / 2], the host's cosf/sinf
    int kv_blocks = 0;                                // attention blocks of kAttnBlock positions
    // scratch
    StepParams *sp = nullptr;
    RouteState *route = nullptr;   // [n_layers]
    float *x = nullptr, *qkv_out = nullptr, *rlogits = nullptr;
    _Float16 *q16 = nullptr;   // [max_rows][nh][hd]: the rotated queries
    float *parts = nullptr, *gu_out = nullptr, *y = nullptr, *logits = nullptr;
    _Float16 *act_h = nullptr, *act_core = nullptr, *act_m = nullptr;   // the products' operands (act16)
    uint8_t *arena = nullptr;   // x, qkv_out, rlogits, parts, y, logits, act_h, act_core, act_m: one allocation
    size_t arena_bytes = 0;
    int32_t *route_ids = nullptr;   // [n_layers][max_rows][K]
    _Float16 *kv_all = nullptr;
    bool kv_i8 = false;              // the KV cache in int8 (config kv_int8)
    size_t kv_layer_bytes = 0;       // a layer's cache (values, then the int8 cache's scales)
    int64_t slots = 0;   // KV positions a layer holds: max_ctx rounded up to whole attention blocks
    // host side
    int pos = 0, last_pos = 0, last_n = 0;
    int timed_class = -1;
    bool moe_only = false;   // gv_model_moe: the router takes the rows as they are, the combine no next norm
    bool route_in_router = false;  // the router's last workgroup routes (off: route_kernel; on measured slower:
                                   // 23.5 us vs 10.6 + 6.2, the device-scope fences and one workgroup's route)
    int *counter = nullptr;        // the router's finished-workgroup count (zero between launches)
    bool moe_dec = false;          // the decode MoE kernels (moe_up_kernel, moe_down_kernel), where the shapes fit
    bool fused = true;             // dependent phases chained within one launch where the shapes fit (gv_model_set_fused)
    bool route_in_up = true;       // (fused) the experts' up launch routes the rows itself (gv_model_set_fused 2: off)
    bool router_shared_only = false;   // the MoE block's router launch with the routed logits given (gv_model_moe)
    bool block_up_routes = false;      // the MoE block's experts' up launch routes the rows itself (no route launch)
    const float *block_h = nullptr;    // the MoE block's input rows, which its router reads in place of x
    const float *block_logits = nullptr;   // the MoE block's given logits rows, which its up launch routes from
    int *ctr = nullptr;            // [n_layers][kFlagsPerLayer] the fused launches' flags (each launch clears its own)
    int *err = nullptr;            // set by a fused launch whose wait ran out (read back by gv_verify)
    uint64_t *trace = nullptr;     // gv_model_trace's stamps [GV_K_COUNT][8192 workgroups][8] (allocated when on)
    Prefill pf;
    std::vector<hipEvent_t> events;   // pairs around the timed class's launches
    // the verify step as a HIP graph per row count (captured on its second use; the step's parameters are read
    // from device memory, so one graph serves every position, token set and tree)
    bool use_graphs = true;
    hipGraphExec_t graphs[kMaxRows + 1] = {};
    bool seen[kMaxRows + 1] = {};
    size_t events_used = 0;
    StepParams host_sp{};
    int max_slots = 0, max_picks = 0;
    float *gdn_core = nullptr;   // [max_rows][nv dv] the delta rule's outputs
    int gdn_base = 0;            // the Gated DeltaNet layers' base slot (StepParams::gdn_base)
    std::vector<int> attn_layers, gdn_layers;   // the attention / Gated DeltaNet layers' indices, in order
    int *attn_index = nullptr;   // device copy of attn_layers
    // the MTP draft layer (mtp.hip): layers[n_layers] is its decoder layer, its KV after the main layers'
    bool has_mtp = false;
    Q4 mtp_fc;                                            // [H x 2 H]
    float *mtp_norm = nullptr, *mtp_pre_e = nullptr, *mtp_pre_h = nullptr;
    float *hbuf = nullptr;        // [3][max_rows][H]: the last verify's final-normed rows, the last MTP pass's
                                  // mtp.norm rows, rows given by the caller
    int hid_n = 0;                // rows of the first part the last verify wrote
    std::vector<int> keep_rows;   // after a keep with a path: the kept rows (an MTP row t's hidden: keep_rows[t])
    _Float16 *mtp_act = nullptr;  // [max_rows] fc's operands (2 H values a row)
    float *mtp_logits = nullptr;  // [vocab] the last MTP pass's last row
    StepParams *sp_mtp = nullptr;
    StepParams host_sp_mtp{};
    int mtp_last_n = 0;           // rows of the last MTP pass with logits (0: none yet)
    bool replaying = false;       // gv_model_replay's launches: each fused launch clears its own flags
    Q4 draft_head;                // lm_head's rows of the draft vocabulary (rows 0: the whole vocabulary)
    int32_t *draft_ids = nullptr; // device [draft_head.rows]
    uint8_t *draft_mem = nullptr;
    void *pick = nullptr;         // the draft pick's partials and result (mtp.hip)
    int *pick_host = nullptr;     // pinned: the pick's draft and probability, and the fused launches' error flag
    // an MTP pass as a HIP graph per (rows, with head), captured on its second use like the verify step's
    hipGraphExec_t mtp_graphs[kMaxRows + 1][2] = {};
    bool mtp_seen[kMaxRows + 1][2] = {};
};

constexpr int kAttnBlock = 64;   // positions an attention workgroup takes
constexpr int kFlagsPerLayer = 1024;   // flag words a layer's fused launches have (one a producer workgroup)
constexpr int kGdnFlagBase = 512;      // the Gated DeltaNet launch's: words [512, 1024); the output projection's below

// the model behind a C-ABI handle (model.hip), for the entry points of other files
Model &model_of(gv_model *g);

// the Gated DeltaNet layer (gdn.hip)
bool gdn_shape_ok(const gv_model_config &c, std::string &why);
int64_t gdn_conv_dim(const gv_model_config &c);
int64_t gdn_s_floats(const gv_model_config &c);   // a slot's recurrent state
int64_t gdn_c_floats(const gv_model_config &c);   // a slot's conv state
// the layer after its projections in one launch (ab_given: the a / b dots already in rlogits, launched apart)
int gdn_launch(Model &m, LayerW &L, int l, int M, bool ab_given, hipStream_t st);
int gdn_put_state(Model &m, LayerW &L, int slot, const float *conv, const float *S);
int gdn_get_state(const Model &m, const LayerW &L, int slot, float *conv, float *S);

// the verify step's launches (model.hip): one kernel class of layer l for M rows, and a layer's classes in order
int run_class(Model &m, int cls, int l, int M, hipStream_t st);
const int *layer_classes(int &count);
// the prefill MoE's work before the experts' products in two launches (prefill.hip): the rows' routes, then the
// picks grouped by expert and placed with the shared expert's gate and the rows' operands as roles of one launch;
// hidden sizes up to kPrefillFrontMaxH (the gate role's LDS, 20 bytes a hidden value, within a workgroup's 160 KB)
constexpr int kPrefillFrontMaxH = 4096;
int prefill_route(const float *logits, int M, int E, int K, int *ids, float *w, hipStream_t st);
int prefill_rest(const uint16_t *gate_row, int H, const float *h, int M, int E, int K, float *logits, float *gate,
                 _Float16 *act, int64_t act_stride, const int *ids, int *start, int *n_slots, int *slot_expert,
                 int *slot_start, int *slot_count, int *n_picks, int *pick_token, int *pick_of, hipStream_t st);
// the same launch's gate and operand roles alone (the MoE block at up to 8 rows with its routed logits given)
int prefill_gate_ops(const uint16_t *gate_row, int H, const float *h, int M, int E, float *logits, float *gate,
                     _Float16 *act, int64_t act_stride, hipStream_t st);
// the MTP layer's buffers (mtp.hip), at gv_model_create
int mtp_alloc(Model &m);
void mtp_free(Model &m);      // the draft head
void mtp_release(Model &m);   // everything the MTP layer holds outside Model::allocs (at gv_model_free)

}  // namespace gv
