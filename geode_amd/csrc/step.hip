// step.hip - the whole verify step (the embedding, every layer, the final norm and lm_head) as ONE persistent kernel
// on MI355X: a workgroup per compute unit, all resident (a cooperative launch), the step's phases separated by grid
// barriers. The arithmetic is the per-phase kernels' (model.hip: the reference's int8 path, kernels.cpp:1254-1420,
// model.cpp:3690-4587) operation for operation, so both paths give the same bits; what changes is how phases meet:
//
// * No kernel boundary between phases. A barrier is a flag per workgroup, gathered by workgroup 0, which then
//   releases eight words (one per XCD): about 1.5 us for 256 workgroups.
// * No cache flush or invalidate either (on gfx950 each costs about as much as the barrier): every buffer that one
//   workgroup writes and another reads within the step is written and read with device-coherent (sc1) vector memory
//   operations (common.hpp: xld16 / xst16), which are coherent across the XCDs' separate L2 caches; weights and the
//   KV cache of earlier steps, written before the launch, are read as usual.
// * Each phase's weights are loaded while its barrier is still waiting (a workgroup's share of a phase's weights is
//   a few tens of KB: registers hold it), so after the barrier only the activations' round trip remains.
// * The route of the step's rows is computed by every workgroup from the router logits (the same bits everywhere),
//   so no barrier separates the route from the experts' products; the SwiGLU and its operands come out of the
//   gate|up products (a workgroup takes the gate and the up tile of the same 16 values).
//
// Per layer, eight barriers: qkv products | attention per (block of 64 positions, KV head), with the queries' and
// the new keys' norm and rotation and the new keys and values appended | the blocks' merge | the output projection
// (+= residual) | the router (with the post-attention norm and the experts' operands) | route + the experts'
// gate|up products + SwiGLU | the down products | the combine (+= residual, the next norm and operands).
#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "layer_common.hpp"
#include "mfma_gemv.hpp"
#include "model.hpp"
#include "step.hpp"

namespace gv {

namespace {

// ---------------------------------------------------------------- the grid barrier
constexpr unsigned kSpinLimit = 1u << 21;   // polls before a wait gives up (about a second): the kernel then ends
constexpr unsigned kAbort = 0xFFFFFFFFu;

__device__ inline unsigned ld_flag(const unsigned *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline void st_flag(unsigned *p, unsigned v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

__device__ inline bool spin_ge(const unsigned *p, unsigned target) {
    for (unsigned it = 0; it < kSpinLimit; ++it)
        if (ld_flag(p) >= target) return true;
    return false;
}

__device__ inline void sync_fail(const StepDev &a) {
    __hip_atomic_fetch_or(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int i = 0; i < 8; ++i) st_flag(a.rel + i * 64, kAbort);
}

// arrive at barrier `gen`: this workgroup's stores are complete (each thread waits for its own, then the workgroup
// meets), then its flag
__device__ inline void stamp(const StepDev &a, unsigned gen, int which) {
    if (a.stamps && threadIdx.x == 0) {
        const unsigned nb = 1u + 8u * static_cast<unsigned>(a.n_layers);
        const unsigned i = (gen - 1u) % nb;   // the barrier's index within the step (gen0 is a multiple of nb)
        a.stamps[(static_cast<size_t>(blockIdx.x) * nb + i) * 2 + which] = __builtin_amdgcn_s_memrealtime();
    }
}

// sub-phase stamps of layer kDbgLayer (a measurement aid): slot i of the workgroup's 32 after the barrier stamps
constexpr int kDbgLayer = 5;
__device__ inline void dstamp(const StepDev &a, int l, int i) {
    if (a.stamps && l == kDbgLayer && threadIdx.x == 0) {
        const size_t nb = 1u + 8u * static_cast<unsigned>(a.n_layers);
        a.stamps[static_cast<size_t>(gridDim.x) * nb * 2 + blockIdx.x * 32 + i] = __builtin_amdgcn_s_memrealtime();
    }
}

__device__ inline void arrive(const StepDev &a, unsigned gen) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    stamp(a, gen, 0);
    if (threadIdx.x == 0) st_flag(a.flags + blockIdx.x * 16, gen);
}

// wait at barrier `gen`: workgroup 0 gathers every flag and releases the eight words, every workgroup polls its
// XCD's word. A wait that polls kSpinLimit times sets the error word and releases everyone with kAbort: every later
// wait then passes at once (abort: the workgroup's LDS flag) and the kernel ends with an error for the host.
__device__ inline void wait(const StepDev &a, unsigned gen, int *abort) {
    const bool aborted = *abort != 0;
    if (blockIdx.x == 0 && !aborted) {
        bool ok = true;
        for (int b = threadIdx.x; b < static_cast<int>(gridDim.x); b += blockDim.x) ok = ok && spin_ge(a.flags + b * 16, gen);
        if (!ok) {
            sync_fail(a);
            *abort = 1;
        }
        __syncthreads();
        if (threadIdx.x < 8 && *abort == 0) st_flag(a.rel + threadIdx.x * 64, gen);
    }
    if (threadIdx.x == 0 && !aborted) {
        const unsigned *w = a.rel + (blockIdx.x % 8) * 64;
        if (!spin_ge(w, gen)) {
            sync_fail(a);
            *abort = 1;
        } else if (ld_flag(w) == kAbort) {
            *abort = 1;
        }
    }
    __syncthreads();
    stamp(a, gen, 1);
    asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------- the exchange arena
// byte offsets into StepDev::arena, through a descriptor of exactly the arena's size: loads and stores at kNoStore
// (past the arena: the arena is under 2 GB) read 0 and write nothing
constexpr uint32_t kNoStore = 0xFFFFF000u;   // far from wrapping with an instruction offset (< 4 KB)
__device__ inline __amdgpu_buffer_rsrc_t ars(const StepDev &a) { return uniform_rsrc(a.arena, a.arena_bytes); }
__device__ inline float aldf(const StepDev &a, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ars(a), off, 0, kSc1));
}
__device__ inline xu4 ald16(const StepDev &a, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(ars(a), off, 0, kSc1); }
__device__ inline float4 ald4f(const StepDev &a, uint32_t off) { return __builtin_bit_cast(float4, ald16(a, off)); }
__device__ inline void astf(const StepDev &a, uint32_t off, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), ars(a), off, 0, kSc1);
}
__device__ inline void ast16(const StepDev &a, uint32_t off, xu4 v) { __builtin_amdgcn_raw_buffer_store_b128(v, ars(a), off, 0, kSc1); }
__device__ inline void ast4f(const StepDev &a, uint32_t off, float4 v) { ast16(a, off, __builtin_bit_cast(xu4, v)); }
// float index i of the part at byte offset base
__device__ inline uint32_t fo(uint32_t base, int64_t i) { return base + static_cast<uint32_t>(i) * 4u; }

// ---------------------------------------------------------------- LDS
// [0, 2 KB) the E4M3 table; the route state (kept from the route to the combine); the abort flag and a small
// reduction buffer; then one region the phases reuse
constexpr size_t kLdsTab = 0;
constexpr size_t kLdsRoute = 2048;
constexpr size_t kLdsRouteBytes = (sizeof(RouteState) + 255) / 256 * 256;
constexpr size_t kLdsGlob = kLdsRoute + kLdsRouteBytes;   // [E + 1][3] the layer's expert globals (E <= 256)
constexpr size_t kLdsMisc = kLdsGlob + 257 * 3 * 4 + 4;
constexpr size_t kLdsScratch = (kLdsMisc + 256 + 15) / 16 * 16;

struct Lds {
    uint2 *tab;
    RouteState *rs;
    float *eg;     // [E + 1][3] gate half, up half, down globals of the layer's experts
    int *abort;
    double *red;   // 16 doubles
    float *segg;   // [3] the qkv product's q | gate, k, v globals
    uint8_t *scratch;
    __device__ explicit Lds(uint8_t *p)
        : tab(reinterpret_cast<uint2 *>(p + kLdsTab)), rs(reinterpret_cast<RouteState *>(p + kLdsRoute)),
          eg(reinterpret_cast<float *>(p + kLdsGlob)), abort(reinterpret_cast<int *>(p + kLdsMisc)), red(reinterpret_cast<double *>(p + kLdsMisc + 16)),
          segg(reinterpret_cast<float *>(p + kLdsMisc + 144)), scratch(p + kLdsScratch) {}
};

// ---------------------------------------------------------------- the skinny products
// A phase's products on one workgroup: its units (16-row tiles, or pairs of tiles), each RP ranges of NS
// super-chunks; task k = unit (k / RP), range (k % RP) goes to wave k % 4, its weights held in a ring of D tasks (the
// first D loaded before the phase's barrier ends). A task's MFMA chain is mfma_tiles' (mfma_gemv.hpp) for one wave's
// range; the ranges' sums go to LDS, and fin adds them in range order once a batch of whole units is done
// (UB = max(1, 4 / RP) units, BR = max(1, RP / 4) rounds of the four waves).
//
// The loop body holds no conditional load or store: a wave's loads return in order and the compiler can only count
// the ones in flight when every path issues the same, so a conditional one makes it wait for all of them (the ring
// would then be one task deep). A task past the end loads through a zero-length buffer descriptor (no memory is
// read), fin stores of rows past the end go to an offset past the buffer (dropped), and the B operands load once per
// run when they stay the same for the wave (RELOAD = false), else every round.
template <int NS, int NTT, int D, int RP>
struct Prod {
    static constexpr int BR = RP >= 4 ? RP / 4 : 1, UB = RP >= 4 ? 1 : 4 / RP;
    static_assert(D % BR == 0, "a batch of rounds fits the ring's unrolled rounds");
    uint4 cw[D][NS];
    uint32_t sw[D][NS];
    int nunits = 0, ntasks = 0;

    __device__ void setup(int units) {
        nunits = units;
        ntasks = units * RP;
    }
    // addr(k, codes, scales): the task's first super-chunk block (1 KB of codes, 128 B of scales), uniform
    template <typename AddrFn>
    __device__ void load(uint4 (&c)[NS], uint32_t (&s)[NS], int k, AddrFn &addr) {
        const int l = threadIdx.x % 64, lq = l % 16, lg = l / 16;
        const bool live = k < ntasks;
        const uint8_t *cb, *sb;
        addr(live ? k : 0, cb, sb);
        const __amdgpu_buffer_rsrc_t rc = uniform_rsrc(cb, live ? NS * 1024 : 0);
        const __amdgpu_buffer_rsrc_t rsc = uniform_rsrc(sb, live ? NS * 128 : 0);
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            const xu4 v = __builtin_amdgcn_raw_buffer_load_b128(rc, i * 1024 + l * 16, 0, 2);   // nt
            c[i] = make_uint4(v.x, v.y, v.z, v.w);
            s[i] = __builtin_amdgcn_raw_buffer_load_b32(rsc, i * 128 + (lq * 2 + lg / 2) * 4, 0, 2);
        }
    }
    template <typename AddrFn>
    __device__ void prefetch(AddrFn &addr) {
        const int w = threadIdx.x / 64;
#pragma unroll
        for (int q = 0; q < D; ++q) load(cw[q], sw[q], 4 * q + w, addr);
    }

    // one round j (task k = 4 j + wave) with ring slot Q (= j % D); false when past the last round
    template <int Q, bool RELOAD, typename AddrFn, typename BFn, typename FinFn>
    __device__ bool round(int j, int nrounds, h8 (&bh)[NS * 4][NTT], h8 (&bl)[NS * 4][NTT], AddrFn &addr, BFn &bops,
                          FinFn &fin, f4 *part, const uint2 *tab) {
        if (j >= nrounds) return false;
        const int w = threadIdx.x / 64, l = threadIdx.x % 64;
        const int k = 4 * j + w;
        const int batch = j / BR;
        if (RELOAD) bops(k < ntasks ? k : ntasks - 1, bh, bl);
        const uint32_t magic = 0x64006400u;
        f4 acc[NTT], acl[NTT];
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt) acc[tt] = acl[tt] = f4{0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const uint32_t words[4] = {cw[Q][s].x, cw[Q][s].y, cw[Q][s].z, cw[Q][s].w};
#pragma unroll
            for (int j4 = 0; j4 < 4; ++j4) {
                const h8 av = decode8(words[j4], tab[(sw[Q][s] >> (8 * j4)) & 0xFFu], magic);
                const int c = s * 4 + j4;
#pragma unroll
                for (int tt = 0; tt < NTT; ++tt) {
                    acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bh[c][tt], acc[tt], 0, 0, 0);
                    acl[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bl[c][tt], acl[tt], 0, 0, 0);
                }
            }
        }
        load(cw[Q], sw[Q], k + 4 * D, addr);
        const int tib = k - batch * BR * 4;   // the task's place in its batch
        if (k < ntasks) {
#pragma unroll
            for (int tt = 0; tt < NTT; ++tt) part[(((batch & 1) * 4 * BR + tib) * NTT + tt) * 64 + l] = acc[tt] + acl[tt];
        }
        if ((Q + 1) % BR == 0) {   // the batch's last round (nrounds is a whole number of batches)
            __syncthreads();
            constexpr int ITEMS = UB * NTT * 64;
#pragma unroll
            for (int o0 = 0; o0 < ITEMS; o0 += 256) {
                const int o = o0 + static_cast<int>(threadIdx.x);
                const bool in = o < ITEMS;
                const int oo = in ? o : o % ITEMS;
                const int ub = oo / (NTT * 64), tt = (oo / 64) % NTT, ll = oo % 64;
                const int unit = batch * UB + ub;
                fin(unit < nunits ? unit : nunits - 1, tt, ll, part + (((batch & 1) * 4 * BR + ub * RP) * NTT + tt) * 64 + ll,
                    NTT * 64, in && unit < nunits);
            }
        }
        return true;
    }

    // bops(k, bh, bl): task k's B operands; fin(unit, tt, lane, part, stride, live): the unit's range sums
    // part[r * stride] (r < RP) for token tile tt and the lane's f4, called by every lane (live false: store nothing)
    template <bool RELOAD, typename AddrFn, typename BFn, typename FinFn>
    __device__ void run(AddrFn &addr, BFn bops, FinFn fin, f4 *part, const uint2 *tab) {
        static_assert(D == 2 || D == 4 || D == 8, "the ring is unrolled for two, four or eight slots");
        if (ntasks > 0) {   // uniform
            const int w = threadIdx.x / 64;
            const int nrounds = (ntasks + 3) / 4;
            h8 bh[NS * 4][NTT], bl[NS * 4][NTT];
            if (!RELOAD) bops(w < ntasks ? w : ntasks - 1, bh, bl);
            for (int j0 = 0; j0 < nrounds; j0 += D) {
                if (!round<0, RELOAD>(j0, nrounds, bh, bl, addr, bops, fin, part, tab)) break;
                if (!round<1, RELOAD>(j0 + 1, nrounds, bh, bl, addr, bops, fin, part, tab)) break;
                if constexpr (D >= 4) {
                    if (!round<2 % D, RELOAD>(j0 + 2, nrounds, bh, bl, addr, bops, fin, part, tab)) break;
                    if (!round<3 % D, RELOAD>(j0 + 3, nrounds, bh, bl, addr, bops, fin, part, tab)) break;
                }
                if constexpr (D == 8) {
                    if (!round<4 % D, RELOAD>(j0 + 4, nrounds, bh, bl, addr, bops, fin, part, tab)) break;
                    if (!round<5 % D, RELOAD>(j0 + 5, nrounds, bh, bl, addr, bops, fin, part, tab)) break;
                    if (!round<6 % D, RELOAD>(j0 + 6, nrounds, bh, bl, addr, bops, fin, part, tab)) break;
                    if (!round<7 % D, RELOAD>(j0 + 7, nrounds, bh, bl, addr, bops, fin, part, tab)) break;
                }
            }
        }
        __syncthreads();   // the last batch's sums are read before the LDS is reused
    }
};

// tasks in flight per wave: about 16 KB of weights (a task is NS KB of codes), and a whole number of batches (the
// ring is unrolled per batch)
template <int NS, int RP>
constexpr int ring_for() { return NS >= 4 ? 4 : 8; }

// the workgroup's share [u0, u1) of n units split evenly over workgroups 1 .. G - 1: workgroup 0 gathers the barrier
// flags, and loads issued before a wait would hold its polls back (a wave's loads return in order), so it takes no
// share of the phases whose weights load before their barrier
__device__ inline void my_units(int n, int &u0, int &u1) {
    const int G = gridDim.x - 1, b = static_cast<int>(blockIdx.x) - 1;
    u0 = b < 0 ? 0 : static_cast<int>(static_cast<int64_t>(n) * b / G);
    u1 = b < 0 ? 0 : static_cast<int>(static_cast<int64_t>(n) * (b + 1) / G);
}

// The units of a per-slot product (per units a slot): with n_slots <= G - 1 a workgroup (1 .. G - 1) takes units of
// one slot only, slot s having workgroups [ceil(s (G - 1) / n), ceil((s + 1) (G - 1) / n)), so its B operands stay
// the same (true); else an even split of all units (false: the operands change with the slot)
__device__ inline bool slot_units(int n_slots, int per, int &u0, int &u1) {
    const int G1 = static_cast<int>(gridDim.x) - 1, b = static_cast<int>(blockIdx.x) - 1;
    if (n_slots > G1 || n_slots < 1) {
        my_units(n_slots * per, u0, u1);
        return false;
    }
    if (b < 0) {
        u0 = u1 = 0;
        return true;
    }
    const int s = b * n_slots / G1;
    const int first = (s * G1 + n_slots - 1) / n_slots, next = ((s + 1) * G1 + n_slots - 1) / n_slots;
    const int nw = next - first, idx = b - first;
    u0 = s * per + per * idx / nw;
    u1 = s * per + per * (idx + 1) / nw;
    return true;
}

// B operands of range r from act16 rows row_of(j) (j < n; operands of rows past n are zero), as mfma_tiles' bload
template <int NS, int NTT, typename RowFn>
__device__ inline void bops_act(const StepDev &a, uint32_t act, int64_t stride, int n, int r, RowFn row_of,
                                h8 (&bh)[NS * 4][NTT], h8 (&bl)[NS * 4][NTT]) {
    const int l = threadIdx.x % 64, lq = l % 16, lg = l / 16;
    xu4 ha[NS * 4][NTT], la[NS * 4][NTT];
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt) {
        const int j = tt * 16 + lq;
        const int row = row_of(j < n ? j : n - 1);
#pragma unroll
        for (int c = 0; c < NS * 4; ++c) {
            const int g = (r * NS * 4 + c) * 4 + lg;
            const uint32_t off = act + static_cast<uint32_t>((row * stride + g * 16) * 2);
            ha[c][tt] = ald16(a, off);
            la[c][tt] = ald16(a, off + 16);
        }
    }
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt) {
        const bool live = tt * 16 + lq < n;
#pragma unroll
        for (int c = 0; c < NS * 4; ++c) {
            bh[c][tt] = live ? __builtin_bit_cast(h8, ha[c][tt]) : h8{0, 0, 0, 0, 0, 0, 0, 0};
            bl[c][tt] = live ? __builtin_bit_cast(h8, la[c][tt]) : h8{0, 0, 0, 0, 0, 0, 0, 0};
        }
    }
}

// the dense products' rows: the step's rows in order
struct Ident {
    __device__ int operator()(int j) const { return j; }
};

// ---------------------------------------------------------------- phases
// Each phase function: its weights' loads (the previous phase has arrived at the barrier), the wait, its work, the
// arrival at the next barrier; it returns the next barrier's generation.

// The embedding rows (embed_kernel: dequant_row bit for bit) into x and, with the first layer's input RMSNorm, the
// products' operands; workgroup t takes row t
__device__ __forceinline__ void ph_embed(const StepDev &a, Lds s) {
    const StepParams *sp = a.sp;
    const int t = blockIdx.x;
    if (t >= sp->M) return;
    const int64_t r = sp->tokens[t];
    const int ng = a.H / 8;
    Q4 w;
    w.codes = a.emb_c;
    w.scales = a.emb_s;
    w.rows = a.V;
    w.cols = a.H;
    float v[4][8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int g = threadIdx.x + q * blockDim.x;
#pragma unroll
        for (int b = 0; b < 8; ++b) v[q][b] = 0.0f;
        if (g >= ng) continue;
        uint32_t word, sb;
        tq4_word(w, r, g, word, sb);
        const float sc = __fmul_rn(e4m3_to_f32(sb), a.emb_g);
#pragma unroll
        for (int b = 0; b < 8; ++b)
            v[q][b] = __fmul_rn(static_cast<float>(2 * static_cast<int>((word >> (4 * b)) & 15u) - 15), sc);
        ast4f(a, fo(a.o_x, t * a.H + g * 8), make_float4(v[q][0], v[q][1], v[q][2], v[q][3]));
        ast4f(a, fo(a.o_x, t * a.H + g * 8 + 4), make_float4(v[q][4], v[q][5], v[q][6], v[q][7]));
    }
    norm_quant_regs(v, ng * 8, a.layers[0].in_norm, a.eps,
                    XDst{a.arena, a.arena_bytes, a.o_act_h + static_cast<uint32_t>(t * act_halves(a.H) * 2)}, nullptr, s.red);
}

// a float4 stored at byte offset off when ok, else nowhere, and the same for a load (0)
__device__ inline void ast4f_if(const StepDev &a, bool ok, uint32_t off, float4 v) { ast4f(a, ok ? off : kNoStore, v); }
__device__ inline float4 ald4f_if(const StepDev &a, bool ok, uint32_t off) { return ald4f(a, ok ? off : kNoStore); }

// the range sums of one pass of R ranges in range order (mfma_tiles' wave order)
template <int R>
__device__ inline f4 pass_sum(const f4 *pp, int stride, int first) {
    f4 sum = pp[first * stride];
#pragma unroll
    for (int r = 1; r < R; ++r) sum += pp[(first + r) * stride];
    return sum;
}

// qkv = W_qkv act_h, each segment's global (q | gate, k, v) applied (qkv_out of model.hip)
template <int NS, int NTT, int RP>
__device__ __forceinline__ unsigned ph_qkv(const StepDev &a, int l, unsigned gen, Lds s) {
    const LayerDev &L = a.layers[l];
    const int M = a.sp->M, H = a.H, nsc = H / kSuperK, rows = a.qkv_rows;
    const int qr = a.nh * 2 * a.hd, kr = qr + a.nkv * a.hd;
    // the segment globals by a lane-varying LDS index (read after the wait's workgroup barrier)
    if (threadIdx.x == 0) s.segg[0] = L.g_q, s.segg[1] = L.g_k, s.segg[2] = L.g_v;
    const float *segg = s.segg;
    int u0, u1;
    my_units(static_cast<int>(tiles_rows(rows)), u0, u1);
    const uint8_t *wc = L.qkv_c, *ws = L.qkv_s;
    auto addr = [=, &a](int k, const uint8_t *&cb, const uint8_t *&sb) {
        const int64_t blk = static_cast<int64_t>(u0 + k / RP) * nsc + (k % RP) * NS;
        cb = wc + blk * 1024;
        sb = ws + blk * 128;
    };
    Prod<NS, NTT, ring_for<NS, RP>(), RP> p;
    p.setup(u1 - u0);
    p.prefetch(addr);
    wait(a, gen, s.abort);
    dstamp(a, l, 30);
    auto bops = [=, &a](int k, h8(&bh)[NS * 4][NTT], h8(&bl)[NS * 4][NTT]) {
        bops_act<NS, NTT>(a, a.o_act_h, act_halves(H), M, k % RP, Ident(), bh, bl);
    };
    auto fin = [=, &a](int unit, int tt, int ll, const f4 *pp, int stride, bool live) {
        const int j = tt * 16 + ll % 16;
        const int row = (u0 + unit) * kTileR + 4 * (ll / 16);
        const float g = segg[(row >= qr) + (row >= kr)];
        const f4 sum = pass_sum<RP>(pp, stride, 0);
        ast4f_if(a, live && j < M && row < rows, fo(a.o_qkv, j * rows + row),
                 make_float4(sum[0] * g, sum[1] * g, sum[2] * g, sum[3] * g));
    };
    if (RP <= 4) p.template run<false>(addr, bops, fin, reinterpret_cast<f4 *>(s.scratch), s.tab);
    else p.template run<true>(addr, bops, fin, reinterpret_cast<f4 *>(s.scratch), s.tab);
    dstamp(a, l, 31);
    arrive(a, gen + 1);
    return gen + 1;
}

// Attention of (block b of 64 positions, KV head kh) items, attn_block_kernel's arithmetic. The block's cached keys
// and values are loaded before the barrier; the step's own rows in the block are made here from qkv_out (the keys'
// RMSNorm(1 + w) and partial RoPE as qk_rope_kernel, model.cpp:3714-3733) and appended to the cache; the queries of
// the KV head are normalized and rotated (qk_rope_kernel) a wave per 16, then the scores, the block's softmax and
// the weighted values on the matrix cores; the partial (weighted values, max, sum) to parts.
struct AttnPre {
    uint4 kr[8], vr[8];
};

__device__ inline void attn_prefetch(const StepDev &a, const LayerDev &L, int item, int total, AttnPre &pre) {
    const int b = item / a.nkv, kh = item % a.nkv;
    const int hd = a.hd, s0 = b * kAttnBlock;
    const _Float16 *kg = L.kv + k_index(a.slots, hd, kh, s0, 0);
    const _Float16 *vg = L.kv + v_index(a.slots, hd, a.nkv, kh, s0, 0);
    const int kpr = hd / 8, nl = hd / 32;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        if (u >= nl) break;
        const int i = threadIdx.x + u * 256;
        const int r = i / kpr, c = i % kpr;
        pre.kr[u] = s0 + r < total ? *reinterpret_cast<const uint4 *>(kg + static_cast<int64_t>(r) * hd + c * 8)
                                   : make_uint4(0, 0, 0, 0);
        pre.vr[u] = *reinterpret_cast<const uint4 *>(vg + static_cast<int64_t>(i) * 8);
    }
}

// one (row, head) vector of qkv_out normalized (RMSNorm(1 + w): the double sum of squares per 64 dims by wave_sum,
// the four added in order, as qk_rope_kernel's four waves) and rotated, by one wave: dims d = lane + 64 i (i < 4) of
// the result from the raw x[i]. The rotated dims are d < 2 half <= 64 (lane d, i = 0); c, sn: this lane's cos and sin
// at the vector's position (rope_cs); rb: the wave's LDS row of 256 floats.
__device__ inline void rope_cs(const float *cos_t, const float *sin_t, int half, int p, float &c, float &sn) {
    const int lane = threadIdx.x % 64;
    const int j = lane < half ? lane : lane - half;
    const bool rot = lane < 2 * half;
    c = rot ? cos_t[static_cast<int64_t>(p) * half + j] : 0.0f;
    sn = rot ? sin_t[static_cast<int64_t>(p) * half + j] : 0.0f;
}

__device__ inline void norm_rope(const float (&x)[4], int hd, int half, float eps, const float (&nw)[4], float c,
                                 float sn, float *rb, float (&out)[4]) {
    const int lane = threadIdx.x % 64;
    double ss[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ss[i] = wave_sum(static_cast<double>(x[i]) * static_cast<double>(x[i]));
    const double tot = ((ss[0] + ss[1]) + ss[2]) + ss[3];
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(static_cast<float>(tot / static_cast<double>(hd)), eps)));
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __fmul_rn(__fmul_rn(x[i], inv), nw[i]);
    if (lane < 2 * half) rb[lane] = v[0];
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = lane + 64 * i < hd ? v[i] : 0.0f;
    if (lane < half) out[0] = __fsub_rn(__fmul_rn(v[0], c), __fmul_rn(rb[lane + half], sn));
    else if (lane < 2 * half) out[0] = __fadd_rn(__fmul_rn(v[0], c), __fmul_rn(rb[lane - half], sn));
    __builtin_amdgcn_wave_barrier();   // rb is rewritten by the wave's next vector
}

// 1 + w of a per-head norm at this lane's dims d = lane + 64 i
__device__ inline void head_norm_w(const float *w, int hd, float (&nw)[4]) {
    const int lane = threadIdx.x % 64;
#pragma unroll
    for (int i = 0; i < 4; ++i) nw[i] = lane + 64 * i < hd ? __fadd_rn(1.0f, w[lane + 64 * i]) : 0.0f;
}

__device__ __forceinline__ void attn_item(const StepDev &a, const LayerDev &L, int item, const AttnPre &pre, uint8_t *scratch, int layer) {
    const StepParams *sp = a.sp;
    const int b = item / a.nkv, kh = item % a.nkv;
    const int pos = sp->pos, M = sp->M, total = pos + M;
    const int hd = a.hd, nh = a.nh, nkv = a.nkv, half = a.half;
    const int s0 = b * kAttnBlock;
    const int kld = attn_k_ld(hd);
    _Float16 *ks = reinterpret_cast<_Float16 *>(scratch), *vs = ks + kAttnBlock * kld;
    float *rowbuf = reinterpret_cast<float *>(vs + hd * kAttnVld);   // [4 waves][256]
    _Float16 *qs = reinterpret_cast<_Float16 *>(rowbuf + 4 * 256);   // [4 waves][2][16][hd]: hi, lo
    const int wave = threadIdx.x / 64, l = threadIdx.x % 64, lq = l % 16, lg = l / 16;
    float *rb = rowbuf + wave * 256;
    {   // stage the cache's keys and values (as attn_block_kernel)
        const int kpr = hd / 8, nl = hd / 32;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (u >= nl) break;
            const int i = threadIdx.x + u * 256;
            const int r = i / kpr, c = i % kpr;
            *reinterpret_cast<uint4 *>(ks + r * kld + c * 8) = pre.kr[u];
            const int d = i / (kAttnBlock / 8), cv = i % (kAttnBlock / 8);
            uint4 v = pre.vr[u];
            const int lim = total - s0 - cv * 8;
            if (lim < 8) {
                uint32_t w4[4] = {v.x, v.y, v.z, v.w};
                for (int k = 0; k < 4; ++k) {
                    if (2 * k >= lim) w4[k] = 0;
                    else if (2 * k + 1 >= lim) w4[k] &= 0xFFFFu;
                }
                v = make_uint4(w4[0], w4[1], w4[2], w4[3]);
            }
            *reinterpret_cast<uint4 *>(vs + d * kAttnVld + cv * 8) = v;
        }
    }
    __syncthreads();
    dstamp(a, layer, 1);
    // the step's rows in this block: keys normalized and rotated, values as they are, into LDS and the cache
    const int kbase = nh * 2 * hd, vbase = kbase + nkv * hd;
    for (int t = wave; t < M; t += 4) {
        const int slot = pos + t;
        if (slot < s0 || slot >= s0 + kAttnBlock) continue;
        float kx[4], vx[4], ko[4], nw[4], c, sn;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = l + 64 * i;
            kx[i] = d < hd ? aldf(a, fo(a.o_qkv, t * a.qkv_rows + kbase + kh * hd + d)) : 0.0f;
            vx[i] = d < hd ? aldf(a, fo(a.o_qkv, t * a.qkv_rows + vbase + kh * hd + d)) : 0.0f;
        }
        head_norm_w(L.k_norm, hd, nw);
        rope_cs(a.rope_cos, a.rope_sin, half, pos + sp->depth[t], c, sn);
        norm_rope(kx, hd, half, a.eps, nw, c, sn, rb, ko);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = l + 64 * i;
            if (d >= hd) continue;
            const _Float16 k16 = f16_of(ko[i]), v16 = static_cast<_Float16>(vx[i]);
            ks[(slot - s0) * kld + d] = k16;
            vs[d * kAttnVld + (slot - s0)] = v16;
            L.kv[k_index(a.slots, hd, kh, slot, d)] = k16;
            L.kv[v_index(a.slots, hd, nkv, kh, slot, d)] = v16;
        }
    }
    __syncthreads();
    dstamp(a, layer, 2);
    const int group = nh / nkv, NQ = group * M, nqt = (NQ + 15) / 16;
    const int nch = hd / 32;
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn(static_cast<float>(hd)));
    _Float16 *qh = qs + wave * 2 * 16 * hd, *qlo = qh + 16 * hd;
    for (int qt = wave; qt < nqt; qt += 4) {
        {   // the tile's 16 queries normalized and rotated (qk_rope_kernel's arithmetic: the double sum of squares
            // per 64 dims by wave_sum, the four added in order), eight at a time: every raw value and table entry of
            // the eight loaded first, the 32 wave sums in batches of sixteen independent chains, the rotated dims
            // (lane < 2 half <= 64) through LDS, then hi + lo halves to LDS
            constexpr int QB = 8;
            float *qrot = rb;   // [64] per query: the wave's row buffer (free during the prepass)
            float nw[4];
            head_norm_w(L.q_norm, hd, nw);
#pragma unroll 1
            for (int qb0 = 0; qb0 < 16; qb0 += QB) {
                float xr[QB][4], cq[QB], sq[QB], inv[QB];
#pragma unroll
                for (int q = 0; q < QB; ++q) {
                    const int qi = qt * 16 + qb0 + q;
                    const int tq = qi < NQ ? qi / group : 0, hq = kh * group + (qi < NQ ? qi % group : 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int d = l + 64 * i;
                        xr[q][i] = d < hd ? aldf(a, fo(a.o_qkv, tq * a.qkv_rows + hq * 2 * hd + d)) : 0.0f;
                    }
                    rope_cs(a.rope_cos, a.rope_sin, half, pos + sp->depth[tq], cq[q], sq[q]);
                }
#pragma unroll
                for (int q0 = 0; q0 < QB; q0 += 4) {
                    double ss[4][4];
#pragma unroll
                    for (int qq = 0; qq < 4; ++qq)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            ss[qq][i] =
                                wave_sum(static_cast<double>(xr[q0 + qq][i]) * static_cast<double>(xr[q0 + qq][i]));
#pragma unroll
                    for (int qq = 0; qq < 4; ++qq) {
                        const double tot = ((ss[qq][0] + ss[qq][1]) + ss[qq][2]) + ss[qq][3];
                        inv[q0 + qq] = __fdiv_rn(
                            1.0f, __fsqrt_rn(__fadd_rn(static_cast<float>(tot / static_cast<double>(hd)), a.eps)));
                    }
                }
#pragma unroll
                for (int q = 0; q < QB; ++q)
#pragma unroll
                    for (int i = 0; i < 4; ++i) xr[q][i] = __fmul_rn(__fmul_rn(xr[q][i], inv[q]), nw[i]);
#pragma unroll
                for (int q0 = 0; q0 < QB; q0 += 4) {   // rb holds four rotated vectors at a time
#pragma unroll
                    for (int qq = 0; qq < 4; ++qq)
                        if (l < 2 * half) qrot[qq * 64 + l] = xr[q0 + qq][0];
                    __builtin_amdgcn_wave_barrier();
                    float partner[4];
#pragma unroll
                    for (int qq = 0; qq < 4; ++qq)
                        partner[qq] = l < half ? qrot[qq * 64 + l + half] : l < 2 * half ? qrot[qq * 64 + l - half] : 0.0f;
                    __builtin_amdgcn_wave_barrier();
#pragma unroll
                    for (int qq = 0; qq < 4; ++qq) {
                        const int q = q0 + qq;
                        if (l < half) xr[q][0] = __fsub_rn(__fmul_rn(xr[q][0], cq[q]), __fmul_rn(partner[qq], sq[q]));
                        else if (l < 2 * half)
                            xr[q][0] = __fadd_rn(__fmul_rn(xr[q][0], cq[q]), __fmul_rn(partner[qq], sq[q]));
                    }
                }
#pragma unroll
                for (int q = 0; q < QB; ++q)
                    if (qt * 16 + qb0 + q < NQ) {   // uniform
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int d = l + 64 * i;
                            if (d >= hd) continue;
                            _Float16 hi, lo;
                            split_f16(xr[q][i], hi, lo);
                            qh[(qb0 + q) * hd + d] = hi;
                            qlo[(qb0 + q) * hd + d] = lo;
                        }
                    }
            }
            __builtin_amdgcn_wave_barrier();
        }
        dstamp(a, layer, 3);
        const int qi = qt * 16 + lq;
        const bool qvalid = qi < NQ;
        const int tq = qvalid ? qi / group : 0, hq = kh * group + (qvalid ? qi % group : 0);
        half8 qb[8], ql[8];
#pragma unroll
        for (int ch = 0; ch < 8; ++ch) {
            const half8 z = {0, 0, 0, 0, 0, 0, 0, 0};
            qb[ch] = (qvalid && ch < nch) ? *reinterpret_cast<const half8 *>(qh + lq * hd + ch * 32 + 8 * lg) : z;
            ql[ch] = (qvalid && ch < nch) ? *reinterpret_cast<const half8 *>(qlo + lq * hd + ch * 32 + 8 * lg) : z;
        }
        __builtin_amdgcn_wave_barrier();   // qh / qlo are rewritten by the wave's next tile
        const uint32_t vis = qvalid ? sp->vis[tq] : 0u;
        float4v ch_[4], cl_[4];
#pragma unroll
        for (int pt = 0; pt < 4; ++pt) ch_[pt] = cl_[pt] = float4v{0, 0, 0, 0};
#pragma unroll
        for (int ch = 0; ch < 8; ++ch) {
            if (ch >= nch) break;
#pragma unroll
            for (int pt = 0; pt < 4; ++pt) {
                const half8 av = *reinterpret_cast<const half8 *>(ks + (pt * 16 + lq) * kld + 8 * lg + ch * 32);
                ch_[pt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, qb[ch], ch_[pt], 0, 0, 0);
                cl_[pt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, ql[ch], cl_[pt], 0, 0, 0);
            }
        }
        float sc[4][4];
        float mx = -__builtin_inff();
#pragma unroll
        for (int pt = 0; pt < 4; ++pt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int slot = s0 + pt * 16 + 4 * lg + r;
                const bool ok = qvalid && slot < total && (slot < pos || ((vis >> (slot - pos)) & 1u));
                sc[pt][r] = ok ? (ch_[pt][r] + cl_[pt][r]) * scale : -__builtin_inff();
                mx = fmaxf(mx, sc[pt][r]);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        float lsum = 0.0f;
        half4 pe[4], pl[4];
#pragma unroll
        for (int pt = 0; pt < 4; ++pt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = sc[pt][r] == -__builtin_inff() ? 0.0f : expf(sc[pt][r] - mx);
                _Float16 eh, el;
                split_f16(e, eh, el);
                pe[pt][r] = eh;
                pl[pt][r] = el;
                lsum += e;
            }
        lsum += __shfl_xor(lsum, 16, 64);
        lsum += __shfl_xor(lsum, 32, 64);
        half8 pb[2], pbl[2];
#pragma unroll
        for (int kc = 0; kc < 2; ++kc)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                pb[kc][j] = pe[2 * kc][j];
                pb[kc][4 + j] = pe[2 * kc + 1][j];
                pbl[kc][j] = pl[2 * kc][j];
                pbl[kc][4 + j] = pl[2 * kc + 1][j];
            }
        dstamp(a, layer, 4);
        const uint32_t dst = static_cast<uint32_t>(((tq * nh + hq) * a.nb_max + b) * (hd + 2));
        for (int dt0 = 0; dt0 < hd / 16; dt0 += 4) {
            float4v oh[4], ol[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) oh[k] = ol[k] = float4v{0, 0, 0, 0};
#pragma unroll
            for (int kc = 0; kc < 2; ++kc)
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const _Float16 *vrow = vs + ((dt0 + k) * 16 + lq) * kAttnVld;
                    const half4 lo4 = *reinterpret_cast<const half4 *>(vrow + kc * 32 + 4 * lg);
                    const half4 hi4 = *reinterpret_cast<const half4 *>(vrow + kc * 32 + 16 + 4 * lg);
                    const half8 av = {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
                    oh[k] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, pb[kc], oh[k], 0, 0, 0);
                    ol[k] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, pbl[kc], ol[k], 0, 0, 0);
                }
            if (qvalid)
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float4v c = oh[k] + ol[k];
                    ast4f(a, fo(a.o_parts, dst + (dt0 + k) * 16 + 4 * lg), make_float4(c[0], c[1], c[2], c[3]));
                }
        }
        if (qvalid && lg == 0) {
            astf(a, fo(a.o_parts, dst + hd), mx);
            astf(a, fo(a.o_parts, dst + hd + 1), lsum);
        }
    }
    dstamp(a, layer, 5);
    __syncthreads();   // the staged block is read before the next item restages it
}

__device__ __forceinline__ unsigned ph_attn(const StepDev &a, int l, unsigned gen, Lds s) {
    const LayerDev &L = a.layers[l];
    const int total = a.sp->pos + a.sp->M;
    const int nitems = (total + kAttnBlock - 1) / kAttnBlock * a.nkv;
    AttnPre pre;
    const int first = static_cast<int>(blockIdx.x) - 1, stride = static_cast<int>(gridDim.x) - 1;   // not workgroup 0
    if (first >= 0 && first < nitems) attn_prefetch(a, L, first, total, pre);
    wait(a, gen, s.abort);
    dstamp(a, l, 0);
    for (int it = first; first >= 0 && it < nitems; it += stride) {
        if (it != first) attn_prefetch(a, L, it, total, pre);
        attn_item(a, L, it, pre, s.scratch, l);
    }
    arrive(a, gen + 1);
    return gen + 1;
}

// The blocks of (row t, head h) joined and gated (attn_merge_kernel's arithmetic, model.cpp:3830-3855), the row's
// operands for the output projection written for the head's dims
__device__ __forceinline__ void merge_item(const StepDev &a, int t, int h, uint8_t *scratch) {
    float *fw = reinterpret_cast<float *>(scratch);        // [1024]
    float *red = fw + 1024;                                // [2][4]
    float4 *osum = reinterpret_cast<float4 *>(red + 16);   // [4][64]
    const int hd = a.hd, nh = a.nh;
    const int nbw = (a.sp->pos + a.sp->M + kAttnBlock - 1) / kAttnBlock;   // <= 1024
    const int ld = hd + 2;
    const uint32_t base = static_cast<uint32_t>(((t * nh + h) * a.nb_max) * ld);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // the blocks' maxima and sums, up to four blocks a thread, loaded at once
    float mb[4], sb[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int b = threadIdx.x + q * 256;
        mb[q] = b < nbw ? aldf(a, fo(a.o_parts, base + b * ld + hd)) : -__builtin_inff();
        sb[q] = b < nbw ? aldf(a, fo(a.o_parts, base + b * ld + hd + 1)) : 0.0f;
    }
    float mx = fmaxf(fmaxf(mb[0], mb[1]), fmaxf(mb[2], mb[3]));
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float lsum = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int b = threadIdx.x + q * 256;
        if (b < nbw) {
            const float f = mb[q] == -__builtin_inff() ? 0.0f : expf(__fsub_rn(mb[q], mx));
            fw[b] = f;
            lsum = __builtin_fmaf(sb[q], f, lsum);
        }
    }
    lsum = static_cast<float>(wave_sum(static_cast<double>(lsum)));
    if (lane == 0) red[4 + wave] = lsum;
    __syncthreads();
    const float inv = __fdiv_rn(1.0f, ((red[4] + red[5]) + red[6]) + red[7]);
    // wave w adds the blocks w, w + 4, ... in that order (attn_merge_kernel's order), 48 blocks' loads at a time
    float4 o = make_float4(0, 0, 0, 0);
    if (lane * 4 < hd) {
        for (int b0 = wave; b0 < nbw; b0 += 4 * 48) {
            float4 v[48];
#pragma unroll
            for (int u = 0; u < 48; ++u) {
                const int b = b0 + 4 * u;
                v[u] = b < nbw ? ald4f(a, fo(a.o_parts, base + b * ld + lane * 4)) : make_float4(0, 0, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < 48; ++u) {
                const int b = b0 + 4 * u;
                if (b < nbw) {
                    const float f = fw[b];
                    o.x = __builtin_fmaf(v[u].x, f, o.x);
                    o.y = __builtin_fmaf(v[u].y, f, o.y);
                    o.z = __builtin_fmaf(v[u].z, f, o.z);
                    o.w = __builtin_fmaf(v[u].w, f, o.w);
                }
            }
        }
    }
    osum[wave * 64 + lane] = o;
    __syncthreads();
    if (wave == 0) {
        const int g = lane, ng = hd / 8;
        const bool live = g < ng;
        float v[8];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int li = live ? 2 * g + hh : 0;
            float4 s4 = osum[li];
#pragma unroll
            for (int w = 1; w < 4; ++w) {
                const float4 q = osum[w * 64 + li];
                s4.x += q.x, s4.y += q.y, s4.z += q.z, s4.w += q.w;
            }
            const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = 8 * g + 4 * hh + i;
                const float gate = live ? aldf(a, fo(a.o_qkv, t * a.qkv_rows + h * 2 * hd + hd + d)) : 0.0f;
                const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-gate)));
                v[4 * hh + i] = __fmul_rn(__fmul_rn(sv[i], inv), sig);
            }
        }
        act16_group(v, h * ng + g, live, XDst{a.arena, a.arena_bytes, a.o_act_core + static_cast<uint32_t>(t * act_halves(static_cast<int64_t>(nh) * hd) * 2)});
    }
    __syncthreads();
}

__device__ __forceinline__ unsigned ph_merge(const StepDev &a, unsigned gen, Lds s) {
    wait(a, gen, s.abort);
    const int M = a.sp->M;
    for (int it = blockIdx.x; it < M * a.nh; it += gridDim.x) merge_item(a, it / a.nh, it % a.nh, s.scratch);
    arrive(a, gen + 1);
    return gen + 1;
}

// x += o act_core (the residual add; passes of R ranges applied in order, gemv_q4's accumulate)
template <int NS, int NTT, int RP, int R>
__device__ __forceinline__ unsigned ph_o(const StepDev &a, int l, unsigned gen, Lds s) {
    const LayerDev &L = a.layers[l];
    const int M = a.sp->M, H = a.H, nsc = a.nh * a.hd / kSuperK;
    const float go = L.g_o;
    int u0, u1;
    my_units(H / kTileR, u0, u1);
    const uint8_t *wc = L.o_c, *ws = L.o_s;
    auto addr = [=, &a](int k, const uint8_t *&cb, const uint8_t *&sb) {
        const int64_t blk = static_cast<int64_t>(u0 + k / RP) * nsc + (k % RP) * NS;
        cb = wc + blk * 1024;
        sb = ws + blk * 128;
    };
    Prod<NS, NTT, ring_for<NS, RP>(), RP> p;
    p.setup(u1 - u0);
    p.prefetch(addr);
    wait(a, gen, s.abort);
    const int64_t abC = act_halves(static_cast<int64_t>(a.nh) * a.hd);
    auto bops = [=, &a](int k, h8(&bh)[NS * 4][NTT], h8(&bl)[NS * 4][NTT]) {
        bops_act<NS, NTT>(a, a.o_act_core, abC, M, k % RP, Ident(), bh, bl);
    };
    auto fin = [=, &a](int unit, int tt, int ll, const f4 *pp, int stride, bool live) {
        const int j = tt * 16 + ll % 16;
        const int row = (u0 + unit) * kTileR + 4 * (ll / 16);
        const bool ok = live && j < M;
        const uint32_t xo = fo(a.o_x, j * H + row);
        const float4 xv = ald4f_if(a, ok, xo);
        float xa[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int ps = 0; ps < RP / R; ++ps) {
            const f4 sum = pass_sum<R>(pp, stride, ps * R);
#pragma unroll
            for (int i = 0; i < 4; ++i) xa[i] = xa[i] + sum[i] * go;
        }
        ast4f_if(a, ok, xo, make_float4(xa[0], xa[1], xa[2], xa[3]));
    };
    if (RP <= 4) p.template run<false>(addr, bops, fin, reinterpret_cast<f4 *>(s.scratch), s.tab);
    else p.template run<true>(addr, bops, fin, reinterpret_cast<f4 *>(s.scratch), s.tab);
    arrive(a, gen + 1);
    return gen + 1;
}

// The router (router_kernel's arithmetic): the post-attention RMSNorm of every row in every workgroup that needs it
// (for its router rows, and in workgroup b for row b's operands of the experts' products), the router rows
// blockIdx + i G (wave i) in eight partial sums in the reference's fixed order (bf16_row_dots, kernels.cpp:1446-1483)
__device__ __forceinline__ unsigned ph_router(const StepDev &a, int l, unsigned gen, Lds s) {
    const LayerDev &L = a.layers[l];
    const int H = a.H, E1 = a.E + 1, M = a.sp->M;
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    // workgroup w >= 1 (not the barrier's gatherer) takes the router rows (w - 1) + i (G - 1) (wave i) and writes
    // row w - 1's operands
    const int wgi = static_cast<int>(blockIdx.x) - 1, G1 = static_cast<int>(gridDim.x) - 1;
    const int ra = wgi < 0 ? E1 : wgi + wave * G1;
    const bool busy = wgi >= 0 && (wgi < E1 || wgi < M);
    // the wave's router row, 8 bf16 a load (H <= 4096: up to 8 loads a lane), loaded before the barrier ends
    uint4 wr[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int c8 = lane + k * 64;
        wr[k] = ra < E1 && c8 < H / 8 ? *reinterpret_cast<const uint4 *>(L.router + static_cast<int64_t>(ra) * H + c8 * 8)
                                      : make_uint4(0, 0, 0, 0);
    }
    float nw[2][8];   // 1 + w of the post-attention norm, groups threadIdx + q 256
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int g = threadIdx.x + q * 256;
        const bool ld = g < H / 8;
        const float4 wa = ld ? *reinterpret_cast<const float4 *>(L.post_norm + g * 8) : make_float4(0, 0, 0, 0);
        const float4 wb = ld ? *reinterpret_cast<const float4 *>(L.post_norm + g * 8 + 4) : make_float4(0, 0, 0, 0);
        const float t8[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) nw[q][i] = __fadd_rn(1.0f, t8[i]);
    }
    wait(a, gen, s.abort);
    if (busy) {
        constexpr int TG = 8;
        const int ldh = H + 8;
        float *hs = reinterpret_cast<float *>(s.scratch);       // [TG][ldh] the normalized rows
        float *ws = hs + TG * ldh;                               // [4][H] the router rows as fp32
        double *red = reinterpret_cast<double *>(ws + 4 * H);   // [4][TG]
        if (ra < E1) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int c8 = lane + k * 64;
                if (c8 < H / 8) {
                    const uint32_t u[4] = {wr[k].x, wr[k].y, wr[k].z, wr[k].w};
                    float *d = ws + wave * H + c8 * 8;
#pragma unroll
                    for (int hh = 0; hh < 4; ++hh) {
                        d[2 * hh] = __uint_as_float(u[hh] << 16);
                        d[2 * hh + 1] = __uint_as_float(u[hh] & 0xFFFF0000u);
                    }
                }
            }
        }
        for (int t0 = 0; t0 < M; t0 += TG) {
            const int nt = min(TG, M - t0);
            float xv[TG][2][8];
#pragma unroll
            for (int tt = 0; tt < TG; ++tt)
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    float4 p = make_float4(0, 0, 0, 0), r = p;
                    const int g = threadIdx.x + q * 256;
                    if (tt < nt && g < H / 8) {
                        p = ald4f(a, fo(a.o_x, (t0 + tt) * H + g * 8));
                        r = ald4f(a, fo(a.o_x, (t0 + tt) * H + g * 8 + 4));
                    }
                    const float t8[8] = {p.x, p.y, p.z, p.w, r.x, r.y, r.z, r.w};
#pragma unroll
                    for (int i = 0; i < 8; ++i) xv[tt][q][i] = t8[i];
                }
            __syncthreads();   // the previous group's sums are done with hs and red
#pragma unroll
            for (int tt = 0; tt < TG; ++tt) {
                double ss = 0.0;
#pragma unroll
                for (int q = 0; q < 2; ++q)
#pragma unroll
                    for (int i = 0; i < 8; ++i) ss += static_cast<double>(xv[tt][q][i]) * static_cast<double>(xv[tt][q][i]);
                ss = wave_sum(ss);
                if (lane == 0) red[wave * TG + tt] = ss;
            }
            __syncthreads();
            const int tq = wgi - t0;
#pragma unroll
            for (int tt = 0; tt < TG; ++tt) {
                if (tt < nt) {   // uniform
                    const double tot = ((red[tt] + red[TG + tt]) + red[2 * TG + tt]) + red[3 * TG + tt];
                    const float inv =
                        __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(static_cast<float>(tot / static_cast<double>(H)), a.eps)));
#pragma unroll
                    for (int q = 0; q < 2; ++q) {
                        if (q * 256 < H / 8) {   // uniform
                            float v[8];
#pragma unroll
                            for (int i = 0; i < 8; ++i) v[i] = __fmul_rn(__fmul_rn(xv[tt][q][i], inv), nw[q][i]);
                            const int g = threadIdx.x + q * 256;
                            const bool live = g < H / 8;
                            if (live) {
                                *reinterpret_cast<float4 *>(hs + tt * ldh + g * 8) = make_float4(v[0], v[1], v[2], v[3]);
                                *reinterpret_cast<float4 *>(hs + tt * ldh + g * 8 + 4) = make_float4(v[4], v[5], v[6], v[7]);
                            }
                            if (tt == tq) act16_group(v, g, live, XDst{a.arena, a.arena_bytes, a.o_act_h + static_cast<uint32_t>(wgi * act_halves(H) * 2)});
                        }
                    }
                }
            }
            __syncthreads();
            if (ra >= E1) continue;
            const int tt = lane / 8, j = lane % 8;
            const float *hr = hs + (tt < nt ? tt : 0) * ldh;
            const float *wrow = ws + wave * H;
            float a0 = 0.0f;
            for (int c0 = j; c0 < H; c0 += 8 * 16) {
                float hv[16], wv[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    hv[u] = hr[c0 + 8 * u];
                    wv[u] = wrow[c0 + 8 * u];
                }
#pragma unroll
                for (int u = 0; u < 16; ++u) a0 = __fadd_rn(a0, __fmul_rn(wv[u], hv[u]));
            }
            const float s1 = __fadd_rn(a0, __shfl_down(a0, 4, 64));
            const float s2 = __fadd_rn(s1, __shfl_down(s1, 1, 64));
            const float s3 = __fadd_rn(s2, __shfl_down(s2, 2, 64));
            astf(a, j == 0 && tt < nt ? fo(a.o_rlog, (t0 + tt) * E1 + ra) : kNoStore, s3);
        }
    }
    arrive(a, gen + 1);
    return gen + 1;
}

// The route of every row (route_all: each workgroup the same bits, into its LDS), then the experts' gate|up
// products: a unit is (slot, tile pair p): the gate rows 16 p .. 16 p + 15 and their up rows, whose SwiGLU
// (swiglu_quant_kernel: silu(g) u, kernels.hpp:141) is one 16-value block of the down products' operands
template <int NS, int NTT, int RH>
__device__ __forceinline__ unsigned ph_up(const StepDev &a, int l, unsigned gen, Lds s) {
    const LayerDev &L = a.layers[l];
    const int M = a.sp->M, H = a.H, F = a.F, E1 = a.E + 1, K = a.K;
    wait(a, gen, s.abort);
    dstamp(a, l, 10);
    {
        float *lg = reinterpret_cast<float *>(s.scratch + 64 * 1024);   // [M][E1] the logits
        const int nl = M * E1;
        {   // the layer's expert globals (E1 <= 257: up to 4 a thread) and the logits, all loads in flight at once
            float eg[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int i = threadIdx.x + q * 256;
                eg[q] = i < E1 * 3 ? L.eglob[i] : 0.0f;
            }
            for (int i0 = 0; i0 < nl; i0 += 8 * 256) {
                float v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int i = i0 + threadIdx.x + u * 256;
                    v[u] = i < nl ? aldf(a, fo(a.o_rlog, i)) : 0.0f;
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int i = i0 + threadIdx.x + u * 256;
                    if (i < nl) lg[i] = v[u];
                }
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int i = threadIdx.x + q * 256;
                if (i < E1 * 3) s.eg[i] = eg[q];
            }
        }
        __syncthreads();
        int *ids = reinterpret_cast<int *>(s.scratch);
        int *cnt = ids + kMaxRows * 16, *start = cnt + 260, *slot_of = start + 260;
        unsigned *rows = reinterpret_cast<unsigned *>(slot_of + 260);
        int(*wtot)[16] = reinterpret_cast<int(*)[16]>(rows + 260);
        int *ids_dummy = reinterpret_cast<int *>(wtot + 2);
        int32_t *ids_out = blockIdx.x == 0 ? a.route_ids + static_cast<int64_t>(l) * a.max_rows * K : ids_dummy;
        dstamp(a, l, 11);
        route_all(lg, a.E, K, M, s.rs, ids_out, RouteLds{ids, cnt, start, slot_of, rows, wtot});
        __syncthreads();
        dstamp(a, l, 12);
        if (blockIdx.x == 0) {   // a copy for the per-phase kernels (read after this launch)
            const uint32_t *src = reinterpret_cast<const uint32_t *>(s.rs);
            uint32_t *dst = reinterpret_cast<uint32_t *>(a.route + l);
            for (int i = threadIdx.x; i < static_cast<int>(sizeof(RouteState) / 4); i += blockDim.x) dst[i] = src[i];
        }
    }
    const RouteState *rs = s.rs;
    constexpr int RU = 2 * RH;   // a unit: the gate tile's RH ranges, then the up tile's
    const int npair = F / kTileR, nsc = H / kSuperK;
    int u0, u1;
    const bool one_slot = slot_units(rs->n_slots, npair, u0, u1);
    const uint8_t *gc = L.gu_c, *gs = L.gu_s;
    auto addr = [=, &a](int k, const uint8_t *&cb, const uint8_t *&sb) {
        const int u = u0 + k / RU, rr = k % RU;
        const int slot = u / npair, pr = u % npair;
        const int e = rs->slot_expert[slot];
        const int64_t tile = rr < RH ? pr : pr + npair;
        const int64_t blk = tile * nsc + (rr % RH) * NS;
        cb = gc + static_cast<size_t>(e) * a.gu_cs + blk * 1024;
        sb = gs + static_cast<size_t>(e) * a.gu_ss + blk * 128;
    };
    Prod<NS, NTT, ring_for<NS, RU>(), RU> p;
    p.setup(u1 - u0);
    p.prefetch(addr);
    dstamp(a, l, 13);
    auto bops = [=, &a](int k, h8(&bh)[NS * 4][NTT], h8(&bl)[NS * 4][NTT]) {
        const int slot = (u0 + k / RU) / npair;
        const int st = rs->slot_start[slot];
        bops_act<NS, NTT>(a, a.o_act_h, act_halves(H), rs->slot_count[slot], (k % RU) % RH,
                          [=](int j) { return rs->pick_token[st + j]; }, bh, bl);
    };
    auto fin = [=, &a](int unit, int tt, int ll, const f4 *pp, int stride, bool live) {
        const int u = u0 + unit;
        const int slot = u / npair, pr = u % npair;
        const int e = rs->slot_expert[slot], st = rs->slot_start[slot], cnt = rs->slot_count[slot];
        const f4 gsum = pass_sum<RH>(pp, stride, 0), usum = pass_sum<RH>(pp, stride, RH);
        const float g0 = s.eg[e * 3], g1 = s.eg[e * 3 + 1];
        float m4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float gv = gsum[i] * g0, uv = usum[i] * g1;
            m4[i] = __fmul_rn(__fdiv_rn(gv, __fadd_rn(1.0f, expf(-gv))), uv);
        }
        // the lane has values 16 pr + 4 lg + i of pick j; a k-group of 8 is lanes lg = 2 c, 2 c + 1
        const int lgq = ll / 16;
        float oth[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) oth[i] = __shfl_xor(m4[i], 16, 64);
        float v[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = (lgq & 1) ? oth[i] : m4[i];
            v[4 + i] = (lgq & 1) ? m4[i] : oth[i];
        }
        float am = amax8(v);
        am = fmaxf(am, __shfl_xor(am, 32, 64));
        const int j = tt * 16 + ll % 16;
        const bool ok = live && (lgq & 1) == 0 && j < cnt;
        h8 hi, lo;
        act16_operands(v, am, hi, lo);
        const uint32_t off = a.o_act_m + static_cast<uint32_t>(((st + j) * act_halves(F) + (2 * pr + lgq / 2) * 16) * 2);
        ast16(a, ok ? off : kNoStore, __builtin_bit_cast(xu4, hi));
        ast16(a, ok ? off + 16 : kNoStore, __builtin_bit_cast(xu4, lo));
    };
    if (one_slot && RH <= 4) p.template run<false>(addr, bops, fin, reinterpret_cast<f4 *>(s.scratch), s.tab);
    else p.template run<true>(addr, bops, fin, reinterpret_cast<f4 *>(s.scratch), s.tab);
    dstamp(a, l, 14);
    arrive(a, gen + 1);
    return gen + 1;
}

// y[pick] = down m[pick]: units (slot, tile), the slots from the workgroup's route (LDS), weights loaded before the
// barrier ends
template <int NS, int NTT, int RP>
__device__ __forceinline__ unsigned ph_down(const StepDev &a, int l, unsigned gen, Lds s) {
    const LayerDev &L = a.layers[l];
    const int H = a.H, F = a.F, nsc = F / kSuperK, htiles = H / kTileR;
    const RouteState *rs = s.rs;
    int u0, u1;
    const bool one_slot = slot_units(rs->n_slots, htiles, u0, u1);
    const uint8_t *dc = L.dn_c, *ds = L.dn_s;
    auto addr = [=, &a](int k, const uint8_t *&cb, const uint8_t *&sb) {
        const int u = u0 + k / RP;
        const int slot = u / htiles;
        const int64_t tile = u % htiles;
        const int e = rs->slot_expert[slot];
        const int64_t blk = tile * nsc + (k % RP) * NS;
        cb = dc + static_cast<size_t>(e) * a.dn_cs + blk * 1024;
        sb = ds + static_cast<size_t>(e) * a.dn_ss + blk * 128;
    };
    Prod<NS, NTT, ring_for<NS, RP>(), RP> p;
    p.setup(u1 - u0);
    p.prefetch(addr);
    wait(a, gen, s.abort);
    dstamp(a, l, 20);
    auto bops = [=, &a](int k, h8(&bh)[NS * 4][NTT], h8(&bl)[NS * 4][NTT]) {
        const int slot = (u0 + k / RP) / htiles;
        const int st = rs->slot_start[slot];
        bops_act<NS, NTT>(a, a.o_act_m, act_halves(F), rs->slot_count[slot], k % RP, [=](int j) { return st + j; }, bh, bl);
    };
    auto fin = [=, &a](int unit, int tt, int ll, const f4 *pp, int stride, bool live) {
        const int u = u0 + unit;
        const int slot = u / htiles, tile = u % htiles;
        const int e = rs->slot_expert[slot], st = rs->slot_start[slot], cnt = rs->slot_count[slot];
        const f4 sum = pass_sum<RP>(pp, stride, 0);
        const int j = tt * 16 + ll % 16;
        const float g2 = s.eg[e * 3 + 2];
        const int row = tile * kTileR + 4 * (ll / 16);
        ast4f_if(a, live && j < cnt, fo(a.o_y, (st + j) * H + row),
                 make_float4(sum[0] * g2, sum[1] * g2, sum[2] * g2, sum[3] * g2));
    };
    if (one_slot && RP <= 4) p.template run<false>(addr, bops, fin, reinterpret_cast<f4 *>(s.scratch), s.tab);
    else p.template run<true>(addr, bops, fin, reinterpret_cast<f4 *>(s.scratch), s.tab);
    dstamp(a, l, 21);
    arrive(a, gen + 1);
    return gen + 1;
}

// x += sigmoid(gate) shared + sum_k w_k y_k in rank order, then the next layer's input RMSNorm (after the last: the
// final norm) and the products' operands (combine_kernel's arithmetic, model.cpp:4554-4585, :5363-5365); workgroup
// t takes row t
__device__ __forceinline__ unsigned ph_combine(const StepDev &a, int l, unsigned gen, Lds s) {
    wait(a, gen, s.abort);
    const RouteState *rs = s.rs;
    const int t = blockIdx.x, H = a.H, K = a.K;
    if (t < a.sp->M) {
        const int ng = H / 8;
        const float gs = rs->gate[t];
        const uint32_t ysh = fo(a.o_y, rs->pick_of[t * (K + 1) + K] * H);
        float v[4][8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int g = threadIdx.x + q * blockDim.x;
#pragma unroll
            for (int i = 0; i < 8; ++i) v[q][i] = 0.0f;
            if (g >= ng) continue;
            // every load first (the shared expert's row, the K <= 16 picks' rows, the residual), then the sums in
            // rank order
            const uint32_t xo = fo(a.o_x, t * H + g * 8);
            const float4 sa = ald4f(a, ysh + g * 32), sb4 = ald4f(a, ysh + g * 32 + 16);
            const float4 p = ald4f(a, xo), r = ald4f(a, xo + 16);
            float4 ya[16], yb[16];
            float wk[16];
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                wk[k] = k < K ? rs->weight[t * K + k] : 0.0f;
                const uint32_t yo = fo(a.o_y, rs->pick_of[t * (K + 1) + (k < K ? k : 0)] * H + g * 8);
                ya[k] = ald4f(a, k < K ? yo : kNoStore);
                yb[k] = ald4f(a, k < K ? yo + 16 : kNoStore);
            }
            float o[8];
            {
                const float yv[8] = {sa.x, sa.y, sa.z, sa.w, sb4.x, sb4.y, sb4.z, sb4.w};
#pragma unroll
                for (int i = 0; i < 8; ++i) o[i] = __fmul_rn(gs, yv[i]);
            }
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                if (k >= K || wk[k] == 0.0f) continue;
                const float yv[8] = {ya[k].x, ya[k].y, ya[k].z, ya[k].w, yb[k].x, yb[k].y, yb[k].z, yb[k].w};
#pragma unroll
                for (int i = 0; i < 8; ++i) o[i] = __fadd_rn(o[i], __fmul_rn(wk[k], yv[i]));
            }
            const float xv[8] = {p.x, p.y, p.z, p.w, r.x, r.y, r.z, r.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) v[q][i] = __fadd_rn(xv[i], o[i]);
            ast4f(a, xo, make_float4(v[q][0], v[q][1], v[q][2], v[q][3]));
            ast4f(a, xo + 16, make_float4(v[q][4], v[q][5], v[q][6], v[q][7]));
        }
        const float *next_norm = l + 1 < a.n_layers ? a.layers[l + 1].in_norm : a.final_norm;
        norm_quant_regs(v, H, next_norm, a.eps, XDst{a.arena, a.arena_bytes, a.o_act_h + static_cast<uint32_t>(t * act_halves(H) * 2)}, nullptr, s.red);
    }
    arrive(a, gen + 1);
    return gen + 1;
}

// the final norm's operands came with the last combine: logits = lm_head act_h
template <int NS, int NTT, int RP>
__device__ __forceinline__ void ph_lm(const StepDev &a, unsigned gen, Lds s) {
    const int M = a.sp->M, H = a.H, nsc = H / kSuperK, V = a.V;
    const float glm = a.lm_g;
    int u0, u1;
    my_units(static_cast<int>(tiles_rows(V)), u0, u1);
    const uint8_t *wc = a.lm_c, *ws = a.lm_s;
    auto addr = [=, &a](int k, const uint8_t *&cb, const uint8_t *&sb) {
        const int64_t blk = static_cast<int64_t>(u0 + k / RP) * nsc + (k % RP) * NS;
        cb = wc + blk * 1024;
        sb = ws + blk * 128;
    };
    Prod<NS, NTT, ring_for<NS, RP>(), RP> p;
    p.setup(u1 - u0);
    p.prefetch(addr);
    wait(a, gen, s.abort);
    auto bops = [=, &a](int k, h8(&bh)[NS * 4][NTT], h8(&bl)[NS * 4][NTT]) {
        bops_act<NS, NTT>(a, a.o_act_h, act_halves(H), M, k % RP, Ident(), bh, bl);
    };
    auto fin = [=, &a](int unit, int tt, int ll, const f4 *pp, int stride, bool live) {
        const int j = tt * 16 + ll % 16;
        const int row = (u0 + unit) * kTileR + 4 * (ll / 16);
        const f4 sum = pass_sum<RP>(pp, stride, 0);
        const bool ok = live && j < M;
        const uint32_t o = fo(a.o_logits, static_cast<int64_t>(j) * V + row);
        // whole float4s inside the vocabulary; a last partial one element by element
        ast4f_if(a, ok && row + 3 < V, o, make_float4(sum[0] * glm, sum[1] * glm, sum[2] * glm, sum[3] * glm));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const bool one = ok && row + 3 >= V && row + i < V;
            astf(a, one ? o + i * 4u : kNoStore, sum[i] * glm);
        }
    };
    if (RP <= 4) p.template run<false>(addr, bops, fin, reinterpret_cast<f4 *>(s.scratch), s.tab);
    else p.template run<true>(addr, bops, fin, reinterpret_cast<f4 *>(s.scratch), s.tab);
}

// ---------------------------------------------------------------- the kernel
template <int NTT, int NSH, int NSO, int NSF, int RPH, int RPO, int RO, int RPF>
__global__ __launch_bounds__(256) void step_kernel(const StepDev *__restrict__ ap, unsigned gen0) {
    extern __shared__ uint4 lds4[];
    const StepDev &a = *ap;
    Lds s(reinterpret_cast<uint8_t *>(lds4));
    if (threadIdx.x == 0) *s.abort = 0;
    fill_e4m3_table(s.tab);
    __syncthreads();
    unsigned gen = gen0 + 1;
    ph_embed(a, s);
    arrive(a, gen);
    for (int l = 0; l < a.n_layers; ++l) {
        gen = ph_qkv<NSH, NTT, RPH>(a, l, gen, s);
        gen = ph_attn(a, l, gen, s);
        gen = ph_merge(a, gen, s);
        gen = ph_o<NSO, NTT, RPO, RO>(a, l, gen, s);
        gen = ph_router(a, l, gen, s);
        gen = ph_up<NSH, NTT, RPH>(a, l, gen, s);
        gen = ph_down<NSF, NTT, RPF>(a, l, gen, s);
        gen = ph_combine(a, l, gen, s);
    }
    ph_lm<NSH, NTT, RPH>(a, gen, s);
}

// the LDS the kernel takes: the fixed part plus the largest phase's scratch
size_t step_lds(const Model &m) {
    const auto &c = m.c;
    const size_t hd = c.head_dim, H = c.hidden;
    const size_t attn = attn_lds(c.head_dim) + 4 * 256 * 4 + 4 * 2 * 16 * hd * 2;
    const size_t router = (8 * (H + 8) + 4 * H) * 4 + 4 * 8 * 8;
    const size_t route = 64 * 1024 + static_cast<size_t>(kMaxRows) * (c.n_experts + 1) * 4;
    const size_t prod = 2 * 16 * 2 * 1024;   // batches of up to 16 tasks, two token tiles, double-buffered
    const size_t merge = (1024 + 16) * 4 + 4 * 64 * 16;
    return kLdsScratch + std::max({attn, router, route, prod, merge});
}

// (NS, R, P) of a product of K values at the row count's token tiles, as gemv_q4 (one_pass: moe_run) splits it
bool prod_shape(int64_t K, int ntt, bool one_pass, ProdShape &sh) {
    const int64_t nsc = K / kSuperK;
    const int64_t lim = ntt == 1 ? 32 : 16;
    const int64_t n = one_pass ? nsc : std::min(nsc, lim);
    int waves = 0, kw = 0;
    if (n < 1 || nsc % n != 0 || !mfma_split(n * kSuperK, ntt, waves, kw)) return false;
    sh.NS = kw / 4;
    sh.R = waves;
    sh.P = static_cast<int>(nsc / n);
    return sh.R == 1 || sh.R == 2 || sh.R == 4 || sh.R == 8;
}

template <int NTT, int NSH, int NSO, int NSF, int RPH, int RPO, int RO, int RPF>
const void *kernel_ptr() {
    return reinterpret_cast<const void *>(&step_kernel<NTT, NSH, NSO, NSF, RPH, RPO, RO, RPF>);
}

// the instantiations: the configs' shapes (H = 2048, nh hd = 4096, F = 512) and the tests' small model (H = 256,
// nh hd = 256, F = 128); the product shapes must match one exactly
struct StepInst {
    int ntt;
    ProdShape h, o, f;
    const void *(*ptr)();
};
const StepInst kInsts[] = {
    {1, {4, 4, 1}, {4, 8, 1}, {2, 2, 1}, &kernel_ptr<1, 4, 4, 2, 4, 8, 8, 2>},
    {2, {2, 8, 1}, {2, 8, 2}, {2, 2, 1}, &kernel_ptr<2, 2, 2, 2, 8, 16, 8, 2>},
    {1, {1, 2, 1}, {1, 2, 1}, {1, 1, 1}, &kernel_ptr<1, 1, 1, 1, 2, 2, 2, 1>},
    {2, {1, 2, 1}, {1, 2, 1}, {1, 1, 1}, &kernel_ptr<2, 1, 1, 1, 2, 2, 2, 1>},
};

bool same(const ProdShape &x, const ProdShape &y) { return x.NS == y.NS && x.R == y.R && x.P == y.P; }

const void *pick_kernel(int ntt, const ProdShape &h, const ProdShape &o, const ProdShape &f, int &slot) {
    slot = -1;
    for (int i = 0; i < static_cast<int>(sizeof(kInsts) / sizeof(kInsts[0])); ++i)
        if (kInsts[i].ntt == ntt && same(kInsts[i].h, h) && same(kInsts[i].o, o) && same(kInsts[i].f, f)) {
            slot = i;
            return kInsts[i].ptr();
        }
    return nullptr;
}

bool shapes_for(const Model &m, int M, ProdShape &h, ProdShape &o, ProdShape &f) {
    const auto &c = m.c;
    const int ntt = M <= 16 ? 1 : 2;
    // the dense products split K per launch; the experts' take K whole (moe_run): theirs must be one pass, and the
    // gate|up products (K = H) must split as the dense K = H ones do
    if (!prod_shape(c.hidden, ntt, false, h) || !prod_shape(static_cast<int64_t>(c.n_heads) * c.head_dim, ntt, false, o) ||
        !prod_shape(c.moe_ff, ntt, true, f))
        return false;
    ProdShape hu;
    return prod_shape(c.hidden, ntt, true, hu) && hu.NS == h.NS && hu.R == h.R && h.P == 1 && f.P == 1;
}

}  // namespace

bool step_supported(const Model &m, int M, const char **why) {
    const auto &c = m.c;
    auto no = [&](const char *w) {
        if (why) *why = w;
        return false;
    };
    ProdShape h, o, f;
    int slot;
    if (M < 1 || M > kMaxRows) return no("rows");
    if (!shapes_for(m, M, h, o, f)) return no("product shapes outside the step kernel's splits");
    if (!pick_kernel(M <= 16 ? 1 : 2, h, o, f, slot)) return no("no step kernel instantiated for these product shapes");
    if (c.head_dim > 256 || c.hidden > 4096 || c.rope_dim > 64) return no("hidden, head_dim or rope_dim");
    if (c.n_experts > 256) return no("experts");
    if (step_lds(m) > 160 * 1024) return no("LDS");
    return true;
}

int step_setup(Model &m) {
    if (m.step_dev) return 0;
    const auto &c = m.c;
    int dev = 0, cus = 0;
    GV_CHECK_HIP(hipGetDevice(&dev));
    GV_CHECK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    GV_REQUIRE(cus >= 8, "step kernel: too few compute units");
    std::vector<LayerDev> ld(static_cast<size_t>(c.n_layers));
    for (int l = 0; l < c.n_layers; ++l) {
        const LayerW &L = m.layers[static_cast<size_t>(l)];
        LayerDev &d = ld[static_cast<size_t>(l)];
        d.qkv_c = L.qkv.codes, d.qkv_s = L.qkv.scales, d.o_c = L.o.codes, d.o_s = L.o.scales;
        d.g_q = L.g_q, d.g_k = L.g_k, d.g_v = L.g_v, d.g_o = L.o.global;
        d.in_norm = L.in_norm, d.post_norm = L.post_norm, d.q_norm = L.q_norm, d.k_norm = L.k_norm;
        d.router = L.router;
        d.gu_c = L.gu_codes, d.gu_s = L.gu_scales, d.dn_c = L.dn_codes, d.dn_s = L.dn_scales;
        d.eglob = L.expert_globals;
        d.kv = L.kv;
    }
    void *p = nullptr;
    GV_CHECK_HIP(hipMalloc(&p, ld.size() * sizeof(LayerDev)));
    m.allocs.push_back(p);
    GV_CHECK_HIP(hipMemcpy(p, ld.data(), ld.size() * sizeof(LayerDev), hipMemcpyHostToDevice));
    m.layers_dev = p;
    if (!m.bar) {
        GV_CHECK_HIP(hipMalloc(&p, 64 * 1024));
        m.allocs.push_back(p);
        GV_CHECK_HIP(hipMemset(p, 0, 64 * 1024));
        m.bar = static_cast<unsigned *>(p);
        m.step_err = m.bar + 16 * 1024 - 64;
        m.bar_gen = 0;
    }
    // the step's arguments for 1..16 and 17..32 rows
    StepDev sd[2];
    for (int i = 0; i < 2; ++i) {
        StepDev &a = sd[i];
        a = StepDev{};
        a.layers = static_cast<const LayerDev *>(m.layers_dev);
        a.n_layers = c.n_layers, a.H = c.hidden, a.V = c.vocab, a.E = c.n_experts, a.K = c.top_k, a.F = c.moe_ff;
        a.nh = c.n_heads, a.nkv = c.n_kv_heads, a.hd = c.head_dim, a.half = c.rope_dim / 2, a.max_rows = c.max_rows;
        a.eps = c.eps;
        a.slots = m.slots;
        a.nb_max = m.kv_blocks;
        a.qkv_rows = static_cast<int>(m.layers[0].qkv.rows);
        a.gu_cs = m.gu_code_stride, a.gu_ss = m.gu_scale_stride, a.dn_cs = m.dn_code_stride, a.dn_ss = m.dn_scale_stride;
        a.emb_c = m.embed.codes, a.emb_s = m.embed.scales, a.emb_g = m.embed.global;
        a.lm_c = m.lm_head.codes, a.lm_s = m.lm_head.scales, a.lm_g = m.lm_head.global;
        a.final_norm = m.final_norm, a.rope_cos = m.rope_cos, a.rope_sin = m.rope_sin;
        a.sp = m.sp;
        auto off = [&](const void *p) { return static_cast<uint32_t>(static_cast<const uint8_t *>(p) - m.arena); };
        a.arena = m.arena;
        a.arena_bytes = static_cast<uint32_t>(m.arena_bytes);
        a.o_x = off(m.x), a.o_qkv = off(m.qkv_out), a.o_rlog = off(m.rlogits), a.o_parts = off(m.parts);
        a.o_y = off(m.y), a.o_logits = off(m.logits), a.o_act_h = off(m.act_h), a.o_act_core = off(m.act_core);
        a.o_act_m = off(m.act_m);
        a.route_ids = m.route_ids;
        a.route = m.route;
        a.flags = m.bar, a.rel = m.bar + 8192, a.err = m.step_err;
        a.stamps = m.stamps;
        ProdShape h{}, o{}, f{};
        if (shapes_for(m, i == 0 ? 16 : 32, h, o, f)) a.sh_h = h, a.sh_o = o, a.sh_f = f;
    }
    GV_CHECK_HIP(hipMalloc(&p, sizeof sd));
    m.allocs.push_back(p);
    GV_CHECK_HIP(hipMemcpy(p, sd, sizeof sd, hipMemcpyHostToDevice));
    m.step_dev = p;
    m.step_grid = cus;
    return 0;
}

// the globals of the weights are copied into the step's arguments: rebuild them after an adoption
int step_invalidate(Model &m) {
    if (!m.step_dev) return 0;
    GV_CHECK_HIP(hipStreamSynchronize(stream()));
    auto drop = [&](void *&p) {
        if (!p) return;
        (void)hipFree(p);
        m.allocs.erase(std::remove(m.allocs.begin(), m.allocs.end(), p), m.allocs.end());
        p = nullptr;
    };
    drop(m.layers_dev);
    drop(m.step_dev);
    return 0;
}

int step_run(Model &m, int M, hipStream_t st) {
    if (step_setup(m) != 0) return -1;
    const auto &c = m.c;
    ProdShape h, o, f;
    GV_REQUIRE(M >= 1 && M <= c.max_rows && shapes_for(m, M, h, o, f), "step kernel: product shapes");
    const int ntt = M <= 16 ? 1 : 2;
    int slot = -1;
    const void *kern = pick_kernel(ntt, h, o, f, slot);
    GV_REQUIRE(kern, "step kernel: no instantiation for these shapes");
    const size_t lds = step_lds(m);
    static int granted[4] = {0, 0, 0, 0};
    if (lds_grant(kern, lds, granted[slot]) != 0) return -1;
    const unsigned need = step_barriers(c.n_layers);
    if (m.bar_gen > 0xF0000000u - need) {   // restart the generations before they wrap
        GV_CHECK_HIP(hipStreamSynchronize(st));
        GV_CHECK_HIP(hipMemset(m.bar, 0, 16 * 1024 * 4 - 256));
        m.bar_gen = 0;
    }
    const StepDev *ad = static_cast<const StepDev *>(m.step_dev) + (ntt - 1);
    unsigned gen0 = m.bar_gen;
    void *args[] = {&ad, &gen0};
    GV_CHECK_HIP(hipLaunchCooperativeKernel(kern, dim3(m.step_grid), dim3(256), args, static_cast<unsigned>(lds), st));
    m.bar_gen += need;
    return 0;
}

int step_trace(Model &m, bool on) {
    if (step_invalidate(m) != 0) return -1;
    if (m.stamps) {
        (void)hipFree(m.stamps);
        m.allocs.erase(std::remove(m.allocs.begin(), m.allocs.end(), static_cast<void *>(m.stamps)), m.allocs.end());
        m.stamps = nullptr;
    }
    if (!on) return 0;
    int dev = 0, cus = 0;
    GV_CHECK_HIP(hipGetDevice(&dev));
    GV_CHECK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    const size_t n = static_cast<size_t>(cus) * (step_barriers(m.c.n_layers) * 2 + 32);
    void *p = nullptr;
    GV_CHECK_HIP(hipMalloc(&p, n * 8));
    GV_CHECK_HIP(hipMemset(p, 0, n * 8));
    m.allocs.push_back(p);
    m.stamps = static_cast<uint64_t *>(p);
    return 0;
}

int64_t step_trace_read(Model &m, uint64_t *out, int64_t n) {
    if (!m.stamps || !out) return 0;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return -1;
    const int64_t have = static_cast<int64_t>(cus) * (step_barriers(m.c.n_layers) * 2 + 32);
    const int64_t k = std::min(n, have);
    if (hipStreamSynchronize(stream()) != hipSuccess || hipMemcpy(out, m.stamps, static_cast<size_t>(k) * 8, hipMemcpyDeviceToHost) != hipSuccess)
        return -1;
    return k;
}

int step_check(Model &m) {
    if (!m.step_err) return 0;
    unsigned e = 0;
    GV_CHECK_HIP(hipMemcpy(&e, m.step_err, 4, hipMemcpyDeviceToHost));
    if (e != 0) {
        (void)hipMemset(m.step_err, 0, 4);
        set_error("step kernel: a grid barrier timed out (a workgroup never arrived); the step's results are invalid");
        return -1;
    }
    return 0;
}

}  // namespace gv
