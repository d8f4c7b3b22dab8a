// capi.hip - the C ABI of libgeode_verify.so (include/geode_verify.h): run time, the q4 format, products, and the
// NPU plugin's calls (npu/host/npu_api.h) served by this GPU.
#include <algorithm>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/geode_verify.h"
#include "common.hpp"
#include "kernels.hpp"

namespace gv {

// The workspace of gv_ffn_swiglu_noalloc: a file-scope device array, one copy on each GPU the library runs on, held
// until the process ends. Host code never passes `scratch` itself (on the host it is only a stand-in for the symbol):
// gv_init looks up the array's device address once per device (hipGetSymbolAddress) and every use goes through that.
constexpr size_t kNoAllocScratchBytes = size_t{4} << 20;   // 4 MiB: C1's shape (2048 -> 6144 -> 2048) up to 32 rows
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

struct Runtime {
    int device = -1;
    hipStream_t stream = nullptr;
    int act_exact = 0;   // the products' operands now in every source file's g_act_exact
    std::vector<hipEvent_t> events;
    void *scratch_dev[kMaxDevices] = {};   // scratch's device address on each device (set by gv_init)
};

Runtime &rt() {
    static Runtime r;
    return r;
}

hipStream_t stream() { return rt().stream; }

// Every source file's copy of the operands' mode to `exact`, when it differs: the device idle before (no kernel may
// read a copy while it changes) and after
int use_act_mode(int exact) {
    exact = exact ? 1 : 0;
    if (rt().act_exact == exact) return 0;
    GV_CHECK_HIP(hipStreamSynchronize(stream()));
    GV_CHECK_HIP(hipDeviceSynchronize());
    if (act_mode_set_model(exact) != 0 || act_mode_set_q4(exact) != 0 || act_mode_set_gdn(exact) != 0 ||
        act_mode_set_mtp(exact) != 0 || act_mode_set_prefill(exact) != 0)
        return -1;
    GV_CHECK_HIP(hipDeviceSynchronize());
    rt().act_exact = exact;
    return 0;
}

int ensure_init() {
    if (rt().stream) return 0;
    return gv_init(0);
}

Q4 to_q4(const gv_q4 &w) {
    Q4 q;
    q.codes = w.codes;
    q.scales = w.scales;
    q.rows = w.rows;
    q.cols = w.cols;
    q.S = w.lanes;
    q.steps = w.steps;
    q.global = w.global;
    return q;
}

gv_q4 from_q4(const Q4 &q) {
    gv_q4 w;
    w.codes = q.codes;
    w.scales = q.scales;
    w.rows = q.rows;
    w.cols = q.cols;
    w.lanes = q.S;
    w.steps = q.steps;
    w.global = q.global;
    return w;
}

// device scratch that grows (one host thread drives the library)
struct Scratch {
    void *p = nullptr;
    size_t n = 0;
    void *get(size_t want) {
        if (want <= n) return p;
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
        if (hipMalloc(&p, want) != hipSuccess) return nullptr;
        n = want;
        return p;
    }
    ~Scratch() {
        if (p) (void)hipFree(p);
    }
};

int ffn_swiglu_ws(const gv_q4 *gate, const gv_q4 *up, const gv_q4 *down, int M, const uint16_t *x_f16, float *y,
                  void *ws);

}  // namespace gv

using namespace gv;

extern "C" {

const char *gv_last_error(void) { return last_error(); }

int gv_init(int device) {
    Runtime &r = rt();
    if (r.stream && r.device == device) return 0;
    int n = 0;
    GV_CHECK_HIP(hipGetDeviceCount(&n));
    GV_REQUIRE(device >= 0 && device < n && device < kMaxDevices, "gv_init: no such device");
    GV_CHECK_HIP(hipSetDevice(device));
    if (!r.scratch_dev[device]) {   // this device's copy of the no-alloc entry point's scratch
        void *p = nullptr;
        GV_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        GV_REQUIRE(p, "gv_init: no device address for the scratch array");
        r.scratch_dev[device] = p;
    }
    if (r.stream) GV_CHECK_HIP(hipStreamDestroy(r.stream));
    GV_CHECK_HIP(hipStreamCreateWithFlags(&r.stream, hipStreamNonBlocking));
    r.device = device;
    return q4_init_constants();
}

int gv_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

void *gv_malloc(size_t bytes) {
    if (ensure_init() != 0) return nullptr;
    void *p = nullptr;
    const hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) {
        set_error(std::string("gv_malloc: ") + hipGetErrorString(e));
        return nullptr;
    }
    return p;
}

int gv_free(void *p) {
    if (!p) return 0;
    GV_CHECK_HIP(hipFree(p));
    return 0;
}

int gv_memcpy_h2d(void *dst, const void *src, size_t bytes) {
    if (ensure_init() != 0) return -1;
    GV_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream()));
    GV_CHECK_HIP(hipStreamSynchronize(stream()));
    return 0;
}

int gv_memcpy_d2h(void *dst, const void *src, size_t bytes) {
    if (ensure_init() != 0) return -1;
    GV_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, stream()));
    GV_CHECK_HIP(hipStreamSynchronize(stream()));
    return 0;
}

int gv_memcpy_d2d(void *dst, const void *src, size_t bytes) {
    if (ensure_init() != 0) return -1;
    if (bytes % 16 == 0 && reinterpret_cast<uintptr_t>(dst) % 16 == 0 && reinterpret_cast<uintptr_t>(src) % 16 == 0)
        return copy16(src, static_cast<int64_t>(bytes / 16), dst, stream());   // a vector copy kernel
    GV_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, stream()));
    return 0;
}

int gv_memset(void *dst, int value, size_t bytes) {
    if (ensure_init() != 0) return -1;
    GV_CHECK_HIP(hipMemsetAsync(dst, value, bytes, stream()));
    return 0;
}

int gv_synchronize(void) {
    if (ensure_init() != 0) return -1;
    GV_CHECK_HIP(hipStreamSynchronize(stream()));
    return 0;
}

int gv_event_record(void) {
    if (ensure_init() != 0) return -1;
    hipEvent_t e;
    GV_CHECK_HIP(hipEventCreate(&e));
    GV_CHECK_HIP(hipEventRecord(e, stream()));
    rt().events.push_back(e);
    return static_cast<int>(rt().events.size()) - 1;
}

float gv_event_elapsed_ms(int start, int stop) {
    auto &ev = rt().events;
    if (start < 0 || stop < 0 || start >= static_cast<int>(ev.size()) || stop >= static_cast<int>(ev.size())) {
        set_error("gv_event_elapsed_ms: no such event");
        return -1.0f;
    }
    if (hipEventSynchronize(ev[static_cast<size_t>(stop)]) != hipSuccess) return -1.0f;
    float ms = -1.0f;
    if (hipEventElapsedTime(&ms, ev[static_cast<size_t>(start)], ev[static_cast<size_t>(stop)]) != hipSuccess)
        return -1.0f;
    return ms;
}

size_t gv_q4_device_bytes(int64_t rows, int64_t cols) {
    return q4_code_bytes(rows, cols) + q4_scale_bytes(rows, cols);
}

int gv_q4_from_pack(const uint8_t *pack_dev, int64_t rows, int64_t cols, float global, void *dst, gv_q4 *out) {
    if (ensure_init() != 0) return -1;
    GV_REQUIRE(pack_dev && dst && out, "gv_q4_from_pack: null pointer");
    uint8_t *codes = static_cast<uint8_t *>(dst);
    uint8_t *scales = codes + q4_code_bytes(rows, cols);
    Q4 q;
    if (q4_from_pack(pack_dev, rows, cols, global, codes, scales, q, stream()) != 0) return -1;
    *out = from_q4(q);
    return 0;
}

int gv_q4_dequant(const gv_q4 *w, float *out) {
    if (ensure_init() != 0) return -1;
    GV_REQUIRE(w && out, "gv_q4_dequant: null pointer");
    return q4_dequant(to_q4(*w), out, stream());
}

int gv_q4_pack(const float *w_dev, int64_t rows, int64_t cols, uint8_t *pack_out_dev, float *global_out_dev) {
    if (ensure_init() != 0) return -1;
    static Scratch s;
    auto *u = static_cast<unsigned int *>(s.get(256));
    GV_REQUIRE(u, "gv_q4_pack: scratch");
    return q4_pack(w_dev, rows, cols, u, pack_out_dev, global_out_dev, stream());
}

size_t gv_act_bytes(int64_t cols) { return act_bytes(cols); }

int gv_quantize(const float *x, int64_t ldx, int M, int cols, const float *norm_w, float eps, uint8_t *act,
                float *h_out) {
    if (ensure_init() != 0 || use_act_mode(0) != 0) return -1;
    return quantize_act(x, ldx, M, cols, norm_w, eps, reinterpret_cast<_Float16 *>(act), act_halves(cols), h_out, cols,
                        stream());
}

int gv_gemv_q4(const gv_q4 *w, const uint8_t *act, int M, float *y, int64_t ldy, int accumulate) {
    if (ensure_init() != 0) return -1;
    GV_REQUIRE(w && act && y, "gv_gemv_q4: null pointer");
    return gemv_q4(to_q4(*w), reinterpret_cast<const _Float16 *>(act), act_halves(w->cols), M,
                   gemv_out(y, ldy, w->global, accumulate), stream());
}

size_t gv_ffn_workspace_bytes(int64_t hidden, int64_t ff, int M) {
    const size_t a = act_bytes(std::max(hidden, ff)) * static_cast<size_t>(M);
    return (static_cast<size_t>(M) * hidden + 3 * static_cast<size_t>(M) * ff) * sizeof(float) + a + 256;
}

int gv_ffn_swiglu(const gv_q4 *gate, const gv_q4 *up, const gv_q4 *down, int M, const uint16_t *x_f16, float *y,
                  void *ws) {
    if (ensure_init() != 0 || use_act_mode(0) != 0) return -1;
    return ffn_swiglu_ws(gate, up, down, M, x_f16, y, ws);
}

int gv_ffn_swiglu_noalloc(const gv_q4 *gate, const gv_q4 *up, const gv_q4 *down, int M, const uint16_t *x_f16,
                          float *y) {
    if (ensure_init() != 0 || use_act_mode(0) != 0) return -1;
    GV_REQUIRE(gate && up && down, "gv_ffn_swiglu_noalloc: null pointer");
    GV_REQUIRE(M >= 1 && M <= kMaxRows, "gv_ffn_swiglu_noalloc: 1 <= M <= 32");
    const size_t need = gv_ffn_workspace_bytes(gate->cols, gate->rows, M);
    GV_REQUIRE(need <= kNoAllocScratchBytes,
               "gv_ffn_swiglu_noalloc: this shape needs " + std::to_string(need) +
                   " bytes of workspace, more than the 4 MiB scratch holds (use gv_ffn_swiglu)");
    void *ws = rt().scratch_dev[rt().device];
    GV_REQUIRE(ws, "gv_ffn_swiglu_noalloc: no scratch address for this device");
    return ffn_swiglu_ws(gate, up, down, M, x_f16, y, ws);
}

}  // extern "C"

namespace gv {
// The C1 products on a caller's workspace ws (gv_ffn_workspace_bytes of it): every piece of it is written before it
// is read (x, the gate and up products, m, the operands), so nothing is cleared between calls.
int ffn_swiglu_ws(const gv_q4 *gate, const gv_q4 *up, const gv_q4 *down, int M, const uint16_t *x_f16, float *y,
                  void *ws) {
    GV_REQUIRE(gate && up && down && x_f16 && y && ws, "gv_ffn_swiglu: null pointer");
    const int64_t H = gate->cols, F = gate->rows;
    GV_REQUIRE(up->rows == F && up->cols == H && down->rows == H && down->cols == F, "gv_ffn_swiglu: shapes");
    GV_REQUIRE(M >= 1 && M <= kMaxRows, "gv_ffn_swiglu: 1 <= M <= 32");
    float *x = static_cast<float *>(ws);
    float *g = x + static_cast<size_t>(M) * H;
    float *u = g + static_cast<size_t>(M) * F;
    float *m = u + static_cast<size_t>(M) * F;
    _Float16 *act = reinterpret_cast<_Float16 *>(m + static_cast<size_t>(M) * F);
    hipStream_t st = stream();
    const int64_t ab_h = act_halves(H), ab_f = act_halves(F);
    int waves = 0, kw = 0;
    if (M <= 8 && F % 16 == 0 && H <= 8192 && mfma_split(H, 1, waves, kw) && waves <= 4) {
        // three launches: x's operands (in x's place: M act rows of H fit its M x H floats), gate | up with the
        // SwiGLU and its quantization (act), down
        _Float16 *act_x = reinterpret_cast<_Float16 *>(x);
        if (quantize_f16(x_f16, M, static_cast<int>(H), act_x, ab_h, st) != 0) return -1;
        if (ffn_up(to_q4(*gate), to_q4(*up), act_x, ab_h, M, act, ab_f, st) != 0) return -1;
        return gemv_q4(to_q4(*down), act, ab_f, M, gemv_out(y, H, down->global), st);
    }
    if (f16_to_f32(x_f16, static_cast<int64_t>(M) * H, x, st) != 0) return -1;
    if (quantize_act(x, H, M, static_cast<int>(H), nullptr, 0.0f, act, ab_h, nullptr, 0, st) != 0) return -1;
    if (gemv_q4(to_q4(*gate), act, ab_h, M, gemv_out(g, F, gate->global), st) != 0) return -1;
    if (gemv_q4(to_q4(*up), act, ab_h, M, gemv_out(u, F, up->global), st) != 0) return -1;
    if (swiglu(g, u, static_cast<int64_t>(M) * F, m, st) != 0) return -1;
    if (quantize_act(m, F, M, static_cast<int>(F), nullptr, 0.0f, act, ab_f, nullptr, 0, st) != 0) return -1;
    return gemv_q4(to_q4(*down), act, ab_f, M, gemv_out(y, H, down->global), st);
}
}  // namespace gv

// ---------------------------------------------------------------- the NPU plugin's calls (npu/host/npu_api.h)
struct gv_ctx {
    struct Mat {
        void *buf = nullptr;
        Q4 q;
    };
    std::vector<Mat> mats;
    Scratch io, work;
    ~gv_ctx() {
        for (auto &m : mats)
            if (m.buf) (void)hipFree(m.buf);
    }
};

namespace {
void put_err(char *err, int err_len, const char *msg) {
    if (err && err_len > 0) {
        std::strncpy(err, msg, static_cast<size_t>(err_len) - 1);
        err[err_len - 1] = '\0';
    }
}
}  // namespace

extern "C" {

gv_ctx *gv_open(int device, char *err, int err_len) {
    if (gv_init(device) != 0) {
        put_err(err, err_len, last_error());
        return nullptr;
    }
    return new gv_ctx();
}

void gv_close(gv_ctx *g) { delete g; }

int gv_adopt_q4(gv_ctx *g, const uint8_t *data, int64_t rows, int64_t cols, size_t row_bytes, float global) {
    if (!g || !data || rows <= 0 || cols % 128 != 0 || row_bytes != static_cast<size_t>(cols / 16) * 9) {
        set_error("gv_adopt_q4: bad arguments (rows > 0, cols a multiple of 128, the pack's row bytes)");
        return -1;
    }
    const size_t pack = static_cast<size_t>(rows) * row_bytes;
    void *tmp = g->io.get(pack);
    void *buf = nullptr;
    if (!tmp || hipMalloc(&buf, gv_q4_device_bytes(rows, cols)) != hipSuccess) {
        set_error("gv_adopt_q4: out of device memory");
        return -1;
    }
    gv_ctx::Mat m;
    m.buf = buf;
    if (hipMemcpyAsync(tmp, data, pack, hipMemcpyHostToDevice, stream()) != hipSuccess ||
        q4_from_pack(static_cast<uint8_t *>(tmp), rows, cols, global, static_cast<uint8_t *>(buf),
                     static_cast<uint8_t *>(buf) + q4_code_bytes(rows, cols), m.q, stream()) != 0 ||
        hipStreamSynchronize(stream()) != hipSuccess) {
        (void)hipFree(buf);
        if (std::string(last_error()).empty()) set_error("gv_adopt_q4: copy failed");
        return -1;
    }
    g->mats.push_back(m);
    return static_cast<int>(g->mats.size()) - 1;
}

int gv_gemm(gv_ctx *g, int id, int n, const float *const *xs, float *const *ys) {
    GV_REQUIRE(g && id >= 0 && id < static_cast<int>(g->mats.size()) && n >= 0, "gv_gemm: bad arguments");
    if (use_act_mode(0) != 0) return -1;   // the plugin's products: the int8 path
    const Q4 &q = g->mats[static_cast<size_t>(id)].q;
    hipStream_t st = stream();
    for (int t0 = 0; t0 < n; t0 += kMaxRows) {
        const int m = std::min(kMaxRows, n - t0);
        const size_t xb = static_cast<size_t>(m) * q.cols * 4, yb = static_cast<size_t>(m) * q.rows * 4;
        auto *base = static_cast<uint8_t *>(g->io.get(xb + yb + static_cast<size_t>(m) * act_bytes(q.cols)));
        GV_REQUIRE(base, "gv_gemm: out of device memory");
        float *x = reinterpret_cast<float *>(base), *y = reinterpret_cast<float *>(base + xb);
        _Float16 *act = reinterpret_cast<_Float16 *>(base + xb + yb);
        for (int t = 0; t < m; ++t)
            GV_CHECK_HIP(hipMemcpyAsync(x + static_cast<size_t>(t) * q.cols, xs[t0 + t], q.cols * 4,
                                        hipMemcpyHostToDevice, st));
        if (quantize_act(x, q.cols, m, static_cast<int>(q.cols), nullptr, 0.0f, act, act_halves(q.cols), nullptr, 0,
                         st) != 0)
            return -1;
        if (gemv_q4(q, act, act_halves(q.cols), m, gemv_out(y, q.rows, q.global), st) != 0)
            return -1;
        for (int t = 0; t < m; ++t)
            GV_CHECK_HIP(hipMemcpyAsync(ys[t0 + t], y + static_cast<size_t>(t) * q.rows, q.rows * 4,
                                        hipMemcpyDeviceToHost, st));
        GV_CHECK_HIP(hipStreamSynchronize(st));
    }
    return 0;
}

int gv_mlp(gv_ctx *g, int gate, int up, int n_down, const int *downs, int act, int n, const float *const *xs,
           float *const *ys) {
    const int nm = g ? static_cast<int>(g->mats.size()) : 0;
    GV_REQUIRE(g && gate >= 0 && gate < nm && up >= 0 && up < nm && n_down >= 1 && downs && n >= 0,
               "gv_mlp: bad arguments");
    GV_REQUIRE(act == 1, "gv_mlp: only act 1 (silu) is supported");
    if (use_act_mode(0) != 0) return -1;
    const Q4 &qg = g->mats[static_cast<size_t>(gate)].q, &qu = g->mats[static_cast<size_t>(up)].q;
    GV_REQUIRE(qg.rows == qu.rows && qg.cols == qu.cols, "gv_mlp: gate and up differ");
    const int64_t H = qg.cols, F = qg.rows;
    int64_t dcols = 0, drows = -1;
    for (int j = 0; j < n_down; ++j) {
        GV_REQUIRE(downs[j] >= 0 && downs[j] < nm, "gv_mlp: bad down id");
        const Q4 &qd = g->mats[static_cast<size_t>(downs[j])].q;
        GV_REQUIRE(drows < 0 || qd.rows == drows, "gv_mlp: down parts differ in rows");
        drows = qd.rows;
        dcols += qd.cols;
    }
    GV_REQUIRE(dcols == F, "gv_mlp: the down parts' inputs must add up to the gate's rows");
    hipStream_t st = stream();
    for (int t0 = 0; t0 < n; t0 += kMaxRows) {
        const int m = std::min(kMaxRows, n - t0);
        const size_t need = (static_cast<size_t>(m) * (H + 3 * F + drows)) * 4 + static_cast<size_t>(m) * act_bytes(std::max(H, F));
        auto *base = static_cast<float *>(g->work.get(need));
        GV_REQUIRE(base, "gv_mlp: out of device memory");
        float *x = base, *gg = x + static_cast<size_t>(m) * H, *uu = gg + static_cast<size_t>(m) * F,
              *mm = uu + static_cast<size_t>(m) * F, *y = mm + static_cast<size_t>(m) * F;
        auto *a = reinterpret_cast<_Float16 *>(y + static_cast<size_t>(m) * drows);
        for (int t = 0; t < m; ++t)
            GV_CHECK_HIP(hipMemcpyAsync(x + static_cast<size_t>(t) * H, xs[t0 + t], H * 4, hipMemcpyHostToDevice, st));
        const int64_t abh = act_halves(H);
        if (quantize_act(x, H, m, static_cast<int>(H), nullptr, 0.0f, a, abh, nullptr, 0, st) != 0) return -1;
        if (gemv_q4(qg, a, abh, m, gemv_out(gg, F, qg.global), st) != 0) return -1;
        if (gemv_q4(qu, a, abh, m, gemv_out(uu, F, qu.global), st) != 0) return -1;
        if (swiglu(gg, uu, static_cast<int64_t>(m) * F, mm, st) != 0) return -1;
        int64_t c0 = 0;
        for (int j = 0; j < n_down; ++j) {   // each part's results added (npu_api.h:62-65)
            const Q4 &qd = g->mats[static_cast<size_t>(downs[j])].q;
            const int64_t ab = act_halves(qd.cols);
            if (quantize_act(mm + c0, F, m, static_cast<int>(qd.cols), nullptr, 0.0f, a, ab, nullptr, 0, st) != 0)
                return -1;
            if (gemv_q4(qd, a, ab, m, gemv_out(y, drows, qd.global, j > 0), st) != 0) return -1;
            c0 += qd.cols;
        }
        for (int t = 0; t < m; ++t)
            GV_CHECK_HIP(hipMemcpyAsync(ys[t0 + t], y + static_cast<size_t>(t) * drows, drows * 4,
                                        hipMemcpyDeviceToHost, st));
        GV_CHECK_HIP(hipStreamSynchronize(st));
    }
    return 0;
}

}  // extern "C"
