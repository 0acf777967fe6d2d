// api.cpp -- the C ABI (include/fish_w8a8.h): argument checks, scratch
// management and kernel dispatch.
//
// Dispatch for the linear layer (reference dispatcher: int8_gemm.cu:384-511):
//   16-byte aligned W and X_q, N <= 16 and a shape plan_gemv takes:
//       N == 1        -> v_dot4 GEMV, one wave per 1-2 weight rows (gemv.hip)
//       2 <= N <= 16  -> int8 MFMA GEMV, 16-row tiles (gemv.hip); fa_w8a8_gemm
//                        lets it quantize the fp16 tokens itself when the
//                        shape allows, and fa_w8a8_gemm_swiglu lets its
//                        epilogue form the SwiGLU pairs
//   aligned, K % 64 == 0, group % 64 == 0 -> LDS-tiled int8 MFMA GEMM (gemm.hip)
//   anything else -> the exact any-shape kernel (gemm.hip, generic)
// All paths sum the K-groups in the same order, so they agree bit for bit.
// The error convention mirrors CUDA_CHECK (src/utils/cuda_utils.h:10-17): a
// failing HIP call is reported with file/line and hipGetErrorString, here as
// a status code plus a per-thread message instead of an exception.
#include "common.h"
#include "chain.h"
#include "../../include/fish_w8a8.h"

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

#define FA_HIP(call)                                                                   \
    do {                                                                               \
        hipError_t e_ = (call);                                                        \
        if (e_ != hipSuccess)                                                          \
            return fail(FA_ERR_HIP, "HIP error at %s:%d: %s", __FILE__, __LINE__,      \
                        hipGetErrorString(e_));                                        \
    } while (0)

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }
// (the one-token kernels read smooth_inv 16 bytes at a time)
bool aligned16_or_null(const void* p) { return !p || aligned16(p); }

// Per-thread, per-device grow-only scratch (the reference keeps a thread_local
// workspace, int8_gemm.cu:31-44).
struct Workspace {
    int8_t* xq = nullptr;
    size_t xq_bytes = 0;
    float* xs = nullptr;
    size_t xs_bytes = 0;
    float* st = nullptr;        // group-major scale tables of the pipelined GEMM
    size_t st_bytes = 0;
    uint16_t* yt = nullptr;     // fp16 [N, 2F] of the SwiGLU entry's separate-launch path
    size_t yt_bytes = 0;
    int* sk = nullptr;          // prefill K split: kSplitCounters zeroed ints, then partials
    size_t sk_bytes = 0;
};

constexpr size_t kSplitCounters = 16384;   // tiles a split launch may have

thread_local std::unordered_map<int, Workspace> g_ws;

int current_ws(Workspace** out) {
    int dev = 0;
    FA_HIP(hipGetDevice(&dev));
    *out = &g_ws[dev];
    return FA_OK;
}

int grow(void** p, size_t* have, size_t need, hipStream_t stream) {
    if (*have >= need) return FA_OK;
    need = (need + 255) & ~(size_t)255;
    if (*p) {
        FA_HIP(hipStreamSynchronize(stream));
        FA_HIP(hipFree(*p));
        *p = nullptr;
        *have = 0;
    }
    FA_HIP(hipMalloc(p, need));
    *have = need;
    return FA_OK;
}

int eff_group(int K, int g) { return (g <= 0 || g > K) ? K : g; }

// tables: device memory of gemm_pipe_tables_bytes(M, N, G) for the prefill
// kernels' scale tables, or nullptr to use (and grow) this thread's scratch.
int linear_quantized(const char* fn, const int8_t* W, const uint16_t* w_scale, int g, int G,
                     const int8_t* xq, const float* xs, uint16_t* Y, int32_t* dbg, int row0,
                     int rows, int tok0, int toks, int M, int N, int K, hipStream_t stream,
                     float* tables = nullptr) {
    const bool aligned = aligned16(W) && aligned16(xq);
    if (aligned && N <= 16) {
        fa::GemvPlan p = fa::plan_gemv(M, N, K, g, G, false);
        if (p.kind != 0) {
            FA_HIP(fa::launch_gemv(p, W, w_scale, xq, xs, nullptr, nullptr, nullptr, Y, dbg, row0,
                                   rows, tok0, toks, M, N, K, g, G, stream));
            return FA_OK;
        }
    }
    const bool tile = aligned && fa::gemm_tile_ok(M, N, K, g);
    if (tile || (aligned && fa::gemm_pipe_ok(M, N, K, g))) {
        const bool own_tables = tables == nullptr;
        if (!tables) {
            Workspace* ws = nullptr;
            int rc = current_ws(&ws);
            if (rc) return rc;
            void* p = ws->st;
            rc = grow(&p, &ws->st_bytes, fa::gemm_pipe_tables_bytes(M, N, G), stream);
            ws->st = (float*)p;
            if (rc) return rc;
            tables = ws->st;
        }
        if (tile) {
            // K split for few-tile grids, on the thread's scratch only (the
            // no-alloc entry runs unsplit)
            const int variant = fa::gemm_tile_choice(M, N, K, g);
            int nsplit = own_tables ? fa::gemm_tile_split(M, N, K, g, variant) : 1;
            float* part = nullptr;
            int* cnt = nullptr;
            if (nsplit > 1) {
                Workspace* ws = nullptr;
                int rc = current_ws(&ws);
                if (rc) return rc;
                const size_t need = kSplitCounters * sizeof(int) +
                                    fa::gemm_tile_split_bytes(M, N, variant, nsplit);
                if (ws->sk_bytes < need) {
                    void* p = ws->sk;
                    rc = grow(&p, &ws->sk_bytes, need, stream);
                    ws->sk = (int*)p;
                    if (rc) return rc;
                    // counters start at zero; every launch leaves them so
                    FA_HIP(hipMemsetAsync(ws->sk, 0, kSplitCounters * sizeof(int), stream));
                }
                cnt = ws->sk;
                part = reinterpret_cast<float*>(ws->sk + kSplitCounters);
            }
            FA_HIP(fa::launch_gemm_tile(W, w_scale, xq, xs, tables, Y, dbg, row0, rows, tok0, toks,
                                        M, N, K, g, G, stream, variant, -1, nsplit, part, cnt));
        }
        else
            FA_HIP(fa::launch_gemm_pipe(W, w_scale, xq, xs, tables, Y, dbg, row0, rows, tok0, toks,
                                        M, N, K, g, G, stream));
        return FA_OK;
    }
    if (aligned && K % 64 == 0 && g % 64 == 0) {
        FA_HIP(fa::launch_gemm(W, w_scale, xq, xs, Y, dbg, row0, rows, tok0, toks, M, N, K, g, G,
                               stream));
        return FA_OK;
    }
    if (N > 65535) return fail(FA_ERR_INVALID_ARG, "%s: N=%d too large for the generic path", fn, N);
    FA_HIP(fa::launch_gemm_generic(W, w_scale, xq, xs, Y, dbg, row0, rows, tok0, toks, M, N, K, g,
                                   G, stream));
    return FA_OK;
}

int check_dims(const char* fn, int M, int N, int K) {
    if (M < 0 || N < 0) return fail(FA_ERR_INVALID_ARG, "%s: negative M=%d or N=%d", fn, M, N);
    if (K <= 0) return fail(FA_ERR_INVALID_ARG, "%s: K=%d must be positive", fn, K);
    return FA_OK;
}

// [a, a + n) and [b, b + m) overlap (fp16 element counts)
bool overlaps(const uint16_t* a, size_t n, const uint16_t* b, size_t m) {
    return a && b && a < b + m && b < a + n;
}

// ---------------------------------------------------- per-shape timing ----
//
// The reference's FISH_INT8_PROFILE (src/kernels/int8_gemm.cu:45-145,
// 398-510): with the variable set to a non-empty value other than "0" (or
// after fa_profile_enable(1)), each call of the linear entry points is timed
// with events on its stream, waited for, and added to a bucket keyed by
// entry, shape, group size and quantization mode; the buckets are printed
// to stderr at exit and can be read with fa_profile_summary.  Calls on a
// stream under graph capture are not timed (waiting is not allowed there),
// and an entry point called from another one is timed once, as the outer
// call.

struct ProfBucket {
    uint64_t calls = 0;
    uint64_t groups = 0;
    double total_ms = 0.0, quant_ms = 0.0, linear_ms = 0.0;
};

struct ProfState {
    std::mutex mu;
    std::map<std::string, ProfBucket> buckets;
    std::string summary() {
        std::lock_guard<std::mutex> lock(mu);
        if (buckets.empty()) return std::string();
        std::string out = "INT8 profile summary:\n";
        char line[512];
        for (const auto& kv : buckets) {
            const ProfBucket& b = kv.second;
            const double c = b.calls ? (double)b.calls : 1.0;
            snprintf(line, sizeof line,
                     "  %s calls=%llu avg_groups=%.1f total=%.3fms avg=%.3fms "
                     "(quant=%.3f gemm=%.3f)\n",
                     kv.first.c_str(), (unsigned long long)b.calls, (double)b.groups / c,
                     b.total_ms, b.total_ms / c, b.quant_ms / c, b.linear_ms / c);
            out += line;
        }
        return out;
    }
    ~ProfState() {   // host data only: no device call at exit
        const std::string t = summary();
        if (!t.empty()) fputs(t.c_str(), stderr);
    }
};

ProfState& prof_state() {
    static ProfState state;
    return state;
}

std::atomic<int> g_prof_on{-1};   // -1: not yet read from the environment

bool prof_enabled() {
    int v = g_prof_on.load(std::memory_order_relaxed);
    if (v < 0) {
        const char* e = std::getenv("FISH_INT8_PROFILE");
        v = (e && *e && std::string(e) != "0") ? 1 : 0;
        int expect = -1;
        g_prof_on.compare_exchange_strong(expect, v);
        v = g_prof_on.load(std::memory_order_relaxed);
    }
    return v > 0;
}

struct ProfEvents {
    hipEvent_t e[3] = {nullptr, nullptr, nullptr};
};
thread_local std::unordered_map<int, ProfEvents> t_prof_ev;   // per device
thread_local int t_prof_depth = 0;

class ProfCall;
thread_local ProfCall* t_prof = nullptr;

class ProfCall {
  public:
    explicit ProfCall(void* stream) : s_((hipStream_t)stream) {
        if (t_prof_depth++ > 0 || !prof_enabled()) return;
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(s_, &st) != hipSuccess || st != hipStreamCaptureStatusNone) return;
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) return;
        ProfEvents& pe = t_prof_ev[dev];
        for (auto& e : pe.e)
            if (!e && hipEventCreate(&e) != hipSuccess) return;
        if (hipEventRecord(pe.e[0], s_) != hipSuccess) return;
        ev_ = &pe;
        t_prof = this;
    }
    ~ProfCall() {
        --t_prof_depth;
        if (t_prof == this) t_prof = nullptr;
    }
    ProfCall(const ProfCall&) = delete;
    ProfCall& operator=(const ProfCall&) = delete;
    // end of the quantization phase (a separate launch before the linear)
    void mark() {
        if (ev_ && !marked_ && hipEventRecord(ev_->e[1], s_) == hipSuccess) marked_ = true;
    }
    void finish(const char* entry, int M, int N, int K, int group_size, bool static_act,
                bool smooth) {
        if (!ev_) return;
        float total = 0.0f, quant = 0.0f;
        if (hipEventRecord(ev_->e[2], s_) != hipSuccess || hipEventSynchronize(ev_->e[2]) != hipSuccess ||
            hipEventElapsedTime(&total, ev_->e[0], ev_->e[2]) != hipSuccess)
            return;
        if (marked_ && hipEventElapsedTime(&quant, ev_->e[0], ev_->e[1]) != hipSuccess) quant = 0.0f;
        const int g = eff_group(K, group_size);
        char key[256];
        snprintf(key, sizeof key, "%s M=%d N=%d K=%d group=%d act=%s smooth=%s", entry, M, N, K, g,
                 static_act ? "static" : "dynamic", smooth ? "yes" : "no");
        ProfState& ps = prof_state();
        std::lock_guard<std::mutex> lock(ps.mu);
        ProfBucket& b = ps.buckets[key];
        b.calls += 1;
        b.groups += (uint64_t)((K + g - 1) / g);
        b.total_ms += total;
        b.quant_ms += quant;
        b.linear_ms += total - quant;
    }

  private:
    hipStream_t s_;
    ProfEvents* ev_ = nullptr;
    bool marked_ = false;
};

// Called by an entry point between its quantization launch and its linear.
void prof_mark() {
    if (t_prof) t_prof->mark();
}

}  // namespace

namespace fa {
void set_last_error(const std::string& msg) { g_err = msg; }
}  // namespace fa

extern "C" {

const char* fa_last_error(void) { return g_err.c_str(); }

const char* fa_version(void) { return "fish-w8a8-mi355x 0.1.0 (gfx950)"; }

int fa_w8a8_gemm_quantized(const int8_t* W, const uint16_t* w_scale, int group_size,
                           const int8_t* X_q, const float* X_scale, uint16_t* Y, int M, int N,
                           int K, void* stream) {
    const char* fn = "fa_w8a8_gemm_quantized";
    g_err.clear();
    int rc = check_dims(fn, M, N, K);
    if (rc) return rc;
    if (M == 0 || N == 0) return FA_OK;
    if (!W || !w_scale || !X_q || !X_scale || !Y)
        return fail(FA_ERR_INVALID_ARG, "%s: null pointer argument", fn);
    const int g = eff_group(K, group_size);
    const int G = (K + g - 1) / g;
    return linear_quantized(fn, W, w_scale, g, G, X_q, X_scale, Y, nullptr, 0, 0, 0, 0, M, N, K,
                            (hipStream_t)stream);
}

int fa_w8a8_set_k_split(int max_splits) { return fa::set_k_split(max_splits); }

int fa_debug_gemv_plan_rejects(void) { return fa::gemv_plan_rejects(); }

int fa_w8a8_gemm_k_splits(int M, int N, int K, int group_size) {
    g_err.clear();
    if (M <= 0 || N <= 16 || K <= 0) return 1;
    const int g = eff_group(K, group_size);
    if (!fa::gemm_tile_ok(M, N, K, g)) return 1;
    return fa::gemm_tile_split(M, N, K, g, fa::gemm_tile_choice(M, N, K, g));
}

int fa_debug_gemv_plan(int M, int N, int K, int group_size, int qx, int pro, int epi,
                       int smooth, int* out) {
    g_err.clear();
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    const int g = eff_group(K, group_size);
    const int G = (K + g - 1) / g;
    const fa::GemvPlan p = fa::plan_gemv_raw(M, N, K, g, G, qx != 0, pro, epi, smooth != 0);
    if (out) {
        out[0] = p.kind; out[1] = p.grid; out[2] = p.block; out[3] = (int)p.lds;
        out[4] = p.spg; out[5] = p.maxg; out[6] = p.lc ? 1 : 0; out[7] = p.qx; out[8] = p.epi;
        out[9] = p.kind ? (fa::gemv_plan_valid(p, M, N, K, g, G) ? 1 : 0) : 0;
    }
    return p.kind;
}

int fa_w8a8_gemm_partials(const int8_t* W, const uint16_t* w_scale, int group_size,
                          const int8_t* X_q, const float* X_scale, uint16_t* Y, int32_t* partials,
                          int row0, int rows, int tok0, int toks, int M, int N, int K,
                          void* stream) {
    const char* fn = "fa_w8a8_gemm_partials";
    g_err.clear();
    int rc = check_dims(fn, M, N, K);
    if (rc) return rc;
    if (M == 0 || N == 0) return FA_OK;
    if (!W || !w_scale || !X_q || !X_scale || !Y || !partials)
        return fail(FA_ERR_INVALID_ARG, "%s: null pointer argument", fn);
    if (row0 < 0 || rows <= 0 || row0 + rows > M || tok0 < 0 || toks <= 0 || tok0 + toks > N)
        return fail(FA_ERR_INVALID_ARG, "%s: window rows [%d,+%d) toks [%d,+%d) outside M=%d N=%d",
                    fn, row0, rows, tok0, toks, M, N);
    const int g = eff_group(K, group_size);
    const int G = (K + g - 1) / g;
    return linear_quantized(fn, W, w_scale, g, G, X_q, X_scale, Y, partials, row0, rows, tok0,
                            toks, M, N, K, (hipStream_t)stream);
}

static int gemm_impl(const int8_t* W, const uint16_t* w_scale, int group_size,
                 const uint16_t* act_scale, const uint16_t* smooth_inv, const uint16_t* X,
                 uint16_t* Y, int M, int N, int K, void* stream) {
    const char* fn = "fa_w8a8_gemm";
    g_err.clear();
    int rc = check_dims(fn, M, N, K);
    if (rc) return rc;
    if (M == 0 || N == 0) return FA_OK;
    if (!W || !w_scale || !X || !Y) return fail(FA_ERR_INVALID_ARG, "%s: null pointer argument", fn);
    if (overlaps(Y, (size_t)N * M, X, (size_t)N * K))
        return fail(FA_ERR_INVALID_ARG, "%s: Y overlaps X", fn);
    hipStream_t s = (hipStream_t)stream;
    const int g = eff_group(K, group_size);
    const int G = (K + g - 1) / g;
    if (N == 1 && aligned16_or_null(smooth_inv) && aligned16(W) && aligned16(X)) {
        // decode: the GEMV quantizes the token itself (one launch, no scratch)
        fa::GemvPlan gp = fa::plan_gemv(M, N, K, g, G, true);
        if (gp.kind == 1 || gp.kind == 2) {
            FA_HIP(fa::launch_gemv(gp, W, w_scale, nullptr, nullptr, X, act_scale, smooth_inv, Y,
                                   nullptr, 0, 0, 0, 0, M, N, K, g, G, s));
            return FA_OK;
        }
    }
    if (N >= 2 && N <= 16 && aligned16_or_null(smooth_inv) && aligned16(W) && aligned16(X)) {
        // small batch: the MFMA GEMV quantizes the tokens itself when the
        // wave's K range fits its registers
        fa::GemvPlan gp = fa::plan_gemv(M, N, K, g, G, true, 0, 0, smooth_inv != nullptr);
        if (gp.kind == 3) {
            FA_HIP(fa::launch_gemv(gp, W, w_scale, nullptr, nullptr, X, act_scale, smooth_inv, Y,
                                   nullptr, 0, 0, 0, 0, M, N, K, g, G, s));
            return FA_OK;
        }
    }
    Workspace* ws = nullptr;
    rc = current_ws(&ws);
    if (rc) return rc;
    void* p = ws->xq;
    rc = grow(&p, &ws->xq_bytes, (size_t)N * (size_t)K, s);
    ws->xq = (int8_t*)p;
    if (rc) return rc;
    p = ws->xs;
    rc = grow(&p, &ws->xs_bytes, (size_t)N * (size_t)G * sizeof(float), s);
    ws->xs = (float*)p;
    if (rc) return rc;
    FA_HIP(fa::launch_quantize_activations(X, nullptr, fa::Prologue::kPlain, act_scale, smooth_inv,
                                           ws->xq, ws->xs, nullptr, N, K, g, G, s));
    prof_mark();
    return linear_quantized(fn, W, w_scale, g, G, ws->xq, ws->xs, Y, nullptr, 0, 0, 0, 0, M, N, K,
                            s);
}

int fa_w8a8_gemm(const int8_t* W, const uint16_t* w_scale, int group_size,
                 const uint16_t* act_scale, const uint16_t* smooth_inv, const uint16_t* X,
                 uint16_t* Y, int M, int N, int K, void* stream) {
    ProfCall pc(stream);
    const int rc = gemm_impl(W, w_scale, group_size, act_scale, smooth_inv, X, Y, M, N, K, stream);
    if (rc == FA_OK && M > 0 && N > 0)
        pc.finish("fa_w8a8_gemm", M, N, K, group_size, act_scale, smooth_inv);
    return rc;
}

// ------------------------------------------------- no-alloc variant ----
//
// fa_w8a8_gemm_noalloc: fa_w8a8_gemm with its scratch (x_q, x_scale and the
// prefill scale tables) carved from one file-scope device array instead of
// the grow-only per-thread workspace, so the call never allocates.  Each
// device holds its own copy of the array; host code must use the address
// hipGetSymbolAddress reports for the current device, never the symbol.
}  // extern "C"

namespace {

constexpr size_t kNoallocBytes = (size_t)FA_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[kNoallocBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's copy of `scratch` (looked up once per device).
int scratch_for_current_device(const char* fn, unsigned char** out) {
    int dev = 0;
    FA_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(FA_ERR_INVALID_ARG, "%s: device %d", fn, dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        FA_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail(FA_ERR_HIP, "%s: no device address for the scratch array", fn);
        g_scratch_ptr[dev] = p;
    }
    *out = static_cast<unsigned char*>(g_scratch_ptr[dev]);
    return FA_OK;
}

size_t round256(size_t n) { return (n + 255) & ~(size_t)255; }

}  // namespace

extern "C" {

size_t fa_noalloc_scratch_bytes(int M, int N, int K, int group_size) {
    if (M < 0 || N < 0 || K <= 0) return (size_t)-1;
    const int g = eff_group(K, group_size);
    const size_t G = (size_t)((K + g - 1) / g);
    return round256((size_t)N * (size_t)K) + round256((size_t)N * G * sizeof(float)) +
           round256(fa::gemm_pipe_tables_bytes(M, N, (int)G));
}

int fa_w8a8_gemm_noalloc(const int8_t* W, const uint16_t* w_scale, int group_size,
                         const uint16_t* act_scale, const uint16_t* smooth_inv, const uint16_t* X,
                         uint16_t* Y, int M, int N, int K, void* stream) {
    const char* fn = "fa_w8a8_gemm_noalloc";
    g_err.clear();
    int rc = check_dims(fn, M, N, K);
    if (rc) return rc;
    if (M == 0 || N == 0) return FA_OK;
    if (!W || !w_scale || !X || !Y) return fail(FA_ERR_INVALID_ARG, "%s: null pointer argument", fn);
    if (overlaps(Y, (size_t)N * M, X, (size_t)N * K))
        return fail(FA_ERR_INVALID_ARG, "%s: Y overlaps X", fn);
    hipStream_t s = (hipStream_t)stream;
    const int g = eff_group(K, group_size);
    const int G = (K + g - 1) / g;
    if (N == 1 && aligned16_or_null(smooth_inv) && aligned16(W) && aligned16(X)) {
        fa::GemvPlan gp = fa::plan_gemv(M, N, K, g, G, true);
        if (gp.kind == 1 || gp.kind == 2) {
            FA_HIP(fa::launch_gemv(gp, W, w_scale, nullptr, nullptr, X, act_scale, smooth_inv, Y,
                                   nullptr, 0, 0, 0, 0, M, N, K, g, G, s));
            return FA_OK;
        }
    }
    // (one token on a path without in-kernel quantization needs scratch too)
    const size_t xq_bytes = round256((size_t)N * (size_t)K);
    const size_t xs_bytes = round256((size_t)N * (size_t)G * sizeof(float));
    const size_t need = fa_noalloc_scratch_bytes(M, N, K, group_size);
    if (need > kNoallocBytes)
        return fail(FA_ERR_INVALID_ARG,
                    "%s: M=%d N=%d K=%d needs %zu B of scratch, above the %zu B maximum", fn, M, N,
                    K, need, kNoallocBytes);
    unsigned char* base = nullptr;
    rc = scratch_for_current_device(fn, &base);
    if (rc) return rc;
    int8_t* xq = reinterpret_cast<int8_t*>(base);
    float* xs = reinterpret_cast<float*>(base + xq_bytes);
    float* tables = reinterpret_cast<float*>(base + xq_bytes + xs_bytes);
    // every byte the kernels read is written first: nothing to clear
    FA_HIP(fa::launch_quantize_activations(X, nullptr, fa::Prologue::kPlain, act_scale, smooth_inv,
                                           xq, xs, nullptr, N, K, g, G, s));
    return linear_quantized(fn, W, w_scale, g, G, xq, xs, Y, nullptr, 0, 0, 0, 0, M, N, K, s,
                            tables);
}

static int gemm_rms_impl(const int8_t* W, const uint16_t* w_scale, int group_size,
                     const uint16_t* act_scale, const uint16_t* smooth_inv, const uint16_t* x,
                     const uint16_t* resid, uint16_t* h_out, const uint16_t* gamma, float eps,
                     uint16_t* Y, int M, int N, int K, void* stream) {
    const char* fn = "fa_w8a8_gemm_rms";
    g_err.clear();
    int rc = check_dims(fn, M, N, K);
    if (rc) return rc;
    if (M == 0 || N == 0) return FA_OK;
    if (!W || !w_scale || !x || !gamma || !Y)
        return fail(FA_ERR_INVALID_ARG, "%s: null pointer argument", fn);
    if (resid && !h_out)
        return fail(FA_ERR_INVALID_ARG, "%s: a residual addend needs h_out", fn);
    const size_t nk = (size_t)N * (size_t)K;
    if (h_out && (overlaps(h_out, nk, x, nk) || overlaps(h_out, nk, resid, nk)))
        return fail(FA_ERR_INVALID_ARG, "%s: h_out overlaps x or resid", fn);
    const size_t nm = (size_t)N * (size_t)M;
    if (overlaps(Y, nm, x, nk) || overlaps(Y, nm, resid, nk) || overlaps(Y, nm, h_out, nk) ||
        overlaps(Y, nm, gamma, (size_t)K))
        return fail(FA_ERR_INVALID_ARG, "%s: Y overlaps an input or h_out", fn);
    if (K > 65536) return fail(FA_ERR_INVALID_ARG, "%s: K=%d exceeds 65536", fn, K);
    hipStream_t s = (hipStream_t)stream;
    const int g = eff_group(K, group_size);
    const int G = (K + g - 1) / g;
    if (N == 1 && aligned16_or_null(smooth_inv) && aligned16(W) && aligned16(x) &&
        aligned16(gamma) &&
        (!resid || aligned16(resid)) && (!h_out || aligned16(h_out))) {
        fa::GemvPlan gp = fa::plan_gemv(M, N, K, g, G, true, 2);
        if (gp.kind == 1 || gp.kind == 2) {
            FA_HIP(fa::launch_gemv(gp, W, w_scale, nullptr, nullptr, x, act_scale, smooth_inv, Y,
                                   nullptr, 0, 0, 0, 0, M, N, K, g, G, s, resid, gamma, eps,
                                   resid ? h_out : nullptr));
            if (!resid && h_out)
                FA_HIP(hipMemcpyAsync(h_out, x, nk * 2, hipMemcpyDeviceToDevice, s));
            return FA_OK;
        }
    }
    // separate launches: h_out <- x (+ resid), then RMSNorm + quant, then the linear
    Workspace* ws = nullptr;
    rc = current_ws(&ws);
    if (rc) return rc;
    void* p = ws->xq;
    rc = grow(&p, &ws->xq_bytes, nk, s);
    ws->xq = (int8_t*)p;
    if (rc) return rc;
    p = ws->xs;
    rc = grow(&p, &ws->xs_bytes, (size_t)N * (size_t)G * sizeof(float), s);
    ws->xs = (float*)p;
    if (rc) return rc;
    FA_HIP(fa::launch_rms_norm_quant(x, resid, h_out, gamma, eps, smooth_inv, act_scale, g, G, ws->xq,
                                     ws->xs, nullptr, N, K, s));
    return linear_quantized(fn, W, w_scale, g, G, ws->xq, ws->xs, Y, nullptr, 0, 0, 0, 0, M, N, K,
                            s);
}

static int gemm_swiglu_impl(const int8_t* W13, const uint16_t* w13_scale, int group_size,
                        const uint16_t* act_scale, const uint16_t* smooth_inv, const uint16_t* x,
                        const uint16_t* resid, uint16_t* h_out, const uint16_t* gamma, float eps,
                        uint16_t* act, int F, int N, int K, void* stream) {
    const char* fn = "fa_w8a8_gemm_swiglu";
    g_err.clear();
    int rc = check_dims(fn, F, N, K);
    if (rc) return rc;
    if (F == 0 || N == 0) return FA_OK;
    if (F > (1 << 29)) return fail(FA_ERR_INVALID_ARG, "%s: F=%d too large", fn, F);
    if (!W13 || !w13_scale || !x || !act)
        return fail(FA_ERR_INVALID_ARG, "%s: null pointer argument", fn);
    if (!gamma && (resid || h_out))
        return fail(FA_ERR_INVALID_ARG, "%s: resid / h_out need the RMSNorm (gamma)", fn);
    if (resid && !h_out)
        return fail(FA_ERR_INVALID_ARG, "%s: a residual addend needs h_out", fn);
    const size_t nk = (size_t)N * (size_t)K;
    if (h_out && (overlaps(h_out, nk, x, nk) || overlaps(h_out, nk, resid, nk)))
        return fail(FA_ERR_INVALID_ARG, "%s: h_out overlaps x or resid", fn);
    const size_t nf = (size_t)N * (size_t)F;
    if (overlaps(act, nf, x, nk) || overlaps(act, nf, resid, nk) || overlaps(act, nf, h_out, nk) ||
        overlaps(act, nf, gamma, (size_t)K))
        return fail(FA_ERR_INVALID_ARG, "%s: act overlaps an input or h_out", fn);
    if (gamma && K > 65536) return fail(FA_ERR_INVALID_ARG, "%s: K=%d exceeds 65536", fn, K);
    hipStream_t s = (hipStream_t)stream;
    const int M = 2 * F;
    const int g = eff_group(K, group_size);
    const int G = (K + g - 1) / g;
    if (N == 1 && aligned16_or_null(smooth_inv) && aligned16(W13) && aligned16(x) &&
        (!gamma || aligned16(gamma)) &&
        (!resid || aligned16(resid)) && (!h_out || aligned16(h_out))) {
        fa::GemvPlan gp = fa::plan_gemv(M, N, K, g, G, true, gamma ? 2 : 0, 1);
        if (gp.kind == 2) {
            FA_HIP(fa::launch_gemv(gp, W13, w13_scale, nullptr, nullptr, x, act_scale, smooth_inv,
                                   act, nullptr, 0, 0, 0, 0, M, N, K, g, G, s, resid, gamma, eps,
                                   resid ? h_out : nullptr));
            if (!resid && h_out)
                FA_HIP(hipMemcpyAsync(h_out, x, nk * 2, hipMemcpyDeviceToDevice, s));
            return FA_OK;
        }
    }
    if (N >= 2 && N <= 16 && aligned16(W13)) {
        // small batch: the MFMA GEMV's epilogue forms the pairs; without the
        // RMSNorm it also quantizes the tokens when their range fits
        fa::GemvPlan gp{};
        if (!gamma && aligned16(x) && aligned16_or_null(smooth_inv))
            gp = fa::plan_gemv(M, N, K, g, G, true, 0, 1, smooth_inv != nullptr);
        if (gp.kind == 3) {
            FA_HIP(fa::launch_gemv(gp, W13, w13_scale, nullptr, nullptr, x, act_scale, smooth_inv,
                                   act, nullptr, 0, 0, 0, 0, M, N, K, g, G, s));
            return FA_OK;
        }
        gp = fa::plan_gemv(M, N, K, g, G, false, 0, 1);
        if (gp.kind == 3) {
            Workspace* ws = nullptr;
            rc = current_ws(&ws);
            if (rc) return rc;
            void* p = ws->xq;
            rc = grow(&p, &ws->xq_bytes, nk, s);
            ws->xq = (int8_t*)p;
            if (rc) return rc;
            p = ws->xs;
            rc = grow(&p, &ws->xs_bytes, (size_t)N * (size_t)G * sizeof(float), s);
            ws->xs = (float*)p;
            if (rc) return rc;
            if (gamma)
                FA_HIP(fa::launch_rms_norm_quant(x, resid, h_out, gamma, eps, smooth_inv,
                                                 act_scale, g, G, ws->xq, ws->xs, nullptr, N, K,
                                                 s));
            else
                FA_HIP(fa::launch_quantize_activations(x, nullptr, fa::Prologue::kPlain,
                                                       act_scale, smooth_inv, ws->xq, ws->xs,
                                                       nullptr, N, K, g, G, s));
            FA_HIP(fa::launch_gemv(gp, W13, w13_scale, ws->xq, ws->xs, nullptr, nullptr, nullptr,
                                   act, nullptr, 0, 0, 0, 0, M, N, K, g, G, s));
            return FA_OK;
        }
    }
    // separate launches: the linear into scratch [N, 2F], then the pairs
    Workspace* ws = nullptr;
    rc = current_ws(&ws);
    if (rc) return rc;
    void* p = ws->yt;
    rc = grow(&p, &ws->yt_bytes, (size_t)N * (size_t)M * 2, s);
    ws->yt = (uint16_t*)p;
    if (rc) return rc;
    uint16_t* yt = ws->yt;
    rc = gamma ? fa_w8a8_gemm_rms(W13, w13_scale, group_size, act_scale, smooth_inv, x, resid,
                                  h_out, gamma, eps, yt, M, N, K, stream)
               : fa_w8a8_gemm(W13, w13_scale, group_size, act_scale, smooth_inv, x, yt, M, N, K,
                              stream);
    if (rc) return rc;
    FA_HIP(fa::launch_swiglu_pairs(yt, act, (int64_t)N * F, s));
    return FA_OK;
}

static int gemm_swiglu_sep_impl(const int8_t* W1, const uint16_t* w1_scale, const int8_t* W3,
                                const uint16_t* w3_scale, int group_size,
                                const uint16_t* act_scale1, const uint16_t* smooth_inv1,
                                const uint16_t* act_scale3, const uint16_t* smooth_inv3,
                                const uint16_t* x, const uint16_t* resid, uint16_t* h_out,
                                const uint16_t* gamma, float eps, uint16_t* act, int F, int N,
                                int K, void* stream) {
    const char* fn = "fa_w8a8_gemm_swiglu_sep";
    g_err.clear();
    int rc = check_dims(fn, F, N, K);
    if (rc) return rc;
    if (F == 0 || N == 0) return FA_OK;
    if (F > (1 << 29)) return fail(FA_ERR_INVALID_ARG, "%s: F=%d too large", fn, F);
    if (!W1 || !w1_scale || !W3 || !w3_scale || !x || !act)
        return fail(FA_ERR_INVALID_ARG, "%s: null pointer argument", fn);
    if (!gamma && (resid || h_out))
        return fail(FA_ERR_INVALID_ARG, "%s: resid / h_out need the RMSNorm (gamma)", fn);
    if (resid && !h_out)
        return fail(FA_ERR_INVALID_ARG, "%s: a residual addend needs h_out", fn);
    const size_t nk = (size_t)N * (size_t)K;
    if (h_out && (overlaps(h_out, nk, x, nk) || overlaps(h_out, nk, resid, nk)))
        return fail(FA_ERR_INVALID_ARG, "%s: h_out overlaps x or resid", fn);
    const size_t nf = (size_t)N * (size_t)F;
    if (overlaps(act, nf, x, nk) || overlaps(act, nf, resid, nk) || overlaps(act, nf, h_out, nk) ||
        overlaps(act, nf, gamma, (size_t)K))
        return fail(FA_ERR_INVALID_ARG, "%s: act overlaps an input or h_out", fn);
    if (gamma && K > 65536) return fail(FA_ERR_INVALID_ARG, "%s: K=%d exceeds 65536", fn, K);
    hipStream_t s = (hipStream_t)stream;
    const int M = 2 * F;
    const int g = eff_group(K, group_size);
    const int G = (K + g - 1) / g;
    if (N == 1 && aligned16_or_null(smooth_inv1) && aligned16_or_null(smooth_inv3) &&
        aligned16(W1) && aligned16(W3) && aligned16(x) && (!gamma || aligned16(gamma)) &&
        (!resid || aligned16(resid)) && (!h_out || aligned16(h_out))) {
        fa::GemvPlan gp = fa::plan_gemv(M, N, K, g, G, true, gamma ? 2 : 0, 2);
        if (gp.kind == 2) {
            FA_HIP(fa::launch_gemv(gp, W1, w1_scale, nullptr, nullptr, x, act_scale1, smooth_inv1,
                                   act, nullptr, 0, 0, 0, 0, M, N, K, g, G, s, resid, gamma, eps,
                                   resid ? h_out : nullptr, W3, w3_scale, act_scale3,
                                   smooth_inv3));
            if (!resid && h_out)
                FA_HIP(hipMemcpyAsync(h_out, x, nk * 2, hipMemcpyDeviceToDevice, s));
            return FA_OK;
        }
    }
    // separate launches: gate into act, up into scratch, then silu and mul
    Workspace* ws = nullptr;
    rc = current_ws(&ws);
    if (rc) return rc;
    void* p = ws->yt;
    rc = grow(&p, &ws->yt_bytes, nf * 2, s);
    ws->yt = (uint16_t*)p;
    if (rc) return rc;
    uint16_t* up = ws->yt;
    if (gamma) {
        rc = fa_w8a8_gemm_rms(W1, w1_scale, group_size, act_scale1, smooth_inv1, x, resid, h_out,
                              gamma, eps, act, F, N, K, stream);
        if (rc) return rc;
        rc = fa_w8a8_gemm_rms(W3, w3_scale, group_size, act_scale3, smooth_inv3,
                              resid ? h_out : x, nullptr, nullptr, gamma, eps, up, F, N, K, stream);
    } else {
        rc = fa_w8a8_gemm(W1, w1_scale, group_size, act_scale1, smooth_inv1, x, act, F, N, K,
                          stream);
        if (rc) return rc;
        rc = fa_w8a8_gemm(W3, w3_scale, group_size, act_scale3, smooth_inv3, x, up, F, N, K,
                          stream);
    }
    if (rc) return rc;
    FA_HIP(fa::launch_elementwise(0, act, nullptr, (int64_t)nf, s));   // silu_forward
    FA_HIP(fa::launch_elementwise(1, act, up, (int64_t)nf, s));        // mul_forward
    return FA_OK;
}

static int gemm_silu_mul_impl(const int8_t* W, const uint16_t* w_scale, int group_size,
                          const uint16_t* act_scale, const uint16_t* smooth_inv,
                          const uint16_t* gate, const uint16_t* up, uint16_t* Y, int M, int N,
                          int K, void* stream) {
    const char* fn = "fa_w8a8_gemm_silu_mul";
    g_err.clear();
    int rc = check_dims(fn, M, N, K);
    if (rc) return rc;
    if (M == 0 || N == 0) return FA_OK;
    if (!W || !w_scale || !gate || !up || !Y)
        return fail(FA_ERR_INVALID_ARG, "%s: null pointer argument", fn);
    if (overlaps(Y, (size_t)N * M, gate, (size_t)N * K) || overlaps(Y, (size_t)N * M, up, (size_t)N * K))
        return fail(FA_ERR_INVALID_ARG, "%s: Y overlaps gate or up", fn);
    hipStream_t s = (hipStream_t)stream;
    const int g = eff_group(K, group_size);
    const int G = (K + g - 1) / g;
    if (N == 1 && aligned16_or_null(smooth_inv) && aligned16(W) && aligned16(gate) &&
        aligned16(up)) {
        fa::GemvPlan gp = fa::plan_gemv(M, N, K, g, G, true, 1);
        if (gp.kind == 1 || gp.kind == 2) {
            FA_HIP(fa::launch_gemv(gp, W, w_scale, nullptr, nullptr, gate, act_scale, smooth_inv,
                                   Y, nullptr, 0, 0, 0, 0, M, N, K, g, G, s, up));
            return FA_OK;
        }
    }
    Workspace* ws = nullptr;
    rc = current_ws(&ws);
    if (rc) return rc;
    void* p = ws->xq;
    rc = grow(&p, &ws->xq_bytes, (size_t)N * (size_t)K, s);
    ws->xq = (int8_t*)p;
    if (rc) return rc;
    p = ws->xs;
    rc = grow(&p, &ws->xs_bytes, (size_t)N * (size_t)G * sizeof(float), s);
    ws->xs = (float*)p;
    if (rc) return rc;
    FA_HIP(fa::launch_quantize_activations(gate, up, fa::Prologue::kSiluMul, act_scale, smooth_inv,
                                           ws->xq, ws->xs, nullptr, N, K, g, G, s));
    return linear_quantized(fn, W, w_scale, g, G, ws->xq, ws->xs, Y, nullptr, 0, 0, 0, 0, M, N, K,
                            s);
}

int fa_w8a8_gemm_rms(const int8_t* W, const uint16_t* w_scale, int group_size,
                     const uint16_t* act_scale, const uint16_t* smooth_inv, const uint16_t* x,
                     const uint16_t* resid, uint16_t* h_out, const uint16_t* gamma, float eps,
                     uint16_t* Y, int M, int N, int K, void* stream) {
    ProfCall pc(stream);
    const int rc = gemm_rms_impl(W, w_scale, group_size, act_scale, smooth_inv, x, resid, h_out,
                                 gamma, eps, Y, M, N, K, stream);
    if (rc == FA_OK && M > 0 && N > 0)
        pc.finish("fa_w8a8_gemm_rms", M, N, K, group_size, act_scale, smooth_inv);
    return rc;
}

int fa_w8a8_gemm_swiglu(const int8_t* W13, const uint16_t* w13_scale, int group_size,
                        const uint16_t* act_scale, const uint16_t* smooth_inv, const uint16_t* x,
                        const uint16_t* resid, uint16_t* h_out, const uint16_t* gamma, float eps,
                        uint16_t* act, int F, int N, int K, void* stream) {
    ProfCall pc(stream);
    const int rc = gemm_swiglu_impl(W13, w13_scale, group_size, act_scale, smooth_inv, x, resid,
                                    h_out, gamma, eps, act, F, N, K, stream);
    if (rc == FA_OK && F > 0 && N > 0)
        pc.finish("fa_w8a8_gemm_swiglu", 2 * F, N, K, group_size, act_scale, smooth_inv);
    return rc;
}

int fa_w8a8_gemm_silu_mul(const int8_t* W, const uint16_t* w_scale, int group_size,
                          const uint16_t* act_scale, const uint16_t* smooth_inv,
                          const uint16_t* gate, const uint16_t* up, uint16_t* Y, int M, int N,
                          int K, void* stream) {
    ProfCall pc(stream);
    const int rc = gemm_silu_mul_impl(W, w_scale, group_size, act_scale, smooth_inv, gate, up, Y,
                                      M, N, K, stream);
    if (rc == FA_OK && M > 0 && N > 0)
        pc.finish("fa_w8a8_gemm_silu_mul", M, N, K, group_size, act_scale, smooth_inv);
    return rc;
}

int fa_w8a8_gemm_swiglu_sep(const int8_t* W1, const uint16_t* w1_scale, const int8_t* W3,
                            const uint16_t* w3_scale, int group_size,
                            const uint16_t* act_scale1, const uint16_t* smooth_inv1,
                            const uint16_t* act_scale3, const uint16_t* smooth_inv3,
                            const uint16_t* x, const uint16_t* resid, uint16_t* h_out,
                            const uint16_t* gamma, float eps, uint16_t* act, int F, int N, int K,
                            void* stream) {
    ProfCall pc(stream);
    const int rc = gemm_swiglu_sep_impl(W1, w1_scale, W3, w3_scale, group_size, act_scale1,
                                        smooth_inv1, act_scale3, smooth_inv3, x, resid, h_out,
                                        gamma, eps, act, F, N, K, stream);
    if (rc == FA_OK && F > 0 && N > 0)
        pc.finish("fa_w8a8_gemm_swiglu_sep", 2 * F, N, K, group_size,
                  act_scale1 || act_scale3, smooth_inv1 || smooth_inv3);
    return rc;
}

int fa_profile_enable(int on) {
    const int prev = prof_enabled() ? 1 : 0;
    g_prof_on.store(on ? 1 : 0, std::memory_order_relaxed);
    return prev;
}

size_t fa_profile_summary(char* buf, size_t n) {
    const std::string t = prof_state().summary();
    if (buf && n > 0) {
        const size_t c = t.size() < n - 1 ? t.size() : n - 1;
        memcpy(buf, t.data(), c);
        buf[c] = 0;
    }
    return t.size();
}

void fa_profile_reset(void) {
    ProfState& ps = prof_state();
    std::lock_guard<std::mutex> lock(ps.mu);
    ps.buckets.clear();
}

int fa_gemm_fp16(const uint16_t* W, const uint16_t* X, uint16_t* Y, int M, int N, int K,
                 void* stream) {
    const char* fn = "fa_gemm_fp16";
    g_err.clear();
    int rc = check_dims(fn, M, N, K);
    if (rc) return rc;
    if (M == 0 || N == 0) return FA_OK;
    if (!W || !X || !Y) return fail(FA_ERR_INVALID_ARG, "%s: null pointer argument", fn);
    hipStream_t s = (hipStream_t)stream;
    if (aligned16(W) && aligned16(X) && fa::gemv_f16_ok(M, N, K) && N <= 64) {
        FA_HIP(fa::launch_gemv_f16(W, X, Y, M, N, K, s));
        return FA_OK;
    }
    if (N > 65535) return fail(FA_ERR_INVALID_ARG, "%s: N=%d too large", fn, N);
    FA_HIP(fa::launch_gemm_f16_generic(W, X, Y, M, N, K, s));
    return FA_OK;
}

int fa_quantize_activations(const uint16_t* X, const uint16_t* act_scale,
                            const uint16_t* smooth_inv, int8_t* X_q, float* X_scale, int N, int K,
                            int group_size, void* stream) {
    const char* fn = "fa_quantize_activations";
    g_err.clear();
    int rc = check_dims(fn, 0, N, K);
    if (rc) return rc;
    if (N == 0) return FA_OK;
    if (!X || !X_q || !X_scale) return fail(FA_ERR_INVALID_ARG, "%s: null pointer argument", fn);
    const int g = eff_group(K, group_size);
    const int G = (K + g - 1) / g;
    FA_HIP(fa::launch_quantize_activations(X, nullptr, fa::Prologue::kPlain, act_scale, smooth_inv,
                                           X_q, X_scale, nullptr, N, K, g, G,
                                           (hipStream_t)stream));
    return FA_OK;
}

int fa_rms_norm(const uint16_t* x, const uint16_t* weight, uint16_t* out, int n_tokens, int dim,
                float eps, void* stream) {
    const char* fn = "fa_rms_norm";
    g_err.clear();
    if (n_tokens < 0 || dim <= 0)
        return fail(FA_ERR_INVALID_ARG, "%s: bad n_tokens=%d dim=%d", fn, n_tokens, dim);
    if (n_tokens == 0) return FA_OK;
    if (!x || !weight || !out) return fail(FA_ERR_INVALID_ARG, "%s: null pointer argument", fn);
    if (dim > 65536) return fail(FA_ERR_INVALID_ARG, "%s: dim=%d exceeds 65536", fn, dim);
    FA_HIP(fa::launch_rms_norm_quant(x, nullptr, nullptr, weight, eps, nullptr,
                                     nullptr, dim, 1, nullptr, nullptr,
                                     out, n_tokens, dim, (hipStream_t)stream));
    return FA_OK;
}

int fa_rms_norm_quant(const uint16_t* x, const uint16_t* weight, float eps,
                      const uint16_t* smooth_inv, const uint16_t* act_scale, int group_size,
                      int8_t* X_q, float* X_scale, uint16_t* out, int n_tokens, int dim,
                      void* stream) {
    const char* fn = "fa_rms_norm_quant";
    g_err.clear();
    if (n_tokens < 0 || dim <= 0)
        return fail(FA_ERR_INVALID_ARG, "%s: bad n_tokens=%d dim=%d", fn, n_tokens, dim);
    if (n_tokens == 0) return FA_OK;
    if (!x || !weight || !X_q || !X_scale)
        return fail(FA_ERR_INVALID_ARG, "%s: null pointer argument", fn);
    if (dim > 65536) return fail(FA_ERR_INVALID_ARG, "%s: dim=%d exceeds 65536", fn, dim);
    const int g = eff_group(dim, group_size);
    const int G = (dim + g - 1) / g;
    FA_HIP(fa::launch_rms_norm_quant(x, nullptr, nullptr, weight, eps, smooth_inv,
                                     act_scale, g, G, X_q, X_scale, out,
                                     n_tokens, dim, (hipStream_t)stream));
    return FA_OK;
}

int fa_residual_rms_norm_quant(uint16_t* h, const uint16_t* resid, const uint16_t* weight,
                               float eps, const uint16_t* smooth_inv, const uint16_t* act_scale,
                               int group_size, int8_t* X_q, float* X_scale, uint16_t* out,
                               int n_tokens, int dim, void* stream) {
    const char* fn = "fa_residual_rms_norm_quant";
    g_err.clear();
    if (n_tokens < 0 || dim <= 0)
        return fail(FA_ERR_INVALID_ARG, "%s: bad n_tokens=%d dim=%d", fn, n_tokens, dim);
    if (n_tokens == 0) return FA_OK;
    if (!h || !resid || !weight || !X_q || !X_scale)
        return fail(FA_ERR_INVALID_ARG, "%s: null pointer argument", fn);
    if (dim > 65536) return fail(FA_ERR_INVALID_ARG, "%s: dim=%d exceeds 65536", fn, dim);
    const int g = eff_group(dim, group_size);
    const int G = (dim + g - 1) / g;
    FA_HIP(fa::launch_rms_norm_quant(h, resid, h, weight, eps, smooth_inv, act_scale, g, G, X_q,
                                     X_scale, out, n_tokens, dim, (hipStream_t)stream));
    return FA_OK;
}

static int elementwise(const char* fn, int op, uint16_t* a, const uint16_t* b, int64_t n,
                       void* stream) {
    g_err.clear();
    if (n < 0) return fail(FA_ERR_INVALID_ARG, "%s: negative n", fn);
    if (n == 0) return FA_OK;
    if (!a || (op != 0 && !b)) return fail(FA_ERR_INVALID_ARG, "%s: null pointer argument", fn);
    FA_HIP(fa::launch_elementwise(op, a, b, n, (hipStream_t)stream));
    return FA_OK;
}

int fa_silu(uint16_t* x, int64_t n, void* stream) {
    return elementwise("fa_silu", 0, x, nullptr, n, stream);
}
int fa_mul(uint16_t* a, const uint16_t* b, int64_t n, void* stream) {
    return elementwise("fa_mul", 1, a, b, n, stream);
}
int fa_residual_add(uint16_t* a, const uint16_t* b, int64_t n, void* stream) {
    return elementwise("fa_residual_add", 2, a, b, n, stream);
}

int fa_silu_mul_quant(const uint16_t* gate, const uint16_t* up, const uint16_t* smooth_inv,
                      const uint16_t* act_scale, int group_size, int8_t* X_q, float* X_scale,
                      uint16_t* out, int n_tokens, int dim, void* stream) {
    const char* fn = "fa_silu_mul_quant";
    g_err.clear();
    if (n_tokens < 0 || dim <= 0)
        return fail(FA_ERR_INVALID_ARG, "%s: bad n_tokens=%d dim=%d", fn, n_tokens, dim);
    if (n_tokens == 0) return FA_OK;
    if (!gate || !up || !X_q || !X_scale)
        return fail(FA_ERR_INVALID_ARG, "%s: null pointer argument", fn);
    const int g = eff_group(dim, group_size);
    const int G = (dim + g - 1) / g;
    FA_HIP(fa::launch_quantize_activations(gate, up, fa::Prologue::kSiluMul, act_scale, smooth_inv,
                                           X_q, X_scale, out, n_tokens, dim, g, G,
                                           (hipStream_t)stream));
    return FA_OK;
}

int fa_quantize_weights_groupwise(const uint16_t* w, int64_t rows, int64_t K, int group_size,
                                  int8_t* q, uint16_t* scale, void* stream) {
    const char* fn = "fa_quantize_weights_groupwise";
    g_err.clear();
    if (rows < 0 || K <= 0 || group_size <= 0)
        return fail(FA_ERR_INVALID_ARG, "%s: bad rows=%lld K=%lld group_size=%d", fn,
                    (long long)rows, (long long)K, group_size);
    if (rows == 0) return FA_OK;
    if (!w || !q || !scale) return fail(FA_ERR_INVALID_ARG, "%s: null pointer argument", fn);
    FA_HIP(fa::launch_quantize_weights(w, rows, K, group_size, q, scale, (hipStream_t)stream));
    return FA_OK;
}

int fa_qkv_split_heads_gqa(const uint16_t* qkv, uint16_t* q, uint16_t* k, uint16_t* v, int T,
                           int n_q, int n_kv, int head_dim, void* stream) {
    const char* fn = "fa_qkv_split_heads_gqa";
    g_err.clear();
    if (T < 0 || n_q <= 0 || n_kv <= 0 || head_dim <= 0)
        return fail(FA_ERR_INVALID_ARG, "%s: bad T=%d n_q=%d n_kv=%d head_dim=%d", fn, T, n_q,
                    n_kv, head_dim);
    if ((int64_t)T * (n_q + 2 * n_kv) * head_dim > INT32_MAX)
        return fail(FA_ERR_INVALID_ARG, "%s: qkv larger than 2^31 elements", fn);
    if (T == 0) return FA_OK;
    if (!qkv || !q || !k || !v) return fail(FA_ERR_INVALID_ARG, "%s: null pointer argument", fn);
    const bool vec = head_dim % 8 == 0 && aligned16(qkv) && aligned16(q) && aligned16(k) &&
                     aligned16(v);
    FA_HIP(fa::launch_qkv_split(qkv, q, k, v, T, n_q, n_kv, head_dim, vec, (hipStream_t)stream));
    return FA_OK;
}

int fa_qkv_split_heads(const uint16_t* qkv, uint16_t* q, uint16_t* k, uint16_t* v, int T,
                       int n_heads, int head_dim, void* stream) {
    return fa_qkv_split_heads_gqa(qkv, q, k, v, T, n_heads, n_heads, head_dim, stream);
}

int fa_merge_heads(const uint16_t* heads, uint16_t* out, int T, int n_heads, int head_dim,
                   void* stream) {
    const char* fn = "fa_merge_heads";
    g_err.clear();
    if (T < 0 || n_heads <= 0 || head_dim <= 0)
        return fail(FA_ERR_INVALID_ARG, "%s: bad T=%d n_heads=%d head_dim=%d", fn, T, n_heads,
                    head_dim);
    if ((int64_t)T * n_heads * head_dim > INT32_MAX)
        return fail(FA_ERR_INVALID_ARG, "%s: more than 2^31 elements", fn);
    if (T == 0) return FA_OK;
    if (!heads || !out) return fail(FA_ERR_INVALID_ARG, "%s: null pointer argument", fn);
    const bool vec = head_dim % 8 == 0 && aligned16(heads) && aligned16(out);
    FA_HIP(fa::launch_merge_heads(heads, out, T, n_heads, head_dim, vec, (hipStream_t)stream));
    return FA_OK;
}

namespace {
int prefill_attention(const char* fn, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                      uint16_t* out, int n_q, int n_kv, int T, int D, float sm_scale,
                      void* stream, int window_size, bool token_major) {
    g_err.clear();
    if (T < 0 || n_q <= 0 || n_kv <= 0 || D <= 0)
        return fail(FA_ERR_INVALID_ARG, "%s: bad n_q=%d n_kv=%d T=%d D=%d", fn, n_q, n_kv, T, D);
    if (n_q % n_kv != 0)
        return fail(FA_ERR_INVALID_ARG, "%s: n_q=%d is not a multiple of n_kv=%d", fn, n_q, n_kv);
    if (D > fa::attention_max_dim())
        return fail(FA_ERR_INVALID_ARG, "%s: head dim %d above %d", fn, D, fa::attention_max_dim());
    if (!(sm_scale == sm_scale) || sm_scale > 3.0e38f || sm_scale < -3.0e38f)
        return fail(FA_ERR_INVALID_ARG, "%s: sm_scale must be finite", fn);
    if ((int64_t)n_q * T * D > INT32_MAX)
        return fail(FA_ERR_INVALID_ARG, "%s: q larger than 2^31 elements", fn);
    if (T == 0) return FA_OK;
    if (!q || !k || !v || !out) return fail(FA_ERR_INVALID_ARG, "%s: null pointer argument", fn);
    if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) & 1)
        return fail(FA_ERR_INVALID_ARG, "%s: q, k, v and out must be 2-byte aligned", fn);
    const size_t nq = (size_t)n_q * T * D, nkv = (size_t)n_kv * T * D;
    if (overlaps(out, nq, q, nq) || overlaps(out, nq, k, nkv) || overlaps(out, nq, v, nkv))
        return fail(FA_ERR_INVALID_ARG, "%s: out overlaps q, k or v", fn);
    FA_HIP(fa::launch_prefill_attention(q, k, v, out, n_q, n_kv, T, D, sm_scale, window_size,
                                        token_major, (hipStream_t)stream));
    return FA_OK;
}
}  // namespace

int fa_prefill_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out,
                         void* workspace, int n_q, int n_kv, int T, int D, float sm_scale,
                         void* stream, int window_size) {
    (void)workspace;   // the fused kernel keeps scores on chip and needs no scratch
    return prefill_attention("fa_prefill_attention", q, k, v, out, n_q, n_kv, T, D, sm_scale,
                             stream, window_size, false);
}

int fa_prefill_attention_merged(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                uint16_t* out, int n_q, int n_kv, int T, int D, float sm_scale,
                                void* stream, int window_size) {
    return prefill_attention("fa_prefill_attention_merged", q, k, v, out, n_q, n_kv, T, D,
                             sm_scale, stream, window_size, true);
}

int fa_workspace_reserve(int max_tokens, int max_M, int max_K, int min_group_size, void* stream) {
    const char* fn = "fa_workspace_reserve";
    g_err.clear();
    if (max_tokens < 0 || max_M < 0 || max_K <= 0)
        return fail(FA_ERR_INVALID_ARG, "%s: bad sizes", fn);
    hipStream_t s = (hipStream_t)stream;
    const int g = eff_group(max_K, min_group_size);
    const int G = (max_K + g - 1) / g;
    Workspace* ws = nullptr;
    int rc = current_ws(&ws);
    if (rc) return rc;
    void* p = ws->xq;
    rc = grow(&p, &ws->xq_bytes, (size_t)max_tokens * (size_t)max_K, s);
    ws->xq = (int8_t*)p;
    if (rc) return rc;
    p = ws->xs;
    rc = grow(&p, &ws->xs_bytes, (size_t)max_tokens * (size_t)G * sizeof(float), s);
    ws->xs = (float*)p;
    if (rc) return rc;
    p = ws->st;
    rc = grow(&p, &ws->st_bytes, fa::gemm_pipe_tables_bytes(max_M, max_tokens, G), s);
    ws->st = (float*)p;
    if (rc) return rc;
    if (max_tokens > 16 && ws->sk_bytes == 0) {
        // prefill K split: a split launch has at most 2 workgroups per CU,
        // each with a 128 x 128 (or 256 x 128, one per CU) partial tile
        int dev = 0, cus = 0;
        FA_HIP(hipGetDevice(&dev));
        FA_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        const size_t need = kSplitCounters * sizeof(int) + (size_t)cus * 2 * 128 * 128 * 4;
        p = ws->sk;
        rc = grow(&p, &ws->sk_bytes, need, s);
        ws->sk = (int*)p;
        if (rc) return rc;
        FA_HIP(hipMemsetAsync(ws->sk, 0, kSplitCounters * sizeof(int), s));
    }
    if (max_tokens > 1) {   // fa_w8a8_gemm_swiglu's [N, 2F] linear output (max_M = 2F)
        p = ws->yt;
        rc = grow(&p, &ws->yt_bytes, (size_t)max_tokens * (size_t)max_M * 2, s);
        ws->yt = (uint16_t*)p;
        if (rc) return rc;
    }
    return FA_OK;
}

int fa_workspace_release(void) {
    g_err.clear();
    Workspace* ws = nullptr;
    int rc = current_ws(&ws);
    if (rc) return rc;
    FA_HIP(hipDeviceSynchronize());
    if (ws->xq) FA_HIP(hipFree(ws->xq));
    if (ws->xs) FA_HIP(hipFree(ws->xs));
    if (ws->st) FA_HIP(hipFree(ws->st));
    if (ws->yt) FA_HIP(hipFree(ws->yt));
    if (ws->sk) FA_HIP(hipFree(ws->sk));
    *ws = Workspace{};
    return FA_OK;
}

// ------------------------------------------------------------ chain ----

struct fa_chain {
    int dev = 0;
    fa::ch::ChainStepDev* d_steps = nullptr;
    int* d_sync = nullptr;
    int* d_flags = nullptr;
    fa::ChainPlan plan{};
};

static void chain_free(fa_chain* c) {
    if (!c) return;
    if (c->plan.trace) (void)hipFree(c->plan.trace);
    if (c->d_steps) (void)hipFree(c->d_steps);
    if (c->d_sync) (void)hipFree(c->d_sync);
    if (c->d_flags) (void)hipFree(c->d_flags);
    delete c;
}

int fa_chain_create(const fa_chain_step* steps, int n_steps, int group_size, fa_chain** out) {
    const char* fn = "fa_chain_create";
    g_err.clear();
    if (!out) return fail(FA_ERR_INVALID_ARG, "%s: null out", fn);
    *out = nullptr;
    if (!steps || n_steps <= 0 || n_steps > fa::kChainMaxSteps)
        return fail(FA_ERR_INVALID_ARG, "%s: bad steps / n_steps=%d", fn, n_steps);
    if (group_size != 64 && group_size != 128 && group_size != 256)
        return fail(FA_ERR_INVALID_ARG, "%s: group_size=%d (64, 128 or 256)", fn, group_size);
    const int g = group_size;
    const int lg = g == 64 ? 6 : g == 128 ? 7 : 8;
    const int kmax = fa::chain_max_k();
    std::vector<fa::ch::ChainStepDev> h((size_t)n_steps);
    int kp_max = 16, g_pad = 4, kh = 0;
    int64_t term_floats = 0;
    for (int i = 0; i < n_steps; ++i) {
        const fa_chain_step& c = steps[i];
        if (!c.w || !c.w_scale || !c.x || !c.y)
            return fail(FA_ERR_INVALID_ARG, "%s: step %d: null pointer", fn, i);
        if (c.m <= 0 || c.m > (1 << 29) || c.k < 16 || c.k > kmax || c.k % 16 != 0 || g > c.k)
            return fail(FA_ERR_INVALID_ARG,
                        "%s: step %d: m=%d k=%d (k a multiple of 16 in [group_size, %d])", fn, i,
                        c.m, c.k, kmax);
        if (c.prologue != 0 && c.prologue != 2)
            return fail(FA_ERR_INVALID_ARG, "%s: step %d: prologue %d (0 or 2)", fn, i, c.prologue);
        if (c.epilogue != 0 && c.epilogue != 1)
            return fail(FA_ERR_INVALID_ARG, "%s: step %d: epilogue %d (0 or 1)", fn, i, c.epilogue);
        if (c.epilogue == 1 && (c.m & 1))
            return fail(FA_ERR_INVALID_ARG, "%s: step %d: SwiGLU epilogue needs even m", fn, i);
        if (c.prologue == 2 && !c.gamma)
            return fail(FA_ERR_INVALID_ARG, "%s: step %d: prologue 2 needs gamma", fn, i);
        if (c.prologue == 2 && c.k > fa::chain_max_k_pro())
            return fail(FA_ERR_INVALID_ARG, "%s: step %d: prologue 2 takes k <= %d", fn, i,
                        fa::chain_max_k_pro());
        if (c.prologue == 0 && (c.x2 || c.gamma || c.h_out))
            return fail(FA_ERR_INVALID_ARG, "%s: step %d: x2 / gamma / h_out need prologue 2", fn,
                        i);
        const int G = (c.k + g - 1) / g;
        if ((int64_t)c.m * G < 2)
            return fail(FA_ERR_INVALID_ARG, "%s: step %d: fewer than two weight scales", fn, i);
        if ((int64_t)c.m * c.k >= ((int64_t)1 << 31))
            return fail(FA_ERR_INVALID_ARG, "%s: step %d: weight of 2^31 bytes or more", fn, i);
        if (!aligned16(c.w) || !aligned16(c.x) || (c.x2 && !aligned16(c.x2)) ||
            (c.gamma && !aligned16(c.gamma)) || (c.h_out && !aligned16(c.h_out)) ||
            ((uintptr_t)c.y & 1) || ((uintptr_t)c.w_scale & 3))
            return fail(FA_ERR_INVALID_ARG, "%s: step %d: misaligned pointer", fn, i);
        const size_t k = (size_t)c.k;
        const size_t ny = c.epilogue == 1 ? (size_t)c.m / 2 : (size_t)c.m;
        if (overlaps(c.y, ny, c.x, k) || overlaps(c.y, ny, c.x2, k) ||
            overlaps(c.y, ny, c.gamma, k) || overlaps(c.y, ny, c.h_out, k))
            return fail(FA_ERR_INVALID_ARG, "%s: step %d: y overlaps an input or h_out", fn, i);
        if (c.h_out && (overlaps(c.h_out, k, c.x, k) || overlaps(c.h_out, k, c.x2, k) ||
                        overlaps(c.h_out, k, c.gamma, k)))
            return fail(FA_ERR_INVALID_ARG, "%s: step %d: h_out overlaps an input", fn, i);
        fa::ch::ChainStepDev& d = h[(size_t)i];
        d.W = c.w;
        d.w_scale = c.w_scale;
        d.X = c.x;
        d.x2 = c.x2;
        d.gamma = c.gamma;
        d.h_out = c.h_out;
        d.Y = c.y;
        d.M = c.m;
        d.K = c.k;
        d.lg_g = lg;
        d.G = G;
        d.MG = (int64_t)c.m * G;
        d.passes = (c.k + 511) / 512;
        d.pro = c.prologue;
        d.epi = c.epilogue;
        d.eps = c.eps;
        kp_max = c.k > kp_max ? c.k : kp_max;
        g_pad = G > g_pad ? G : g_pad;
        if (c.prologue == 2) kh = c.k > kh ? c.k : kh;
    }
    const int cus = fa::chain_cus();
    if (cus <= 0) return fail(FA_ERR_HIP, "%s: device query failed", fn);
    for (const fa::ch::ChainStepDev& d : h) {
        // a workgroup's term table: 2 rows per pair, at most ceil(pairs / cus) pairs
        const int64_t pairs = ((int64_t)d.M + 1) / 2;
        const int64_t tf = 2 * ((pairs + cus - 1) / cus) * d.G;
        term_floats = tf > term_floats ? tf : term_floats;
    }
    if (term_floats > (1 << 20)) return fail(FA_ERR_INVALID_ARG, "%s: steps too large", fn);
    const fa::ch::ChainLds l8 = fa::chain_lds(8, kp_max, kh, g_pad, (int)term_floats);
    const int depth = fa::chain_depth_for(l8.total);
    const fa::ch::ChainLds lay = fa::chain_lds(depth, kp_max, kh, g_pad, (int)term_floats);
    if (lay.total > 160 * 1024)
        return fail(FA_ERR_INVALID_ARG, "%s: steps need %d B of LDS", fn, lay.total);
    const int grid = fa::chain_grid(lg, depth, (size_t)lay.total);
    if (grid < cus) return fail(FA_ERR_HIP, "%s: occupancy query failed (grid %d)", fn, grid);
    fa_chain* c = new fa_chain();
    if (hipGetDevice(&c->dev) != hipSuccess ||
        hipMalloc((void**)&c->d_steps, h.size() * sizeof(h[0])) != hipSuccess ||
        hipMalloc((void**)&c->d_sync, (size_t)(n_steps + 2) * sizeof(int)) != hipSuccess ||
        hipMemcpy(c->d_steps, h.data(), h.size() * sizeof(h[0]), hipMemcpyHostToDevice) !=
            hipSuccess ||
        hipMemset(c->d_sync, 0, (size_t)(n_steps + 2) * sizeof(int)) != hipSuccess ||
        hipMalloc((void**)&c->d_flags, (size_t)n_steps * 8 * 32 * sizeof(int)) != hipSuccess ||
        hipMemset(c->d_flags, 0, (size_t)n_steps * 8 * 32 * sizeof(int)) != hipSuccess) {
        chain_free(c);
        return fail(FA_ERR_HIP, "%s: device allocation / upload failed", fn);
    }
    c->plan.steps = c->d_steps;
    c->plan.sync = c->d_sync;
    c->plan.flags = c->d_flags;
    c->plan.nsteps = n_steps;
    c->plan.lg = lg;
    c->plan.grid = cus;   // one workgroup per CU (the term tables are sized for it)
    c->plan.spin_limit = 1 << 21;
    c->plan.depth = depth;
    c->plan.lay = lay;
    c->plan.trace = nullptr;
#ifdef FA_CHAIN_TRACE
    if (hipMalloc((void**)&c->plan.trace, (size_t)(n_steps + 1) * cus * 8 * 8) != hipSuccess) {
        chain_free(c);
        return fail(FA_ERR_HIP, "%s: trace allocation failed", fn);
    }
#endif
    *out = c;
    return FA_OK;
}

int fa_chain_run(fa_chain* chain, void* stream) {
    const char* fn = "fa_chain_run";
    g_err.clear();
    if (!chain) return fail(FA_ERR_INVALID_ARG, "%s: null chain", fn);
    int dev = 0;
    FA_HIP(hipGetDevice(&dev));
    if (dev != chain->dev)
        return fail(FA_ERR_INVALID_ARG, "%s: chain lives on device %d, current is %d", fn,
                    chain->dev, dev);
    FA_HIP(fa::launch_chain(chain->plan, (hipStream_t)stream));
    return FA_OK;
}

int fa_chain_status(fa_chain* chain, void* stream) {
    const char* fn = "fa_chain_status";
    g_err.clear();
    if (!chain) return fail(FA_ERR_INVALID_ARG, "%s: null chain", fn);
    FA_HIP(hipStreamSynchronize((hipStream_t)stream));
    int e = 0;
    FA_HIP(hipMemcpy(&e, chain->d_sync + chain->plan.nsteps, sizeof(int),
                     hipMemcpyDeviceToHost));
    if (e != 0) return fail(FA_ERR_HIP, "%s: a step's wait for its predecessor gave up", fn);
    return FA_OK;
}

int fa_chain_set_spin_limit(fa_chain* chain, int polls) {
    g_err.clear();
    if (!chain || polls < 0)
        return fail(FA_ERR_INVALID_ARG, "fa_chain_set_spin_limit: bad chain / polls");
    chain->plan.spin_limit = polls;
    return FA_OK;
}

#ifdef FA_CHAIN_TRACE
// measurement builds only: copy the last run's per-step timestamps
int fa_chain_trace(fa_chain* chain, void* host, size_t bytes) {
    if (!chain || !chain->plan.trace) return FA_ERR_INVALID_ARG;
    FA_HIP(hipDeviceSynchronize());
    FA_HIP(hipMemcpy(host, chain->plan.trace, bytes, hipMemcpyDeviceToHost));
    return FA_OK;
}
#endif

int fa_chain_destroy(fa_chain* chain) {
    g_err.clear();
    if (!chain) return FA_OK;
    (void)hipDeviceSynchronize();
    chain_free(chain);
    return FA_OK;
}

}  // extern "C"
