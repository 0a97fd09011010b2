// C ABI of librwkv7m_wkv.so (declared in include/rwkv7m_wkv.h).
//
// Validates every request before any launch (errors, never undefined
// behaviour: the reference's dispatcher validates at
// src/rwkv7m/model/wkv.py:19-57 and the native layer re-checks), then routes
// it to the chunked MFMA kernels, the single-token kernel or the sequential
// kernels.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <initializer_list>
#include <mutex>
#include <string>

#include "../../include/rwkv7m_screening.h"
#include "../../include/rwkv7m_timemix.h"
#include "../../include/rwkv7m_wkv.h"
#include "wkv7_launch.h"

namespace {

thread_local std::string g_last_error;
// The kernel the last successful WKV-7 call on this thread launched.
thread_local const char* g_last_path = "";

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

bool supported_n(int64_t n) {
    return n == 1 || n == 2 || n == 4 || n == 8 || n == 16 || n == 32 ||
           n == 64 || n == 128;
}

// Copy or clear n floats on the stream with a plain kernel (no memset nodes,
// so a caller may capture these calls in a HIP graph).
__global__ void fill_kernel(float* dst, const float* src, int64_t n) {
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += int64_t(gridDim.x) * blockDim.x)
        dst[i] = src ? src[i] : 0.f;
}

int copy_or_clear(float* dst, const float* src, int64_t n,
                  hipStream_t stream) {
    if (n == 0 || dst == src) return RWKV7M_OK;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(fill_kernel, dim3(unsigned(blocks)), dim3(256), 0,
                       stream, dst, src, n);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail(RWKV7M_ERR_HIP,
                    std::string("fill kernel launch failed: ") +
                        hipGetErrorString(e));
    return RWKV7M_OK;
}

struct Dims {
    int64_t T, B, H, N, vec_elems, state_elems;
};

int check_dims(const char* fn, int dtype, int64_t T, int64_t B, int64_t H,
               int64_t N, Dims* out) {
    const std::string f(fn);
    if (dtype != RWKV7M_DTYPE_F32 && dtype != RWKV7M_DTYPE_BF16)
        return fail(RWKV7M_ERR_INVALID_ARGUMENT,
                    f + ": WKV vectors must be bfloat16 or float32 (dtype=" +
                        std::to_string(dtype) + ")");
    if (T < 0 || B < 0 || H < 0 || N < 0)
        return fail(RWKV7M_ERR_INVALID_ARGUMENT,
                    f + ": negative dimension");
    if (!supported_n(N))
        return fail(RWKV7M_ERR_UNSUPPORTED,
                    f + ": head size N=" + std::to_string(N) +
                        " is not supported (1, 2, 4, ..., 128)");
    const int64_t lim = int64_t(1) << 40;
    if (B > lim || H > lim || T > lim || B * H > 0x7fffffff ||
        (B * H > 0 && T > (int64_t(1) << 46) / (B * H * N)))
        return fail(RWKV7M_ERR_INVALID_ARGUMENT, f + ": sizes too large");
    out->T = T;
    out->B = B;
    out->H = H;
    out->N = N;
    out->vec_elems = T * B * H * N;
    out->state_elems = B * H * N * N;
    return RWKV7M_OK;
}

int need(const void* p, bool nonempty, const char* fn, const char* name) {
    if (nonempty && p == nullptr)
        return fail(RWKV7M_ERR_INVALID_ARGUMENT,
                    std::string(fn) + ": " + name + " is NULL");
    return RWKV7M_OK;
}

#define RWKV7M_TRY(expr)              \
    do {                              \
        int rc_ = (expr);             \
        if (rc_ != RWKV7M_OK) return rc_; \
    } while (0)

int hip_status(const char* what, hipError_t e) {
    if (e == hipSuccess) return RWKV7M_OK;
    return fail(RWKV7M_ERR_HIP, std::string(what) + ": " +
                                    hipGetErrorString(e));
}

// Chunk length of the MFMA forward without checkpoints (16: the
// wave-per-chunk kernel), and the default checkpoint interval: a checkpoint
// per 16-token chunk, so that the MFMA backward recomputes no forward state
// (the fastest training step of the intervals 16, 32 and 64 measured on
// MI355X; the sequential kernels use the same default).
constexpr int64_t kDefaultChunk = 16;
constexpr int64_t kDefaultTrainChunk = 16;

int64_t default_interval(int, int64_t) { return kDefaultTrainChunk; }

// Checkpoints are bf16 for the intervals of the bf16 N = 64 training path
// (the MFMA kernels read them only as bf16 operands); the sequential kernels
// read and write either type, so the choice does not depend on alignment.
bool ckpt_bf16(int dtype, int64_t N, int64_t ci) {
    return dtype == RWKV7M_DTYPE_BF16 && N == 64 &&
           (ci == 16 || ci == 32 || ci == 64);
}

bool aligned16(const void* p) {
    return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// Token vectors' layout: time-major [T][B][H][N] (the reference's) or
// batch-major [B][T][H][N].
rwkv7m::VecLayout vec_layout(bool batch_major, int64_t T, int64_t B,
                             int64_t H, int64_t N) {
    rwkv7m::VecLayout l;
    l.H = H;
    if (batch_major) {
        l.ts = H * N;
        l.bs = T * H * N;
    } else {
        l.ts = B * H * N;
        l.bs = H * N;
    }
    (void)B;
    return l;
}

// Whether the byte ranges [a, a + abytes) and [b, b + bbytes) share a byte
// (a NULL pointer or an empty range shares none).
bool overlaps(const void* a, int64_t abytes, const void* b, int64_t bbytes) {
    if (!a || !b || abytes <= 0 || bbytes <= 0) return false;
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(a);
    const uintptr_t b0 = reinterpret_cast<uintptr_t>(b);
    return a0 < b0 + uintptr_t(bbytes) && b0 < a0 + uintptr_t(abytes);
}

bool all_aligned16(std::initializer_list<const void*> ptrs) {
    for (const void* p : ptrs)
        if (p && !aligned16(p)) return false;
    return true;
}

// The MFMA kernels (16-token chunks) serve bf16 vectors with N = 64, a
// checkpoint interval of 16, 32 or 64, 16-byte aligned buffers, chunks whose
// element span 16 * (token stride) stays below 2^31 (32-bit lane offsets)
// and fewer than 2^31 chunks.
bool use_chunked(int dtype, int64_t N, int64_t ci, int64_t T,
                 int64_t token_stride,
                 std::initializer_list<const void*> ptrs) {
    if (dtype != RWKV7M_DTYPE_BF16 || N != 64) return false;
    if (ci != 16 && ci != 32 && ci != 64) return false;
    if (token_stride * 64 >= (int64_t(1) << 31)) return false;
    if (T / 16 >= (int64_t(1) << 31) - 1) return false;
    return all_aligned16(ptrs);
}

int forward_impl(const char* fn, int dtype, int64_t T, int64_t B, int64_t H,
                 int64_t N, const void* r, const void* w, const void* k,
                 const void* v, const void* a, const void* b,
                 const float* s0, void* y, float* s_t, void* ckpt,
                 int64_t ci, hipStream_t stream, bool batch_major) {
    g_last_path = "";
    Dims d;
    RWKV7M_TRY(check_dims(fn, dtype, T, B, H, N, &d));
    const bool vecs = d.vec_elems > 0, st = d.state_elems > 0;
    RWKV7M_TRY(need(r, vecs, fn, "r"));
    RWKV7M_TRY(need(w, vecs, fn, "w"));
    RWKV7M_TRY(need(k, vecs, fn, "k"));
    RWKV7M_TRY(need(v, vecs, fn, "v"));
    RWKV7M_TRY(need(a, vecs, fn, "neg_kk"));
    RWKV7M_TRY(need(b, vecs, fn, "kka"));
    RWKV7M_TRY(need(y, vecs, fn, "y"));
    RWKV7M_TRY(need(s0, st, fn, "initial_state"));
    RWKV7M_TRY(need(s_t, st, fn, "final_state"));
    if (d.state_elems == 0) return RWKV7M_OK;
    if (T == 0 && !ckpt) return copy_or_clear(s_t, s0, d.state_elems, stream);
    const int64_t L = ckpt ? ci : kDefaultChunk;
    const rwkv7m::VecLayout lay = vec_layout(batch_major, T, B, H, N);
    if (T > 1 && use_chunked(dtype, N, L, T, lay.ts,
                             {r, w, k, v, a, b, y, s0, s_t, ckpt})) {
        rwkv7m::ChunkFwdArgs c{};
        c.L = int(L);
        c.T = T;
        c.B = B;
        c.H = H;
        c.lay = lay;
        c.r = r;
        c.w = w;
        c.k = k;
        c.v = v;
        c.a = a;
        c.b = b;
        c.s0 = s0;
        c.y = y;
        c.s_t = s_t;
        c.ckpt = ckpt;
        RWKV7M_TRY(hip_status("device wait configuration",
                              rwkv7m::wait_config(&c.wait)));
        g_last_path = "wave_forward";
        return hip_status("chunked forward launch",
                          rwkv7m::launch_wave_forward(c, stream));
    }
    rwkv7m::SeqFwdArgs p{};
    p.bf16 = dtype == RWKV7M_DTYPE_BF16;
    p.T = T;
    p.B = B;
    p.H = H;
    p.N = N;
    p.lay = lay;
    p.r = r;
    p.w = w;
    p.k = k;
    p.v = v;
    p.a = a;
    p.b = b;
    p.s0 = s0;
    p.y = y;
    p.s_t = s_t;
    p.ckpt = ckpt;
    p.ckpt_bf16 = ckpt_bf16(dtype, N, ci);
    p.ci = ci;
    if (T == 1 && !ckpt && N == 64 &&
        all_aligned16({r, w, k, v, a, b, y, s0, s_t})) {
        g_last_path = "decode";
        return hip_status("decode launch", rwkv7m::launch_decode(p, stream));
    }
    g_last_path = "seq_forward";
    return hip_status("sequential forward launch",
                      rwkv7m::launch_seq_forward(p, stream));
}

int backward_impl(const char* fn, int dtype, int64_t T, int64_t B, int64_t H,
                         int64_t N, const void* r, const void* w,
                         const void* k, const void* v, const void* neg_kk,
                         const void* kka, const float* initial_state,
                         const void* dy, const float* ds_t,
                         const void* checkpoints,
                         int64_t checkpoint_interval, void* dr, void* dw,
                         void* dk, void* dv, void* dneg_kk, void* dkka,
                         float* ds0, hipStream_t s, bool batch_major,
                         const void* add_dr = nullptr,
                         const void* add_dk = nullptr,
                         const void* add_dv = nullptr) {
    (void)initial_state;  // checkpoints[0] holds it
    g_last_path = "";
    Dims d;
    RWKV7M_TRY(check_dims(fn, dtype, T, B, H, N, &d));
    if (checkpoint_interval < 0)
        return fail(RWKV7M_ERR_INVALID_ARGUMENT,
                    std::string(fn) + ": checkpoint_interval must be >= 0");
    const int64_t ci = checkpoint_interval == 0
                           ? default_interval(dtype, N)
                           : checkpoint_interval;
    const bool vecs = d.vec_elems > 0, st = d.state_elems > 0;
    RWKV7M_TRY(need(r, vecs, fn, "r"));
    RWKV7M_TRY(need(w, vecs, fn, "w"));
    RWKV7M_TRY(need(k, vecs, fn, "k"));
    RWKV7M_TRY(need(v, vecs, fn, "v"));
    RWKV7M_TRY(need(neg_kk, vecs, fn, "neg_kk"));
    RWKV7M_TRY(need(kka, vecs, fn, "kka"));
    RWKV7M_TRY(need(dr, vecs, fn, "dr"));
    RWKV7M_TRY(need(dw, vecs, fn, "dw"));
    RWKV7M_TRY(need(dk, vecs, fn, "dk"));
    RWKV7M_TRY(need(dv, vecs, fn, "dv"));
    RWKV7M_TRY(need(dneg_kk, vecs, fn, "dneg_kk"));
    RWKV7M_TRY(need(dkka, vecs, fn, "dkka"));
    RWKV7M_TRY(need(ds0, st, fn, "ds0"));
    RWKV7M_TRY(need(checkpoints, vecs, fn, "checkpoints"));
    // an added cotangent is read while the gradients are written: it may
    // not share a byte with an output buffer (a head handed to the exact
    // pass is written twice, and its second pass reads the cotangent again)
    const int64_t vbytes =
        d.vec_elems * (dtype == RWKV7M_DTYPE_BF16 ? 2 : 4);
    for (const void* a : {add_dr, add_dk, add_dv})
        for (const void* o : {dr, dw, dk, dv, dneg_kk, dkka})
            if (overlaps(a, vbytes, o, vbytes))
                return fail(RWKV7M_ERR_INVALID_ARGUMENT,
                            std::string(fn) +
                                ": an added cotangent may not overlap an "
                                "output buffer");
    // dS_T is read again by the exact pass of a head whose dS0 already holds
    // the pass's mark: dS0 may not share a byte with it
    const int64_t sbytes = d.state_elems * 4;
    if (overlaps(ds0, sbytes, ds_t, sbytes))
        return fail(RWKV7M_ERR_INVALID_ARGUMENT,
                    std::string(fn) + ": ds0 may not overlap ds_t");
    if (d.state_elems == 0) return RWKV7M_OK;
    if (T == 0) return copy_or_clear(ds0, ds_t, d.state_elems, s);
    const rwkv7m::VecLayout lay = vec_layout(batch_major, T, B, H, N);
    rwkv7m::SeqBwdArgs p{};
    p.bf16 = dtype == RWKV7M_DTYPE_BF16;
    p.T = T;
    p.B = B;
    p.H = H;
    p.N = N;
    p.lay = lay;
    p.r = r;
    p.w = w;
    p.k = k;
    p.v = v;
    p.a = neg_kk;
    p.b = kka;
    p.dy = dy;
    p.ds_t = ds_t;
    p.ckpt = checkpoints;
    p.ckpt_bf16 = ckpt_bf16(dtype, N, ci);
    p.ci = ci;
    p.dr = dr;
    p.dw = dw;
    p.dk = dk;
    p.dv = dv;
    p.da = dneg_kk;
    p.db = dkka;
    p.ds0 = ds0;
    p.add_dr = add_dr;
    p.add_dk = add_dk;
    p.add_dv = add_dv;
    // the wave backward addresses vectors and checkpoints with 32-bit byte
    // offsets below 2^31
    const int64_t nck = (T + ci - 1) / ci + 1;
    const bool small = d.vec_elems * 2 < (int64_t(1) << 31) &&
                       nck * B * H * N * N * 2 < (int64_t(1) << 31);
    if (small &&
        use_chunked(dtype, N, ci, T, lay.ts,
                    {r, w, k, v, neg_kk, kka, dy, ds_t, checkpoints, dr, dw,
                     dk, dv, dneg_kk, dkka, ds0, add_dr, add_dk, add_dv})) {
        rwkv7m::WaveBwdArgs c{};
        c.L = int(ci);
        c.T = T;
        c.B = B;
        c.H = H;
        c.lay = lay;
        c.r = r;
        c.w = w;
        c.k = k;
        c.v = v;
        c.a = neg_kk;
        c.b = kka;
        c.dy = dy;
        c.ds_t = ds_t;
        c.ckpt = checkpoints;
        c.dr = dr;
        c.dw = dw;
        c.dk = dk;
        c.dv = dv;
        c.da = dneg_kk;
        c.db = dkka;
        c.ds0 = ds0;
        c.add_dr = add_dr;
        c.add_dk = add_dk;
        c.add_dv = add_dv;
        RWKV7M_TRY(hip_status("device wait configuration",
                              rwkv7m::wait_config(&c.wait)));
        RWKV7M_TRY(hip_status("wave backward launch",
                              rwkv7m::launch_wave_backward(c, s)));
        // heads with a chunk outside the factored form's range were left to
        // the exact sequential pass (marked in dS0); every other head
        // returns at once
        p.marked_only = true;
        g_last_path = "wave_backward";
        return hip_status("exact pass launch",
                          rwkv7m::launch_seq_backward(p, s));
    }
    g_last_path = "seq_backward";
    return hip_status("sequential backward launch",
                      rwkv7m::launch_seq_backward(p, s));
}

int forward_aux_impl(const char* fn, int dtype, int64_t T, int64_t B,
                     int64_t H, int64_t N, const void* r, const void* w,
                     const void* k, const void* v, const void* neg_kk,
                     const void* kka, const float* initial_state, void* y,
                     float* final_state, void* checkpoints,
                     int64_t checkpoint_interval, hipStream_t stream,
                     bool batch_major) {
    if (checkpoint_interval < 0)
        return fail(RWKV7M_ERR_INVALID_ARGUMENT,
                    std::string(fn) + ": checkpoint_interval must be >= 0");
    const int64_t ci = checkpoint_interval == 0
                           ? default_interval(dtype, N)
                           : checkpoint_interval;
    RWKV7M_TRY(need(checkpoints, B * H * N > 0, fn, "checkpoints"));
    return forward_impl(fn, dtype, T, B, H, N, r, w, k, v, neg_kk, kka,
                        initial_state, y, final_state, checkpoints, ci, stream,
                        batch_major);
}


// ---------------------------------------------------------------------------
// Fused time-mix producers and consumer (include/rwkv7m_timemix.h)
// ---------------------------------------------------------------------------

struct TmDims {
    int64_t rows, C, N;
};

int tm_check(const char* fn, int dtype, int64_t rows, int64_t H, int64_t N,
             TmDims* d) {
    const std::string f(fn);
    if (dtype != RWKV7M_DTYPE_F32 && dtype != RWKV7M_DTYPE_BF16)
        return fail(RWKV7M_ERR_INVALID_ARGUMENT,
                    f + ": activations must be bfloat16 or float32 (dtype=" +
                        std::to_string(dtype) + ")");
    if (rows < 0 || H < 0 || N < 0)
        return fail(RWKV7M_ERR_INVALID_ARGUMENT, f + ": negative dimension");
    if (N != 8 && N != 16 && N != 32 && N != 64 && N != 128)
        return fail(RWKV7M_ERR_UNSUPPORTED,
                    f + ": head size N=" + std::to_string(N) +
                        " is not supported (8, 16, 32, 64, 128)");
    if (H > 0x7fffffff / N)
        return fail(RWKV7M_ERR_INVALID_ARGUMENT, f + ": sizes too large");
    d->rows = rows;
    d->N = N;
    d->C = H * N;
    if (d->C > 0 && rows > (int64_t(1) << 46) / d->C)
        return fail(RWKV7M_ERR_INVALID_ARGUMENT, f + ": sizes too large");
    return RWKV7M_OK;
}

struct Named {
    const char* name;
    const void* p;
};

// Each pointer is required (non-NULL) and 16-byte aligned.
int tm_need(const char* fn, std::initializer_list<Named> ptrs) {
    for (const Named& x : ptrs) {
        if (x.p == nullptr)
            return fail(RWKV7M_ERR_INVALID_ARGUMENT,
                        std::string(fn) + ": " + x.name + " is NULL");
        if (!aligned16(x.p))
            return fail(RWKV7M_ERR_INVALID_ARGUMENT,
                        std::string(fn) + ": " + x.name +
                            " is not 16-byte aligned");
    }
    return RWKV7M_OK;
}

int tm_eps(const char* fn, double eps) {
    if (!(eps >= 0.0) || !std::isfinite(eps))
        return fail(RWKV7M_ERR_INVALID_ARGUMENT,
                    std::string(fn) + ": eps must be finite and >= 0");
    return RWKV7M_OK;
}

int tm_workspace(const char* fn, const TmDims& d, const float* ws,
                 int64_t ws_floats) {
    const int64_t need_floats = rwkv7m::timemix_workspace_floats(d.rows, d.C);
    if (ws_floats < need_floats)
        return fail(RWKV7M_ERR_INVALID_ARGUMENT,
                    std::string(fn) + ": workspace holds " +
                        std::to_string(ws_floats) + " floats, needs " +
                        std::to_string(need_floats));
    return tm_need(fn, {{"workspace", ws}});
}

// ---------------------------------------------------------------------------
// Screening read path (include/rwkv7m_screening.h)
// ---------------------------------------------------------------------------

int sc_dims(const char* fn, int dtype, int64_t B, int64_t T, int64_t M,
            int64_t a, int64_t b) {
    const std::string f(fn);
    if (dtype != RWKV7M_DTYPE_F32 && dtype != RWKV7M_DTYPE_BF16)
        return fail(RWKV7M_ERR_INVALID_ARGUMENT,
                    f + ": activations must be bfloat16 or float32 (dtype=" +
                        std::to_string(dtype) + ")");
    if (B < 0 || T < 0 || M < 0 || a < 0 || b < 0)
        return fail(RWKV7M_ERR_INVALID_ARGUMENT, f + ": negative dimension");
    const int64_t lim = int64_t(1) << 20;
    if (B > lim || T > lim || M > lim || a > lim || b > lim ||
        B * T * (M > 0 ? M : 1) > (int64_t(1) << 31) ||
        B * T * (M > 0 ? M : 1) * (a + b) > (int64_t(1) << 44))
        return fail(RWKV7M_ERR_INVALID_ARGUMENT, f + ": sizes too large");
    return RWKV7M_OK;
}

int sc_need(const char* fn, std::initializer_list<Named> ptrs) {
    for (const Named& x : ptrs)
        if (x.p == nullptr)
            return fail(RWKV7M_ERR_INVALID_ARGUMENT,
                        std::string(fn) + ": " + x.name + " is NULL");
    return RWKV7M_OK;
}

int sc_workspace(const char* fn, int64_t B, int64_t T, int64_t M,
                 int64_t ds, int64_t have) {
    const int64_t need_floats =
        rwkv7m::screen_scan_workspace_floats(B, T, M, ds);
    if (have < need_floats)
        return fail(RWKV7M_ERR_INVALID_ARGUMENT,
                    std::string(fn) + ": workspace holds " +
                        std::to_string(have) + " floats, needs " +
                        std::to_string(need_floats));
    return RWKV7M_OK;
}

int sc_read_checks(const char* fn, int64_t M, int64_t dk, int64_t dv,
                   double trim_eps, double cap, double eps, double alpha,
                   double gamma) {
    const std::string f(fn);
    if (M > 64 || dk > 128 || dv > 512)
        return fail(RWKV7M_ERR_UNSUPPORTED,
                    f + ": supported sizes are M <= 64, dk <= 128, dv <= 512");
    if (!(trim_eps >= 0.0) || !(eps >= 0.0) || !std::isfinite(eps) ||
        !std::isfinite(trim_eps))
        return fail(RWKV7M_ERR_INVALID_ARGUMENT,
                    f + ": eps must be finite and >= 0");
    if (!(cap > 0.0) || !std::isfinite(cap))
        return fail(RWKV7M_ERR_INVALID_ARGUMENT,
                    f + ": cap must be finite and > 0");
    if (!std::isfinite(alpha) || !std::isfinite(gamma))
        return fail(RWKV7M_ERR_INVALID_ARGUMENT,
                    f + ": leaky_alpha and leaky_gamma must be finite");
    return RWKV7M_OK;
}

rwkv7m::ScreenReadArgs sc_read_args(int64_t B, int64_t T, int64_t M,
                                    int64_t dk, int64_t dv, const float* q,
                                    const void* proj, const float* tau,
                                    double trim_eps, const float* age_w,
                                    int age_per_step, int value_unit_norm,
                                    int leaky,
                                    double alpha, double gamma, double cap,
                                    double eps) {
    rwkv7m::ScreenReadArgs A{};
    A.B = B;
    A.T = T;
    A.M = int(M);
    A.dk = int(dk);
    A.dv = int(dv);
    A.q = q;
    A.proj = proj;
    A.tau = tau;
    A.trim_eps = float(trim_eps);
    A.age_w = age_w;
    A.age_bstride = age_per_step ? T * M : M;
    A.age_tstride = age_per_step ? M : 0;
    A.value_unit_norm = value_unit_norm != 0;
    A.leaky = leaky != 0;
    A.leaky_alpha = float(alpha);
    A.leaky_gamma = float(gamma);
    A.cap = float(cap);
    A.eps = float(eps);
    return A;
}

int sc_write_checks(const char* fn, int dtype, int64_t B, int64_t T,
                    int64_t M, int64_t ds, int64_t dk, double floor,
                    double eps) {
    RWKV7M_TRY(sc_dims(fn, dtype, B, T, M, ds, dk));
    if (ds > 1024 || dk > 128 || dk < 1)
        return fail(RWKV7M_ERR_UNSUPPORTED,
                    std::string(fn) +
                        ": supported sizes are ds <= 1024, 1 <= dk <= 128");
    if (!(floor >= 0.0) || !std::isfinite(floor) || !(eps >= 0.0) ||
        !std::isfinite(eps))
        return fail(RWKV7M_ERR_INVALID_ARGUMENT,
                    std::string(fn) + ": floor and eps must be finite, >= 0");
    return RWKV7M_OK;
}

rwkv7m::ScreenWriteArgs sc_write_args(int64_t B, int64_t T, int64_t M,
                                      int64_t ds, int64_t dk,
                                      const void* base, const float* st,
                                      const float* se, const float* kw,
                                      const float* q_w, const float* tau_w,
                                      const float* mu, double floor,
                                      double eps) {
    rwkv7m::ScreenWriteArgs A{};
    A.B = B;
    A.T = T;
    A.M = M;
    A.ds = ds;
    A.dk = int(dk);
    A.base = base;
    A.slot_term = st;
    A.slot_embed = se;
    A.kw = kw;
    A.q_w = q_w;
    A.tau_w = tau_w;
    A.mu = mu;
    A.floor = float(floor);
    A.eps = float(eps);
    return A;
}

}  // namespace

namespace {

// Built-in scratch of the no-allocation consumer backward: the parameter
// gradients' partial rows (3 parameters x row groups x C floats).  The
// geometry keeps row groups x column tiles <= 1024 and a column tile is 2048
// channels, so 3 * 1024 * 2048 floats (24 MiB) serve every C up to
// 2048 * 1024 channels.  Each device holds its own copy for the life of the
// process.  Host code never uses this name as an address: the device
// address comes from hipGetSymbolAddress, looked up once per device with
// that device current.
constexpr int64_t kScratchFloats = int64_t(3) * 1024 * 2048;
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kScratchDevices];

// The current device's address of `scratch` (looked up on first use).
int scratch_address(const char* fn, float** out) {
    int dev = 0;
    RWKV7M_TRY(hip_status(fn, hipGetDevice(&dev)));
    if (dev < 0 || dev >= kScratchDevices)
        return fail(RWKV7M_ERR_UNSUPPORTED,
                    std::string(fn) + ": device index " + std::to_string(dev) +
                        " is beyond the " + std::to_string(kScratchDevices) +
                        " devices the built-in scratch tracks");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        // The lookup may load this code object onto the device.  A first
        // call made under stream capture in the global or thread-local mode
        // would have that refused as unsafe; this thread's capture mode is
        // relaxed for the lookup alone (it queues nothing on any stream)
        // and restored after it.
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        RWKV7M_TRY(hip_status(fn, hipThreadExchangeStreamCaptureMode(&mode)));
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        RWKV7M_TRY(hip_status(fn, hipThreadExchangeStreamCaptureMode(&mode)));
        if (e != hipSuccess || p == nullptr)
            return fail(RWKV7M_ERR_HIP,
                        std::string(fn) +
                            ": address of the built-in scratch: " +
                            hipGetErrorString(e));
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_ptr[dev];
    return RWKV7M_OK;
}

// The consumer backward's checks and launch; `workspace` is the caller's
// (checked against workspace_floats) or, with `builtin`, the device's
// built-in scratch.
int output_backward_impl(
    const char* fn, int dtype, int64_t rows, int64_t H, int64_t N,
    const void* y, const void* r, const void* k, const void* v, const void* g,
    const float* r_k, const float* ln_scale, const float* ln_bias, double eps,
    const void* dout, void* dy, void* dr, void* dk, void* dv, void* dg,
    float* dr_k, float* dln_scale, float* dln_bias, float* workspace,
    int64_t workspace_floats, bool builtin, hipStream_t stream) {
    TmDims d;
    RWKV7M_TRY(tm_check(fn, dtype, rows, H, N, &d));
    RWKV7M_TRY(tm_eps(fn, eps));
    if (d.C == 0) return RWKV7M_OK;
    RWKV7M_TRY(tm_need(fn, {{"r_k", r_k}, {"ln_scale", ln_scale},
                            {"ln_bias", ln_bias}, {"dr_k", dr_k},
                            {"dln_scale", dln_scale},
                            {"dln_bias", dln_bias}}));
    if (builtin) {
        const int64_t need_floats =
            rwkv7m::timemix_workspace_floats(d.rows, d.C);
        if (need_floats > kScratchFloats)
            return fail(RWKV7M_ERR_INVALID_ARGUMENT,
                        std::string(fn) + ": H*N = " + std::to_string(d.C) +
                            " channels need " + std::to_string(need_floats) +
                            " floats of scratch; the built-in scratch holds " +
                            std::to_string(kScratchFloats) +
                            " (use rwkv7m_timemix_wkv_output_backward with a "
                            "workspace)");
    } else {
        RWKV7M_TRY(tm_workspace(fn, d, workspace, workspace_floats));
    }
    if (d.rows > 0)
        RWKV7M_TRY(tm_need(fn, {{"y", y}, {"r", r}, {"k", k}, {"v", v},
                                {"g", g}, {"dout", dout}, {"dy", dy},
                                {"dr", dr}, {"dk", dk}, {"dv", dv},
                                {"dg", dg}}));
    if (builtin) RWKV7M_TRY(scratch_address(fn, &workspace));
    rwkv7m::TmOutputBwdArgs A{d.rows, d.C,     float(eps), y,   r,
                              k,      v,       g,          dout, r_k,
                              ln_scale, ln_bias, dy,       dr,   dk,
                              dv,     dg,      dr_k,       dln_scale,
                              dln_bias, workspace};
    return hip_status("time-mix consumer backward launch",
                      rwkv7m::launch_timemix_output_backward(
                          dtype == RWKV7M_DTYPE_BF16, int(d.N), A, stream));
}

}  // namespace

extern "C" {

int rwkv7m_abi_version(void) { return 1; }

const char* rwkv7m_last_error(void) { return g_last_error.c_str(); }

const char* rwkv7m_wkv7_last_path(void) { return g_last_path; }

int rwkv7m_device_status(void* stream) {
    g_last_error.clear();
    unsigned int n = 0;
    RWKV7M_TRY(hip_status("rwkv7m_device_status",
                          rwkv7m::take_wait_failures(
                              static_cast<hipStream_t>(stream), &n)));
    if (n != 0)
        return fail(RWKV7M_ERR_DEVICE,
                    "rwkv7m_device_status: " + std::to_string(n) +
                        " bounded wait(s) inside the kernels gave up; the "
                        "outputs of the affected (batch, head) pairs were "
                        "set to NaN");
    return RWKV7M_OK;
}

void rwkv7m_debug_set_wait_limit(int64_t polls) {
    rwkv7m::set_wait_limit(polls);
}

void rwkv7m_debug_set_backward_segments(int workgroups_per_head) {
    rwkv7m::set_backward_segments(workgroups_per_head);
}

void rwkv7m_debug_set_forward_segments(int workgroups_per_head) {
    rwkv7m::set_forward_segments(workgroups_per_head);
}

int64_t rwkv7m_wkv7_checkpoint_count(int64_t T, int64_t checkpoint_interval) {
    if (T < 0 || checkpoint_interval <= 0) return -1;
    return (T + checkpoint_interval - 1) / checkpoint_interval + 1;
}

int64_t rwkv7m_wkv7_default_checkpoint_interval(int dtype, int64_t N) {
    return default_interval(dtype, N);
}

int rwkv7m_wkv7_checkpoint_dtype(int dtype, int64_t N,
                                 int64_t checkpoint_interval) {
    const int64_t ci = checkpoint_interval == 0 ? default_interval(dtype, N)
                                                : checkpoint_interval;
    return ckpt_bf16(dtype, N, ci) ? RWKV7M_DTYPE_BF16 : RWKV7M_DTYPE_F32;
}

int rwkv7m_wkv7_forward(int dtype, int64_t T, int64_t B, int64_t H, int64_t N,
                        const void* r, const void* w, const void* k,
                        const void* v, const void* neg_kk, const void* kka,
                        const float* initial_state, void* y,
                        float* final_state, void* stream) {
    g_last_error.clear();
    return forward_impl("rwkv7m_wkv7_forward", dtype, T, B, H, N, r, w, k, v,
                        neg_kk, kka, initial_state, y, final_state, nullptr,
                        0, static_cast<hipStream_t>(stream), false);
}

int rwkv7m_wkv7_forward_bthn(int dtype, int64_t T, int64_t B, int64_t H,
                             int64_t N, const void* r, const void* w,
                             const void* k, const void* v, const void* neg_kk,
                             const void* kka, const float* initial_state,
                             void* y, float* final_state, void* stream) {
    g_last_error.clear();
    return forward_impl("rwkv7m_wkv7_forward_bthn", dtype, T, B, H, N, r, w,
                        k, v, neg_kk, kka, initial_state, y, final_state,
                        nullptr, 0, static_cast<hipStream_t>(stream), true);
}

int rwkv7m_wkv7_forward_with_aux(int dtype, int64_t T, int64_t B, int64_t H,
                                 int64_t N, const void* r, const void* w,
                                 const void* k, const void* v,
                                 const void* neg_kk, const void* kka,
                                 const float* initial_state, void* y,
                                 float* final_state, void* checkpoints,
                                 int64_t checkpoint_interval, void* stream) {
    g_last_error.clear();
    return forward_aux_impl("rwkv7m_wkv7_forward_with_aux", dtype, T, B, H, N,
                            r, w, k, v, neg_kk, kka, initial_state, y,
                            final_state, checkpoints, checkpoint_interval,
                            static_cast<hipStream_t>(stream), false);
}

int rwkv7m_wkv7_forward_with_aux_bthn(
    int dtype, int64_t T, int64_t B, int64_t H, int64_t N, const void* r,
    const void* w, const void* k, const void* v, const void* neg_kk,
    const void* kka, const float* initial_state, void* y, float* final_state,
    void* checkpoints, int64_t checkpoint_interval, void* stream) {
    g_last_error.clear();
    return forward_aux_impl("rwkv7m_wkv7_forward_with_aux_bthn", dtype, T, B,
                            H, N, r, w, k, v, neg_kk, kka, initial_state, y,
                            final_state, checkpoints, checkpoint_interval,
                            static_cast<hipStream_t>(stream), true);
}

int rwkv7m_wkv7_backward(int dtype, int64_t T, int64_t B, int64_t H,
                         int64_t N, const void* r, const void* w,
                         const void* k, const void* v, const void* neg_kk,
                         const void* kka, const float* initial_state,
                         const void* dy, const float* ds_t,
                         const void* checkpoints,
                         int64_t checkpoint_interval, void* dr, void* dw,
                         void* dk, void* dv, void* dneg_kk, void* dkka,
                         float* ds0, void* stream) {
    g_last_error.clear();
    return backward_impl("rwkv7m_wkv7_backward", dtype, T, B, H, N, r, w, k, v,
                         neg_kk, kka, initial_state, dy, ds_t, checkpoints,
                         checkpoint_interval, dr, dw, dk, dv, dneg_kk, dkka,
                         ds0, static_cast<hipStream_t>(stream), false);
}

int rwkv7m_wkv7_backward_bthn(int dtype, int64_t T, int64_t B, int64_t H,
                              int64_t N, const void* r, const void* w,
                              const void* k, const void* v, const void* neg_kk,
                              const void* kka, const float* initial_state,
                              const void* dy, const float* ds_t,
                              const void* checkpoints,
                              int64_t checkpoint_interval, void* dr, void* dw,
                              void* dk, void* dv, void* dneg_kk, void* dkka,
                              float* ds0, void* stream) {
    g_last_error.clear();
    return backward_impl("rwkv7m_wkv7_backward_bthn", dtype, T, B, H, N, r, w,
                         k, v, neg_kk, kka, initial_state, dy, ds_t,
                         checkpoints, checkpoint_interval, dr, dw, dk, dv,
                         dneg_kk, dkka, ds0, static_cast<hipStream_t>(stream),
                         true);
}

int rwkv7m_wkv7_decode_inplace(int dtype, int64_t B, int64_t H, int64_t N,
                               const void* r, const void* w, const void* k,
                               const void* v, const void* neg_kk,
                               const void* kka, float* state, void* y,
                               void* stream) {
    g_last_error.clear();
    return forward_impl("rwkv7m_wkv7_decode_inplace", dtype, 1, B, H, N, r,
                        w, k, v, neg_kk, kka, state, y, state, nullptr, 0,
                        static_cast<hipStream_t>(stream), false);
}

int64_t rwkv7m_timemix_workspace_floats(int64_t rows, int64_t H, int64_t N) {
    TmDims d;
    const std::string saved = g_last_error;
    const int rc = tm_check("rwkv7m_timemix_workspace_floats",
                            RWKV7M_DTYPE_F32, rows, H, N, &d);
    g_last_error = saved;
    if (rc != RWKV7M_OK) return -1;
    return rwkv7m::timemix_workspace_floats(rows, d.C);
}

int rwkv7m_timemix_wkv_inputs(int dtype, int64_t rows, int64_t H, int64_t N,
                              const void* w_raw, const void* k, const void* a,
                              const float* k_k, const float* k_a, void* w,
                              void* k_out, void* neg_kk, void* kka,
                              void* stream) {
    const char* fn = "rwkv7m_timemix_wkv_inputs";
    g_last_error.clear();
    TmDims d;
    RWKV7M_TRY(tm_check(fn, dtype, rows, H, N, &d));
    if (d.rows == 0 || d.C == 0) return RWKV7M_OK;
    RWKV7M_TRY(tm_need(fn, {{"w_raw", w_raw}, {"k", k}, {"a", a},
                            {"k_k", k_k}, {"k_a", k_a}, {"w", w},
                            {"k_out", k_out}, {"neg_kk", neg_kk},
                            {"kka", kka}}));
    rwkv7m::TmInputsArgs A{d.rows, d.C, w_raw, k, a, k_k, k_a,
                           w, k_out, neg_kk, kka};
    return hip_status("time-mix producers launch",
                      rwkv7m::launch_timemix_inputs(
                          dtype == RWKV7M_DTYPE_BF16, int(d.N), A,
                          static_cast<hipStream_t>(stream)));
}

int rwkv7m_timemix_wkv_inputs_backward(
    int dtype, int64_t rows, int64_t H, int64_t N, const void* w_raw,
    const void* k, const void* a, const float* k_k, const float* k_a,
    const void* dw, const void* dk_out, const void* dk_out2,
    const void* dneg_kk, const void* dkka, void* dw_raw, void* dk, void* da,
    float* dk_k, float* dk_a, float* workspace, int64_t workspace_floats,
    void* stream) {
    const char* fn = "rwkv7m_timemix_wkv_inputs_backward";
    g_last_error.clear();
    TmDims d;
    RWKV7M_TRY(tm_check(fn, dtype, rows, H, N, &d));
    if (d.C == 0) return RWKV7M_OK;
    RWKV7M_TRY(tm_need(fn, {{"k_k", k_k}, {"k_a", k_a}, {"dk_k", dk_k},
                            {"dk_a", dk_a}}));
    RWKV7M_TRY(tm_workspace(fn, d, workspace, workspace_floats));
    if (d.rows > 0) {
        RWKV7M_TRY(tm_need(fn, {{"w_raw", w_raw}, {"k", k}, {"a", a},
                                {"dw", dw}, {"dk_out", dk_out},
                                {"dneg_kk", dneg_kk}, {"dkka", dkka},
                                {"dw_raw", dw_raw}, {"dk", dk}, {"da", da}}));
        if (dk_out2) RWKV7M_TRY(tm_need(fn, {{"dk_out2", dk_out2}}));
    }
    rwkv7m::TmInputsBwdArgs A{d.rows, d.C,  w_raw,  k,      a,       k_k,
                              k_a,    dw,   dk_out, dk_out2, dneg_kk, dkka,
                              dw_raw, dk,   da,     dk_k,    dk_a,
                              workspace};
    return hip_status("time-mix producers backward launch",
                      rwkv7m::launch_timemix_inputs_backward(
                          dtype == RWKV7M_DTYPE_BF16, int(d.N), A,
                          static_cast<hipStream_t>(stream)));
}

int rwkv7m_timemix_wkv_output(int dtype, int64_t rows, int64_t H, int64_t N,
                              const void* y, const void* r, const void* k,
                              const void* v, const void* g, const float* r_k,
                              const float* ln_scale, const float* ln_bias,
                              double eps, void* out, void* stream) {
    const char* fn = "rwkv7m_timemix_wkv_output";
    g_last_error.clear();
    TmDims d;
    RWKV7M_TRY(tm_check(fn, dtype, rows, H, N, &d));
    RWKV7M_TRY(tm_eps(fn, eps));
    if (d.rows == 0 || d.C == 0) return RWKV7M_OK;
    RWKV7M_TRY(tm_need(fn, {{"y", y}, {"r", r}, {"k", k}, {"v", v},
                            {"g", g}, {"r_k", r_k}, {"ln_scale", ln_scale},
                            {"ln_bias", ln_bias}, {"out", out}}));
    rwkv7m::TmOutputArgs A{d.rows, d.C, float(eps), y, r, k, v, g,
                           r_k, ln_scale, ln_bias, out};
    return hip_status("time-mix consumer launch",
                      rwkv7m::launch_timemix_output(
                          dtype == RWKV7M_DTYPE_BF16, int(d.N), A,
                          static_cast<hipStream_t>(stream)));
}

int rwkv7m_timemix_wkv_output_backward(
    int dtype, int64_t rows, int64_t H, int64_t N, const void* y,
    const void* r, const void* k, const void* v, const void* g,
    const float* r_k, const float* ln_scale, const float* ln_bias, double eps,
    const void* dout, void* dy, void* dr, void* dk, void* dv, void* dg,
    float* dr_k, float* dln_scale, float* dln_bias, float* workspace,
    int64_t workspace_floats, void* stream) {
    g_last_error.clear();
    return output_backward_impl(
        "rwkv7m_timemix_wkv_output_backward", dtype, rows, H, N, y, r, k, v,
        g, r_k, ln_scale, ln_bias, eps, dout, dy, dr, dk, dv, dg, dr_k,
        dln_scale, dln_bias, workspace, workspace_floats, false,
        static_cast<hipStream_t>(stream));
}

int rwkv7m_timemix_wkv_output_backward_noalloc(
    int dtype, int64_t rows, int64_t H, int64_t N, const void* y,
    const void* r, const void* k, const void* v, const void* g,
    const float* r_k, const float* ln_scale, const float* ln_bias, double eps,
    const void* dout, void* dy, void* dr, void* dk, void* dv, void* dg,
    float* dr_k, float* dln_scale, float* dln_bias, void* stream) {
    g_last_error.clear();
    return output_backward_impl(
        "rwkv7m_timemix_wkv_output_backward_noalloc", dtype, rows, H, N, y, r,
        k, v, g, r_k, ln_scale, ln_bias, eps, dout, dy, dr, dk, dv, dg, dr_k,
        dln_scale, dln_bias, nullptr, 0, true,
        static_cast<hipStream_t>(stream));
}

int rwkv7m_timemix_wkv_backward(
    int dtype, int64_t T, int64_t B, int64_t H, int64_t N, const void* r,
    const void* w, const void* k, const void* v, const void* neg_kk,
    const void* kka, const float* initial_state, const void* dy,
    const float* ds_t, const void* checkpoints, int64_t checkpoint_interval,
    const void* dr_add, const void* dk_add, const void* dv_add, void* dr,
    void* dw, void* dk, void* dv, void* dneg_kk, void* dkka, float* ds0,
    void* stream) {
    g_last_error.clear();
    return backward_impl("rwkv7m_timemix_wkv_backward", dtype, T, B, H, N, r,
                         w, k, v, neg_kk, kka, initial_state, dy, ds_t,
                         checkpoints, checkpoint_interval, dr, dw, dk, dv,
                         dneg_kk, dkka, ds0, static_cast<hipStream_t>(stream),
                         true, dr_add, dk_add, dv_add);
}

int64_t rwkv7m_screen_slot_scan_workspace_floats(int64_t B, int64_t T,
                                                 int64_t M, int64_t ds) {
    const std::string saved = g_last_error;
    const int rc = sc_dims("rwkv7m_screen_slot_scan_workspace_floats",
                           RWKV7M_DTYPE_F32, B, T, M, ds, 0);
    g_last_error = saved;
    if (rc != RWKV7M_OK) return -1;
    return rwkv7m::screen_scan_workspace_floats(B, T, M, ds);
}

int rwkv7m_screen_slot_scan(int dtype, int64_t B, int64_t T, int64_t M,
                            int64_t ds, const void* base,
                            const float* slot_term, const float* mu,
                            const float* slots0, void* slots_seq,
                            float* slots_T, float* upd2, float* workspace,
                            int64_t workspace_floats, void* stream) {
    const char* fn = "rwkv7m_screen_slot_scan";
    g_last_error.clear();
    RWKV7M_TRY(sc_dims(fn, dtype, B, T, M, ds, 0));
    if (B == 0 || M == 0 || ds == 0) return RWKV7M_OK;
    RWKV7M_TRY(sc_need(fn, {{"slot_term", slot_term}, {"mu", mu},
                            {"slots0", slots0}, {"slots_T", slots_T},
                            {"workspace", workspace}}));
    RWKV7M_TRY(sc_workspace(fn, B, T, M, ds, workspace_floats));
    if (T > 0)
        RWKV7M_TRY(sc_need(fn, {{"base", base}, {"slots_seq", slots_seq},
                                {"upd2", upd2}}));
    rwkv7m::ScreenScanArgs A{};
    A.B = B;
    A.T = T;
    A.M = M;
    A.ds = ds;
    A.base = base;
    A.slot_term = slot_term;
    A.mu = mu;
    A.slots0 = slots0;
    A.slots_seq = slots_seq;
    A.slots_T = slots_T;
    A.upd2 = upd2;
    A.workspace = workspace;
    return hip_status("screening slot scan launch",
                      rwkv7m::launch_screen_scan(
                          dtype == RWKV7M_DTYPE_BF16, false, A,
                          static_cast<hipStream_t>(stream)));
}

int rwkv7m_screen_slot_scan_backward(
    int dtype, int64_t B, int64_t T, int64_t M, int64_t ds, const void* base,
    const float* slot_term, const float* mu, const void* slots_seq,
    const void* d_slots_seq, const float* d_slots_T, float* d_pre,
    float* d_slots0, float* d_mu_part, float* workspace,
    int64_t workspace_floats, void* stream) {
    const char* fn = "rwkv7m_screen_slot_scan_backward";
    g_last_error.clear();
    RWKV7M_TRY(sc_dims(fn, dtype, B, T, M, ds, 0));
    if (B == 0 || M == 0 || ds == 0) return RWKV7M_OK;
    RWKV7M_TRY(sc_need(fn, {{"slot_term", slot_term}, {"mu", mu},
                            {"d_slots0", d_slots0},
                            {"d_mu_part", d_mu_part},
                            {"workspace", workspace}}));
    RWKV7M_TRY(sc_workspace(fn, B, T, M, ds, workspace_floats));
    if (T > 0)
        RWKV7M_TRY(sc_need(fn, {{"base", base}, {"slots_seq", slots_seq},
                                {"d_slots_seq", d_slots_seq},
                                {"d_pre", d_pre}}));
    rwkv7m::ScreenScanArgs A{};
    A.B = B;
    A.T = T;
    A.M = M;
    A.ds = ds;
    A.base = base;
    A.slot_term = slot_term;
    A.mu = mu;
    A.slots_seq = const_cast<void*>(slots_seq);
    A.d_slots_seq = d_slots_seq;
    A.d_slots_T = d_slots_T;
    A.d_pre = d_pre;
    A.d_slots0 = d_slots0;
    A.d_mu_part = d_mu_part;
    A.workspace = workspace;
    return hip_status("screening slot scan backward launch",
                      rwkv7m::launch_screen_scan(
                          dtype == RWKV7M_DTYPE_BF16, true, A,
                          static_cast<hipStream_t>(stream)));
}

int rwkv7m_screen_read(int dtype, int64_t B, int64_t T, int64_t M,
                       int64_t dk, int64_t dv, const float* q,
                       const void* proj, const float* tau, double trim_eps,
                       const float* age_w, int age_per_step,
                       int value_unit_norm, int leaky, double leaky_alpha,
                       double leaky_gamma, double cap, double eps, void* u,
                       float* rel, float* z_norm, float* u_norm,
                       void* stream) {
    const char* fn = "rwkv7m_screen_read";
    g_last_error.clear();
    RWKV7M_TRY(sc_dims(fn, dtype, B, T, M, dk, dv));
    RWKV7M_TRY(sc_read_checks(fn, M, dk, dv, trim_eps, cap, eps, leaky_alpha,
                              leaky_gamma));
    if (B == 0 || T == 0) return RWKV7M_OK;
    RWKV7M_TRY(sc_need(fn, {{"q", q}, {"proj", proj}, {"tau", tau}, {"u", u},
                            {"rel", rel}, {"z_norm", z_norm},
                            {"u_norm", u_norm}}));
    rwkv7m::ScreenReadArgs A =
        sc_read_args(B, T, M, dk, dv, q, proj, tau, trim_eps, age_w,
                     age_per_step, value_unit_norm, leaky, leaky_alpha,
                     leaky_gamma, cap, eps);
    A.u = u;
    A.rel = rel;
    A.z_norm = z_norm;
    A.u_norm = u_norm;
    return hip_status("screening read launch",
                      rwkv7m::launch_screen_read(
                          dtype == RWKV7M_DTYPE_BF16, false, A,
                          static_cast<hipStream_t>(stream)));
}

int rwkv7m_screen_read_backward(
    int dtype, int64_t B, int64_t T, int64_t M, int64_t dk, int64_t dv,
    const float* q, const void* proj, const float* tau, double trim_eps,
    const float* age_w, int age_per_step, int value_unit_norm, int leaky,
    double leaky_alpha, double leaky_gamma, double cap, double eps,
    const void* du, const float* d_rel, float* dq, void* d_proj,
    float* d_tau, float* g_age, void* stream) {
    const char* fn = "rwkv7m_screen_read_backward";
    g_last_error.clear();
    RWKV7M_TRY(sc_dims(fn, dtype, B, T, M, dk, dv));
    RWKV7M_TRY(sc_read_checks(fn, M, dk, dv, trim_eps, cap, eps, leaky_alpha,
                              leaky_gamma));
    if (B == 0 || T == 0) return RWKV7M_OK;
    RWKV7M_TRY(sc_need(fn, {{"q", q}, {"proj", proj}, {"tau", tau}, {"du", du},
                            {"dq", dq}, {"d_proj", d_proj}, {"d_tau", d_tau},
                            {"g_age", g_age}}));
    rwkv7m::ScreenReadArgs A =
        sc_read_args(B, T, M, dk, dv, q, proj, tau, trim_eps, age_w,
                     age_per_step, value_unit_norm, leaky, leaky_alpha,
                     leaky_gamma, cap, eps);
    A.du = du;
    A.d_rel = d_rel;
    A.dq = dq;
    A.d_proj = d_proj;
    A.d_tau = d_tau;
    A.g_age = g_age;
    return hip_status("screening read backward launch",
                      rwkv7m::launch_screen_read(
                          dtype == RWKV7M_DTYPE_BF16, true, A,
                          static_cast<hipStream_t>(stream)));
}

int rwkv7m_screen_write(int dtype, int64_t B, int64_t T, int64_t M,
                        int64_t ds, int64_t dk, const void* base,
                        const float* slot_term, const float* slot_embed,
                        const float* kw, const float* q_w, const float* tau_w,
                        const float* mu, double floor, double eps,
                        const float* slots0, const float* ages0,
                        void* slots_seq, float* slots32, float* ages_seq,
                        float* rel_w, float* upd2, float* slots_T,
                        float* ages_T, void* stream) {
    const char* fn = "rwkv7m_screen_write";
    g_last_error.clear();
    RWKV7M_TRY(sc_write_checks(fn, dtype, B, T, M, ds, dk, floor, eps));
    if (B == 0 || M == 0 || ds == 0) return RWKV7M_OK;
    RWKV7M_TRY(sc_need(fn, {{"slot_term", slot_term},
                            {"slot_embed", slot_embed}, {"kw", kw},
                            {"tau_w", tau_w}, {"mu", mu}, {"slots0", slots0},
                            {"ages0", ages0}, {"slots_T", slots_T},
                            {"ages_T", ages_T}}));
    if (T > 0)
        RWKV7M_TRY(sc_need(fn, {{"base", base}, {"q_w", q_w},
                                {"slots_seq", slots_seq},
                                {"slots32", slots32}, {"ages_seq", ages_seq},
                                {"rel_w", rel_w}, {"upd2", upd2}}));
    rwkv7m::ScreenWriteArgs A = sc_write_args(
        B, T, M, ds, dk, base, slot_term, slot_embed, kw, q_w, tau_w, mu,
        floor, eps);
    A.slots0 = slots0;
    A.ages0 = ages0;
    A.slots_seq = slots_seq;
    A.slots32 = slots32;
    A.ages_seq = ages_seq;
    A.rel_w = rel_w;
    A.upd2 = upd2;
    A.slots_T = slots_T;
    A.ages_T = ages_T;
    return hip_status("screening write launch",
                      rwkv7m::launch_screen_write(
                          dtype == RWKV7M_DTYPE_BF16, false, A,
                          static_cast<hipStream_t>(stream)));
}

int rwkv7m_screen_write_backward(
    int dtype, int64_t B, int64_t T, int64_t M, int64_t ds, int64_t dk,
    const void* base, const float* slot_term, const float* slot_embed,
    const float* kw, const float* q_w, const float* tau_w, const float* mu,
    double floor, double eps, const float* slots32, const void* d_slots_seq,
    const float* d_slots_T, const float* d_rel_w, const float* d_ages_seq,
    const float* d_ages_T, float* d_pre, float* d_slots0, float* d_ages0,
    float* d_embed_part, float* d_mu_bm, float* d_kraw, float* dq_w,
    float* d_tau_w, void* stream) {
    const char* fn = "rwkv7m_screen_write_backward";
    g_last_error.clear();
    RWKV7M_TRY(sc_write_checks(fn, dtype, B, T, M, ds, dk, floor, eps));
    if (B == 0 || M == 0 || ds == 0) return RWKV7M_OK;
    RWKV7M_TRY(sc_need(fn, {{"slot_term", slot_term},
                            {"slot_embed", slot_embed}, {"kw", kw},
                            {"tau_w", tau_w}, {"mu", mu},
                            {"d_slots0", d_slots0}, {"d_ages0", d_ages0},
                            {"d_embed_part", d_embed_part},
                            {"d_mu_bm", d_mu_bm}}));
    if (T > 0)
        RWKV7M_TRY(sc_need(fn, {{"base", base}, {"q_w", q_w},
                                {"slots32", slots32},
                                {"d_slots_seq", d_slots_seq},
                                {"d_pre", d_pre}, {"d_kraw", d_kraw},
                                {"dq_w", dq_w}, {"d_tau_w", d_tau_w}}));
    rwkv7m::ScreenWriteArgs A = sc_write_args(
        B, T, M, ds, dk, base, slot_term, slot_embed, kw, q_w, tau_w, mu,
        floor, eps);
    A.slots32 = const_cast<float*>(slots32);
    A.d_slots_seq = d_slots_seq;
    A.d_slots_T = d_slots_T;
    A.d_rel_w = d_rel_w;
    A.d_ages_seq = d_ages_seq;
    A.d_ages_T = d_ages_T;
    A.d_pre = d_pre;
    A.d_slots0 = d_slots0;
    A.d_ages0 = d_ages0;
    A.d_embed_part = d_embed_part;
    A.d_mu_bm = d_mu_bm;
    A.d_kraw = d_kraw;
    A.dq_w = dq_w;
    A.d_tau_w = d_tau_w;
    return hip_status("screening write backward launch",
                      rwkv7m::launch_screen_write(
                          dtype == RWKV7M_DTYPE_BF16, true, A,
                          static_cast<hipStream_t>(stream)));
}

}  // extern "C"
