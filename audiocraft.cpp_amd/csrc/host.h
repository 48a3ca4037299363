// host.h -- library-internal host helpers shared by the library's sources: the status and
// message convention of include/mgx.h, device arenas, ggml tensor lookup and upload, and the
// GEMV argument builders.
#pragma once
#include "mgx.h"
#include "kernels.h"

#include <hip/hip_runtime.h>

#include <chrono>
#include <stdexcept>
#include <string>
#include <vector>

namespace mgxh {

inline thread_local std::string g_error;   // mgx_last_error's message, per thread

struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

#define HIP_OK(expr)                                                                            \
    do {                                                                                        \
        hipError_t e_ = (expr);                                                                 \
        if (e_ != hipSuccess)                                                                   \
            throw mgxh::Error(MGX_ERR_DEVICE, std::string(#expr) + ": " + hipGetErrorString(e_)); \
    } while (0)

template <typename F> inline int guarded(F&& f) {
    try {
        f();
        return MGX_OK;
    } catch (const Error& e) {
        g_error = e.what();
        return e.code;
    } catch (const std::exception& e) {
        g_error = e.what();
        return MGX_ERR_INVALID;
    }
}

inline double now_s() {
    using clock = std::chrono::steady_clock;
    return std::chrono::duration<double>(clock::now().time_since_epoch()).count();
}

// Device allocations owned by one object, freed together.
struct DevArena {
    std::vector<void*> ptrs;
    template <typename T> T* alloc(size_t count) {
        void* p = nullptr;
        if (count == 0) count = 1;
        HIP_OK(hipMalloc(&p, count * sizeof(T)));
        ptrs.push_back(p);
        return (T*)p;
    }
    void release() {
        for (void* p : ptrs) (void)hipFree(p);
        ptrs.clear();
    }
};

inline size_t row_bytes(int type, int64_t in) {
    switch (type) {
    case mgx::T_F32: return (size_t)in * 4;
    case mgx::T_F16: return (size_t)in * 2;
    case mgx::T_Q8_0: return (size_t)(in / 32) * 34;
    case mgx::T_Q4_0: return (size_t)(in / 32) * 18;
    }
    return 0;
}

inline const mgx_tensor* find(const mgx_tensor* t, int n, const std::string& name) {
    for (int i = 0; i < n; ++i)
        if (t[i].name && name == t[i].name) return &t[i];
    return nullptr;
}

inline const mgx_tensor& need(const mgx_tensor* t, int n, const std::string& name, int64_t ne0, int64_t ne1) {
    const mgx_tensor* x = find(t, n, name);
    if (!x) throw Error(MGX_ERR_INVALID, "missing tensor " + name);
    if (x->ne[0] != ne0 || x->ne[1] != ne1 || (x->ne[2] > 1) || (x->ne[3] > 1))
        throw Error(MGX_ERR_INVALID, "bad shape for " + name);
    if (!x->data) throw Error(MGX_ERR_INVALID, "no data for " + name);
    const size_t rb = row_bytes(x->type, ne0);
    if (!rb) throw Error(MGX_ERR_INVALID, "unsupported tensor type for " + name);
    if ((x->type == mgx::T_Q8_0 || x->type == mgx::T_Q4_0) && ne0 % 32)
        throw Error(MGX_ERR_INVALID, name + ": quantized rows must hold whole 32-blocks");
    if (x->nbytes && x->nbytes < rb * (size_t)ne1) throw Error(MGX_ERR_INVALID, "short data for " + name);
    return *x;
}

// Uploads `rows` rows of one ggml tensor into `dst` starting at row `row0` (dst already sized).
inline void upload_rows(const mgx_tensor& t, mgx::DevMat& dst, int64_t row0, hipStream_t s) {
    const int64_t rows = t.ne[1];
    const int in = (int)t.ne[0];
    const size_t rb = row_bytes(t.type, in);
    if (t.type == mgx::T_F32 || t.type == mgx::T_F16) {
        const size_t es = t.type == mgx::T_F32 ? 4 : 2;
        HIP_OK(hipMemcpyAsync((uint8_t*)dst.q + (size_t)row0 * in * es, t.data, rb * rows, hipMemcpyHostToDevice, s));
        return;
    }
    uint8_t* raw = nullptr;
    HIP_OK(hipMalloc(&raw, rb * rows));
    HIP_OK(hipMemcpyAsync(raw, t.data, rb * rows, hipMemcpyHostToDevice, s));
    const size_t qrow = t.type == mgx::T_Q8_0 ? (size_t)in : (size_t)in / 2;
    mgx::launch_repack(t.type, raw, rows, in, (uint8_t*)dst.q + (size_t)row0 * qrow,
                       (uint16_t*)dst.d + (size_t)row0 * (in / 32), s);
    HIP_OK(hipGetLastError());
    HIP_OK(hipStreamSynchronize(s));
    HIP_OK(hipFree(raw));
}

inline mgx::DevMat alloc_mat(DevArena& mem, int type, int in, int out) {
    mgx::DevMat d{};
    d.type = type; d.in = in; d.out = out;
    switch (type) {
    case mgx::T_Q8_0: d.q = mem.alloc<int8_t>((size_t)in * out); d.d = mem.alloc<uint16_t>((size_t)(in / 32) * out); break;
    case mgx::T_Q4_0: d.q = mem.alloc<uint8_t>((size_t)in / 2 * out); d.d = mem.alloc<uint16_t>((size_t)(in / 32) * out); break;
    case mgx::T_F16: d.q = mem.alloc<uint16_t>((size_t)in * out); break;
    default: d.q = mem.alloc<float>((size_t)in * out); break;
    }
    return d;
}

inline mgx::DevMat load_mat(DevArena& mem, const mgx_tensor* t, int n, const std::string& name, int in, int out,
                            hipStream_t s) {
    const mgx_tensor& x = need(t, n, name, in, out);
    mgx::DevMat d = alloc_mat(mem, x.type, in, out);
    upload_rows(x, d, 0, s);
    return d;
}

inline const float* load_vec(DevArena& mem, const mgx_tensor* t, int n, const std::string& name, int len,
                             hipStream_t s) {
    const mgx_tensor* x = find(t, n, name);
    if (!x || x->type != mgx::T_F32 || x->ne[0] != len || !x->data)
        throw Error(MGX_ERR_INVALID, "missing or bad f32 vector " + name);
    float* d = mem.alloc<float>((size_t)len);
    HIP_OK(hipMemcpyAsync(d, x->data, sizeof(float) * (size_t)len, hipMemcpyHostToDevice, s));
    return d;
}

// GEMV argument builders: the weights and column count, then a prologue (LayerNorm, f32 or
// activation-form source) and an epilogue (store or residual add).
inline mgx::GemvArgs ga(const mgx::DevMat& w, int ncol) {
    mgx::GemvArgs a{};
    a.w = w; a.ncol = ncol;
    return a;
}
inline mgx::GemvArgs& pro_ln(mgx::GemvArgs& a, const float* x, int stride, const float* w, const float* b, float eps) {
    a.pro = mgx::PRO_LN; a.x = x; a.x_stride = stride; a.ln_w = w; a.ln_b = b; a.eps = eps;
    return a;
}
inline mgx::GemvArgs& pro_f32(mgx::GemvArgs& a, const float* x, int stride) {
    a.pro = mgx::PRO_F32; a.x = x; a.x_stride = stride;
    return a;
}
inline mgx::GemvArgs& pro_act(mgx::GemvArgs& a, const mgx::ActBuf& src) {
    a.pro = mgx::PRO_ACT; a.src = src;
    return a;
}
inline mgx::GemvArgs& epi_store(mgx::GemvArgs& a, float* y, int stride, bool resid = false) {
    a.epi = resid ? mgx::EPI_RESID : mgx::EPI_STORE; a.y = y; a.y_stride = stride;
    return a;
}

}  // namespace mgxh
