// C ABI of the attention sublayers (include/sdxl_hip/sublayer.h): validation
// and stream-ordered launches of LayerNorm, linear, E4M3 quantisation, the
// whole LN -> fused QKV -> attention -> output projection + residual chain
// (reference src/cuda/unet.cpp:106-118) and its cross-attention counterpart
// with the context K/V projected once per request (src/cuda/unet.cpp:120-131).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <mutex>
#include <string>

#include "../../include/sdxl_hip/sublayer.h"
#include "capi_internal.hpp"
#include "sublayer_kernels.hpp"

namespace {

bool aligned(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0; }

int compute_units() { return sdxl_hip_compute_units(); }

sdxl_status launch_status(hipError_t err, const char* what) {
    if (err != hipSuccess)
        return sdxl_hip_fail(SDXL_STATUS_LAUNCH_FAILED, std::string(what) + ": " + hipGetErrorString(err));
    return SDXL_STATUS_OK;
}

}  // namespace

// Device-resident workspace of sdxl_attn_sublayer_noalloc: one array per GPU,
// held until the process ends (a .bss symbol of the code object: no file size,
// no allocation call). Host code never passes `scratch` itself (on the host it
// names a stand-in, not device memory): the per-device address comes from
// hipGetSymbolAddress, taken once per device with that device current.
constexpr size_t kScratchBytes = size_t{80} << 20;
__device__ __attribute__((aligned(256))) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;

// Address of `scratch` on the current device, looked up on the first call on
// that device; nullptr (and the HIP error text in *err) on failure.
void* scratch_on_current_device(std::string* err) {
    static std::mutex mu;
    static void* ptr[kMaxDevices] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        *err = e != hipSuccess ? hipGetErrorString(e) : "device index out of range";
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            *err = e != hipSuccess ? hipGetErrorString(e) : "null symbol address";
            return nullptr;
        }
        ptr[dev] = p;
    }
    return ptr[dev];
}

namespace {

// Shared by sdxl_layer_norm and sdxl_layer_norm_e4m3 (y_scale set: E4M3 output,
// y row stride in bytes).
sdxl_status layer_norm_impl(const char* name, int64_t rows, int64_t width, const void* x, int64_t x_row_stride,
                            const void* gamma, const void* beta, float eps, void* y, int64_t y_row_stride,
                            float* y_scale, void* stream) {
    // Message of the reference's Ops::layer_norm checks (ops_kernels.cu:1431-1437).
    if (rows < 0 || width <= 0 || x_row_stride < 0 || y_row_stride < 0)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_SHAPE, "CUDA layer norm shape/type mismatch");
    const int64_t ldx = x_row_stride == 0 ? width : x_row_stride;
    const int64_t ldy = y_row_stride == 0 ? width : y_row_stride;
    if (ldx < width || ldy < width)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_SHAPE, "CUDA layer norm shape/type mismatch");
    if (width % 2 != 0 || width > 2048 || ldx % 2 != 0 || ldy % 2 != 0)
        return sdxl_hip_fail(SDXL_STATUS_UNSUPPORTED, std::string(name) + ": width must be even and <= 2048");
    if (rows == 0) return SDXL_STATUS_OK;
    if (x == nullptr || gamma == nullptr || beta == nullptr || y == nullptr)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_ARGUMENT, std::string(name) + ": null tensor pointer");
    if (!aligned(x, 4) || !aligned(y, 4) || !aligned(gamma, 4) || !aligned(beta, 4) ||
        (y_scale != nullptr && !aligned(y_scale, 4)))
        return sdxl_hip_fail(SDXL_STATUS_UNSUPPORTED, std::string(name) + ": tensors must be 4-byte aligned");
    sdxl_hip::LayerNormParams p{};
    p.x = x;
    p.gamma = gamma;
    p.beta = beta;
    p.y = y;
    p.y_scale = y_scale;
    p.rows = rows;
    p.ldx = ldx;
    p.ldy = ldy;
    p.width = (int32_t)width;
    p.eps = eps > 0.0f ? eps : 1.0e-5f;
    return launch_status(sdxl_hip::launch_layer_norm(p, reinterpret_cast<hipStream_t>(stream)), name);
}

}  // namespace

extern "C" {

sdxl_status sdxl_layer_norm(int64_t rows, int64_t width, const void* x, int64_t x_row_stride, const void* gamma,
                            const void* beta, float eps, void* y, int64_t y_row_stride, void* stream) {
    return layer_norm_impl("sdxl_layer_norm", rows, width, x, x_row_stride, gamma, beta, eps, y, y_row_stride,
                           nullptr, stream);
}

sdxl_status sdxl_layer_norm_e4m3(int64_t rows, int64_t width, const void* x, int64_t x_row_stride,
                                 const void* gamma, const void* beta, float eps, uint8_t* q, int64_t q_row_stride,
                                 float* q_scale, void* stream) {
    if (rows > 0 && q_scale == nullptr)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_layer_norm_e4m3: null tensor pointer");
    return layer_norm_impl("sdxl_layer_norm_e4m3", rows, width, x, x_row_stride, gamma, beta, eps, q, q_row_stride,
                           q_scale, stream);
}

}  // extern "C"

namespace {

// Shared by sdxl_linear and sdxl_linear_e4m3 (a_scale set: a holds E4M3 codes,
// a row stride in bytes).
sdxl_status linear_impl(const sdxl_linear_desc* d, const void* a, const float* a_scale, const void* w,
                        const float* w_scale, const void* bias, const void* residual, void* c, void* stream) {
    if (d == nullptr) return sdxl_hip_fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_linear: null descriptor");
    if (d->reserved != 0) return sdxl_hip_fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_linear: reserved field must be 0");
    if (d->w_dtype != SDXL_DTYPE_F16 && d->w_dtype != SDXL_DTYPE_E4M3)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_SHAPE, "sdxl_linear: weights must be fp16 or E4M3");
    if (d->m < 0 || d->n < 0 || d->k < 0 || d->m > INT32_MAX || d->n > INT32_MAX || d->k > INT32_MAX)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_SHAPE, "sdxl_linear: dimensions out of range");
    const int64_t lda = d->a_row_stride ? d->a_row_stride : d->k;
    const int64_t ldw = d->w_row_stride ? d->w_row_stride : d->k;
    const int64_t ldc = d->c_row_stride ? d->c_row_stride : d->n;
    const int64_t ldr = d->residual_row_stride ? d->residual_row_stride : d->n;
    if (lda < d->k || ldw < d->k || ldc < d->n || ldr < d->n)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_SHAPE, "sdxl_linear: row stride smaller than the row");
    const bool fp8 = d->w_dtype == SDXL_DTYPE_E4M3;
    const bool a_fp8 = a_scale != nullptr;
    if (a_fp8 && !fp8)
        return sdxl_hip_fail(SDXL_STATUS_UNSUPPORTED, "sdxl_linear_e4m3: weights must be E4M3");
    if (fp8 && w_scale == nullptr)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_ARGUMENT, "FP8 weight has invalid scaling metadata");
    if (d->m == 0 || d->n == 0) return SDXL_STATUS_OK;
    if (d->k % 64 != 0 || d->n % 4 != 0)
        return sdxl_hip_fail(SDXL_STATUS_UNSUPPORTED, "sdxl_linear: requires k % 64 == 0 and n % 4 == 0");
    if (a == nullptr || w == nullptr || c == nullptr)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_linear: null tensor pointer");
    const int64_t w_elem = fp8 ? 1 : 2;
    const int64_t a_elem = a_fp8 ? 1 : 2;
    if (!aligned(a, 16) || (lda * a_elem) % 16 != 0 || !aligned(w, 16) || (ldw * w_elem) % 16 != 0 ||
        (a_fp8 && !aligned(a_scale, 4)) ||
        !aligned(c, 8) || ldc % 4 != 0 || (w_scale != nullptr && !aligned(w_scale, 16)) ||
        (bias != nullptr && !aligned(bias, 8)) || (residual != nullptr && (!aligned(residual, 8) || ldr % 4 != 0)))
        return sdxl_hip_fail(SDXL_STATUS_UNSUPPORTED, "sdxl_linear: misaligned tensor or row stride");
    if (lda * a_elem * 256 > UINT32_MAX || ldw * w_elem * 128 > UINT32_MAX)
        return sdxl_hip_fail(SDXL_STATUS_UNSUPPORTED, "sdxl_linear: row stride too large");
    sdxl_hip::LinearParams p{};
    p.a = a;
    p.w = w;
    p.w_scale = w_scale;
    p.bias = bias;
    p.residual = residual;
    p.a_scale = a_scale;
    p.c = c;
    p.lda = lda;
    p.ldw = ldw;
    p.ldr = ldr;
    p.ldc = ldc;
    p.m = (int32_t)d->m;
    p.n = (int32_t)d->n;
    p.k = (int32_t)d->k;
    return launch_status(sdxl_hip::launch_linear(p, fp8, compute_units(), reinterpret_cast<hipStream_t>(stream)),
                         a_fp8 ? "sdxl_linear_e4m3" : "sdxl_linear");
}

}  // namespace

namespace {

// Validation of sdxl_layer_norm_linear; fills p. SDXL_STATUS_UNSUPPORTED for
// shapes the fused kernel does not take (the caller may compose instead).
sdxl_status ln_linear_params(const sdxl_linear_desc* d, const void* x, const void* gamma, const void* beta, float eps,
                             const void* w, const float* w_scale, const void* bias, void* c, bool a_fp8,
                             sdxl_hip::LnLinearParams& p) {
    if (d == nullptr) return sdxl_hip_fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_layer_norm_linear: null descriptor");
    if (d->reserved != 0 || d->residual_row_stride != 0)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_ARGUMENT,
                             "sdxl_layer_norm_linear: reserved and residual_row_stride must be 0");
    if (d->m < 0 || d->n < 0 || d->k <= 0 || d->m > INT32_MAX || d->n > INT32_MAX || d->k > INT32_MAX)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_SHAPE, "sdxl_layer_norm_linear: dimensions out of range");
    const int64_t ldx = d->a_row_stride ? d->a_row_stride : d->k;
    const int64_t ldw = d->w_row_stride ? d->w_row_stride : d->k;
    const int64_t ldc = d->c_row_stride ? d->c_row_stride : d->n;
    if (ldx < d->k || ldw < d->k || ldc < d->n)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_SHAPE, "sdxl_layer_norm_linear: row stride smaller than the row");
    if (d->w_dtype != SDXL_DTYPE_E4M3)
        return sdxl_hip_fail(SDXL_STATUS_UNSUPPORTED, "sdxl_layer_norm_linear: weights must be E4M3");
    if (w_scale == nullptr)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_ARGUMENT, "FP8 weight has invalid scaling metadata");
    if (x == nullptr || gamma == nullptr || beta == nullptr || w == nullptr || c == nullptr)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_layer_norm_linear: null tensor pointer");
    p = sdxl_hip::LnLinearParams{};
    p.x = x;
    p.gamma = gamma;
    p.beta = beta;
    p.w = static_cast<const uint8_t*>(w);
    p.w_scale = w_scale;
    p.bias = bias;
    p.c = c;
    p.ldx = ldx;
    p.ldw = ldw;
    p.ldc = ldc;
    p.m = (int32_t)d->m;
    p.n = (int32_t)d->n;
    p.k = (int32_t)d->k;
    p.eps = eps > 0.0f ? eps : 1.0e-5f;
    p.a_fp8 = a_fp8 ? 1 : 0;
    if (d->m > 0 && d->n > 0 && !sdxl_hip::ln_linear_supported(p))
        return sdxl_hip_fail(SDXL_STATUS_UNSUPPORTED,
                             "sdxl_layer_norm_linear: needs k == 640 or 1280, n % 128 == 0, 16-byte aligned x rows, gamma, beta "
                             "and w rows, 8-byte aligned c rows");
    return SDXL_STATUS_OK;
}

}  // namespace

extern "C" {

sdxl_status sdxl_layer_norm_linear(const sdxl_linear_desc* d, const void* x, const void* gamma, const void* beta,
                                   float eps, const void* w, const float* w_scale, const void* bias, void* c,
                                   void* stream) {
    sdxl_hip::LnLinearParams p;
    const sdxl_status st = ln_linear_params(d, x, gamma, beta, eps, w, w_scale, bias, c, false, p);
    if (st != SDXL_STATUS_OK) return st;
    if (p.m == 0 || p.n == 0) return SDXL_STATUS_OK;
    return launch_status(sdxl_hip::launch_ln_linear(p, compute_units(), reinterpret_cast<hipStream_t>(stream)),
                         "sdxl_layer_norm_linear");
}

sdxl_status sdxl_layer_norm_linear_e4m3(const sdxl_linear_desc* d, const void* x, const void* gamma, const void* beta,
                                        float eps, const void* w, const float* w_scale, const void* bias, void* c,
                                        void* stream) {
    sdxl_hip::LnLinearParams p;
    const sdxl_status st = ln_linear_params(d, x, gamma, beta, eps, w, w_scale, bias, c, true, p);
    if (st != SDXL_STATUS_OK) return st;
    if (p.m == 0 || p.n == 0) return SDXL_STATUS_OK;
    return launch_status(sdxl_hip::launch_ln_linear(p, compute_units(), reinterpret_cast<hipStream_t>(stream)),
                         "sdxl_layer_norm_linear_e4m3");
}

sdxl_status sdxl_linear(const sdxl_linear_desc* d, const void* a, const void* w, const float* w_scale,
                        const void* bias, const void* residual, void* c, void* stream) {
    return linear_impl(d, a, nullptr, w, w_scale, bias, residual, c, stream);
}

sdxl_status sdxl_linear_e4m3(const sdxl_linear_desc* d, const uint8_t* a, const float* a_scale, const void* w,
                             const float* w_scale, const void* bias, const void* residual, void* c, void* stream) {
    if (d != nullptr && d->m > 0 && a_scale == nullptr)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_linear_e4m3: null activation scales");
    if (d != nullptr && d->m == 0) return linear_impl(d, a, nullptr, w, w_scale, bias, residual, c, stream);
    return linear_impl(d, a, a_scale, w, w_scale, bias, residual, c, stream);
}

sdxl_status sdxl_quantize_e4m3_rows(int64_t rows, int64_t cols, const void* w, uint8_t* q, float* scales,
                                    void* stream) {
    if (rows < 0 || cols < 0) return sdxl_hip_fail(SDXL_STATUS_INVALID_SHAPE, "sdxl_quantize_e4m3_rows: negative shape");
    if (rows == 0) return SDXL_STATUS_OK;
    if (w == nullptr || q == nullptr || scales == nullptr)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_quantize_e4m3_rows: null tensor pointer");
    if (!aligned(w, 2) || !aligned(scales, 4))
        return sdxl_hip_fail(SDXL_STATUS_UNSUPPORTED, "sdxl_quantize_e4m3_rows: misaligned tensor");
    sdxl_hip::QuantizeParams p{};
    p.w = w;
    p.q = q;
    p.scales = scales;
    p.rows = rows;
    p.cols = cols;
    return launch_status(sdxl_hip::launch_quantize_e4m3_rows(p, reinterpret_cast<hipStream_t>(stream)),
                         "sdxl_quantize_e4m3_rows");
}

size_t sdxl_attn_sublayer_workspace_bytes(const sdxl_sublayer_desc* d) {
    if (d == nullptr || d->batch < 0 || d->seq < 0 || d->heads < 0) return 0;
    return (size_t)d->batch * (size_t)d->seq * (size_t)(d->heads * 64) * 8u;
}

sdxl_status sdxl_attn_sublayer(const sdxl_sublayer_desc* d, const void* x, const void* ln_gamma, const void* ln_beta,
                               const void* w_qkv, const float* w_qkv_scale, const void* w_out, const void* b_out,
                               void* y, void* workspace, size_t workspace_bytes, void* stream) {
    if (d == nullptr) return sdxl_hip_fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_attn_sublayer: null descriptor");
    if (d->qkv_activations != SDXL_DTYPE_F16 && d->qkv_activations != SDXL_DTYPE_E4M3)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_attn_sublayer: qkv_activations must be F16 or E4M3");
    const bool act_fp8 = d->qkv_activations == SDXL_DTYPE_E4M3;
    if (act_fp8 && d->w_qkv_dtype != SDXL_DTYPE_E4M3)
        return sdxl_hip_fail(SDXL_STATUS_UNSUPPORTED, "sdxl_attn_sublayer: E4M3 activations need E4M3 w_qkv");
    if (d->batch < 0 || d->seq < 0 || d->heads <= 0)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_SHAPE, "sdxl_attn_sublayer: invalid shape");
    const int64_t W = d->heads * 64;
    const int64_t M = d->batch * d->seq;
    if (M == 0) return SDXL_STATUS_OK;
    if (workspace == nullptr || workspace_bytes < sdxl_attn_sublayer_workspace_bytes(d) || !aligned(workspace, 256))
        return sdxl_hip_fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_attn_sublayer: workspace missing, small or misaligned");
    char* ws = static_cast<char*>(workspace);
    void* hidden_ws = ws;                                  // [M, W]: LN output, later attention output
    void* qkv = ws + (size_t)M * (size_t)W * 2;            // [M, 3W]
    // E4M3 activations: codes [M, W] bytes, then their row scales [M], both
    // inside the first region (M W + 4 M <= 2 M W bytes for W >= 4).
    uint8_t* codes = static_cast<uint8_t*>(hidden_ws);
    float* code_scale = reinterpret_cast<float*>(ws + (size_t)M * (size_t)W);

    sdxl_linear_desc qd{};
    qd.m = M;
    qd.n = 3 * W;
    qd.k = W;
    qd.w_dtype = d->w_qkv_dtype;
    sdxl_status st;
    // LayerNorm fused into the projection where the kernel takes the shape
    // (E4M3 weights, width 640 or 1280) and is the faster choice (the level-1
    // blocks; not the level-2 ones, whose 2048 rows are normalised again by 8
    // workgroups per row block); else two launches.
    // (checked quietly: an unsupported shape is no error here)
    sdxl_hip::LnLinearParams lp{};
    lp.x = x;
    lp.gamma = ln_gamma;
    lp.beta = ln_beta;
    lp.w = static_cast<const uint8_t*>(w_qkv);
    lp.w_scale = w_qkv_scale;
    lp.c = qkv;
    lp.ldx = W;
    lp.ldw = W;
    lp.ldc = 3 * W;
    lp.m = (int32_t)M;
    lp.n = (int32_t)(3 * W);
    lp.k = (int32_t)W;
    lp.eps = d->ln_eps > 0.0f ? d->ln_eps : 1.0e-5f;
    lp.a_fp8 = act_fp8 ? 1 : 0;
    const bool fuse = d->ln_fusion == 0 && d->w_qkv_dtype == SDXL_DTYPE_E4M3 && M <= INT32_MAX &&
                      3 * W <= INT32_MAX && x != nullptr && ln_gamma != nullptr && ln_beta != nullptr &&
                      w_qkv != nullptr && sdxl_hip::ln_linear_preferred(lp, compute_units());
    if (fuse) {
        st = launch_status(sdxl_hip::launch_ln_linear(lp, compute_units(), reinterpret_cast<hipStream_t>(stream)),
                           "sdxl_attn_sublayer");
    } else if (act_fp8) {
        st = sdxl_layer_norm_e4m3(M, W, x, 0, ln_gamma, ln_beta, d->ln_eps, codes, 0, code_scale, stream);
        if (st != SDXL_STATUS_OK) return st;
        st = sdxl_linear_e4m3(&qd, codes, code_scale, w_qkv, w_qkv_scale, nullptr, nullptr, qkv, stream);
    } else {
        st = sdxl_layer_norm(M, W, x, 0, ln_gamma, ln_beta, d->ln_eps, hidden_ws, 0, stream);
        if (st != SDXL_STATUS_OK) return st;
        st = sdxl_linear(&qd, hidden_ws, w_qkv, w_qkv_scale, nullptr, nullptr, qkv, stream);
    }
    if (st != SDXL_STATUS_OK) return st;

    sdxl_attn_desc ad{};
    ad.batch = d->batch;
    ad.q_seq = d->seq;
    ad.k_seq = d->seq;
    ad.heads = d->heads;
    ad.head_dim = 64;
    ad.q_row_stride = ad.k_row_stride = ad.v_row_stride = 3 * W;
    ad.o_row_stride = W;
    ad.dtype = SDXL_DTYPE_F16;
    ad.backend = d->attn_backend;
    const char* qkv_c = static_cast<const char*>(qkv);
    st = sdxl_attn_fwd(&ad, qkv_c, qkv_c + W * 2, qkv_c + 2 * W * 2, nullptr, hidden_ws, stream);
    if (st != SDXL_STATUS_OK) return st;

    sdxl_linear_desc od{};
    od.m = M;
    od.n = W;
    od.k = W;
    od.w_dtype = SDXL_DTYPE_F16;
    return sdxl_linear(&od, hidden_ws, w_out, nullptr, b_out, x, y, stream);
}

size_t sdxl_attn_sublayer_noalloc_max_workspace_bytes(void) { return kScratchBytes; }

sdxl_status sdxl_attn_sublayer_noalloc(const sdxl_sublayer_desc* d, const void* x, const void* ln_gamma,
                                       const void* ln_beta, const void* w_qkv, const float* w_qkv_scale,
                                       const void* w_out, const void* b_out, void* y, void* stream) {
    if (d == nullptr) return sdxl_hip_fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_attn_sublayer_noalloc: null descriptor");
    if (d->batch < 0 || d->seq < 0 || d->heads <= 0)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_SHAPE, "sdxl_attn_sublayer_noalloc: invalid shape");
    int64_t rows = 0;
    const bool huge = __builtin_mul_overflow(d->batch, d->seq, &rows) || rows > INT32_MAX || d->heads > 65536;
    const size_t need = huge ? SIZE_MAX : sdxl_attn_sublayer_workspace_bytes(d);
    if (need > kScratchBytes)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_SHAPE,
                             "sdxl_attn_sublayer_noalloc: needs " + std::to_string(need) +
                                 " workspace bytes (batch * seq * heads * 512), more than the " +
                                 std::to_string(kScratchBytes) + "-byte device scratch; use sdxl_attn_sublayer");
    if (d->batch * d->seq == 0) return SDXL_STATUS_OK;
    std::string err;
    void* ws = scratch_on_current_device(&err);
    if (ws == nullptr)
        return sdxl_hip_fail(SDXL_STATUS_LAUNCH_FAILED, "sdxl_attn_sublayer_noalloc: scratch address: " + err);
    // Every stage writes its part of the workspace before reading it: nothing
    // needs clearing between calls.
    return sdxl_attn_sublayer(d, x, ln_gamma, ln_beta, w_qkv, w_qkv_scale, w_out, b_out, y, ws, kScratchBytes,
                              stream);
}

size_t sdxl_cross_attn_sublayer_workspace_bytes(const sdxl_cross_sublayer_desc* d) {
    if (d == nullptr || d->batch < 0 || d->seq < 0 || d->heads < 0) return 0;
    return (size_t)d->batch * (size_t)d->seq * (size_t)(d->heads * 64) * 4u;
}

sdxl_status sdxl_cross_attn_sublayer(const sdxl_cross_sublayer_desc* d, const void* x, const void* ln_gamma,
                                     const void* ln_beta, const void* w_q, const float* w_q_scale, const void* kv,
                                     int64_t kv_row_stride, const void* w_out, const void* b_out, void* y,
                                     void* workspace, size_t workspace_bytes, void* stream) {
    if (d == nullptr) return sdxl_hip_fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_cross_attn_sublayer: null descriptor");
    if (d->q_activations != SDXL_DTYPE_F16 && d->q_activations != SDXL_DTYPE_E4M3)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_ARGUMENT,
                             "sdxl_cross_attn_sublayer: q_activations must be F16 or E4M3");
    const bool act_fp8 = d->q_activations == SDXL_DTYPE_E4M3;
    if (act_fp8 && d->w_q_dtype != SDXL_DTYPE_E4M3)
        return sdxl_hip_fail(SDXL_STATUS_UNSUPPORTED, "sdxl_cross_attn_sublayer: E4M3 activations need E4M3 w_q");
    if (d->batch < 0 || d->seq < 0 || d->heads <= 0 || d->ctx_len < 0)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_SHAPE, "sdxl_cross_attn_sublayer: invalid shape");
    const int64_t W = d->heads * 64;
    const int64_t M = d->batch * d->seq;
    const int64_t ldkv = kv_row_stride ? kv_row_stride : 2 * W;
    if (kv_row_stride < 0 || ldkv < 2 * W)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_SHAPE, "sdxl_cross_attn_sublayer: kv row stride below 2W");
    if (M == 0) return SDXL_STATUS_OK;
    if (workspace == nullptr || workspace_bytes < sdxl_cross_attn_sublayer_workspace_bytes(d) ||
        !aligned(workspace, 256))
        return sdxl_hip_fail(SDXL_STATUS_INVALID_ARGUMENT,
                             "sdxl_cross_attn_sublayer: workspace missing, small or misaligned");
    if (d->ctx_len > 0 && kv == nullptr)
        return sdxl_hip_fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_cross_attn_sublayer: null tensor pointer");
    char* ws = static_cast<char*>(workspace);
    void* hidden_ws = ws;                               // [M, W]: LN output, later attention output
    void* q = ws + (size_t)M * (size_t)W * 2;           // [M, W]
    uint8_t* codes = static_cast<uint8_t*>(hidden_ws);  // E4M3 activations: codes, then row scales
    float* code_scale = reinterpret_cast<float*>(ws + (size_t)M * (size_t)W);

    sdxl_linear_desc qd{};
    qd.m = M;
    qd.n = W;
    qd.k = W;
    qd.w_dtype = d->w_q_dtype;
    sdxl_status st;
    if (act_fp8) st = sdxl_layer_norm_e4m3(M, W, x, 0, ln_gamma, ln_beta, d->ln_eps, codes, 0, code_scale, stream);
    else st = sdxl_layer_norm(M, W, x, 0, ln_gamma, ln_beta, d->ln_eps, hidden_ws, 0, stream);
    if (st != SDXL_STATUS_OK) return st;

    // Query projection and attention in one launch where the shapes allow it
    // (the 77-token context, sequences in 64-row tiles, 128-column head
    // pairs, a grid resident at once) and the backend is left to the
    // library: each wave attends with
    // the 32 x 64 query block it has just projected, which never leaves the
    // CU. Its output (the attention output) goes to the second workspace
    // region while other workgroups still read the LayerNorm output.
    const bool w_fp8 = d->w_q_dtype == SDXL_DTYPE_E4M3;
    if (d->attn_backend == SDXL_ATTN_AUTO && (!w_fp8 || w_q_scale != nullptr) && w_q != nullptr &&
        aligned(w_q, 16) && (W * (w_fp8 ? 1 : 2)) % 16 == 0 && (w_q_scale == nullptr || aligned(w_q_scale, 16))) {
        sdxl_hip::LinearParams p{};
        p.a = act_fp8 ? static_cast<const void*>(codes) : hidden_ws;
        p.a_scale = act_fp8 ? code_scale : nullptr;
        p.w = w_q;
        p.w_scale = w_q_scale;
        p.c = q;
        p.lda = p.ldw = p.ldc = p.ldr = W;
        p.m = (int32_t)M;
        p.n = p.k = (int32_t)W;
        p.kv = kv;
        p.ldkv = ldkv;
        p.ctx_len = (int32_t)d->ctx_len;
        p.seq = (int32_t)d->seq;
        p.scale_log2 = (1.0f / std::sqrt(64.0f)) * 1.4426950408889634f;
        if (M <= INT32_MAX && W <= INT32_MAX && sdxl_hip::q_cross_attention_supported(p, w_fp8, compute_units())) {
            st = launch_status(
                sdxl_hip::launch_q_cross_attention(p, w_fp8, compute_units(), reinterpret_cast<hipStream_t>(stream)),
                "sdxl_cross_attn_sublayer");
            if (st != SDXL_STATUS_OK) return st;
            sdxl_linear_desc od{};
            od.m = M;
            od.n = W;
            od.k = W;
            od.w_dtype = SDXL_DTYPE_F16;
            return sdxl_linear(&od, q, w_out, nullptr, b_out, x, y, stream);
        }
    }

    if (act_fp8) st = sdxl_linear_e4m3(&qd, codes, code_scale, w_q, w_q_scale, nullptr, nullptr, q, stream);
    else st = sdxl_linear(&qd, hidden_ws, w_q, w_q_scale, nullptr, nullptr, q, stream);
    if (st != SDXL_STATUS_OK) return st;

    sdxl_attn_desc ad{};
    ad.batch = d->batch;
    ad.q_seq = d->seq;
    ad.k_seq = d->ctx_len;
    ad.heads = d->heads;
    ad.head_dim = 64;
    ad.k_row_stride = ad.v_row_stride = ldkv;
    ad.dtype = SDXL_DTYPE_F16;
    ad.backend = d->attn_backend;
    const char* kv_c = static_cast<const char*>(kv);
    st = sdxl_attn_fwd(&ad, q, kv_c, kv_c == nullptr ? nullptr : kv_c + W * 2, nullptr, hidden_ws, stream);
    if (st != SDXL_STATUS_OK) return st;

    sdxl_linear_desc od{};
    od.m = M;
    od.n = W;
    od.k = W;
    od.w_dtype = SDXL_DTYPE_F16;
    return sdxl_linear(&od, hidden_ws, w_out, nullptr, b_out, x, y, stream);
}

}  // extern "C"
