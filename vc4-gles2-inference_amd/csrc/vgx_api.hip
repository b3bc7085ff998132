// libvgx host side: contexts, weight upload, GEMV entry points, host helpers.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "vgx_internal.h"

// Key slots of vgx_logits_argmax_rms_noalloc: one u64 per workgroup of its
// LM-head launch, in static device memory instead of the group's allocation.
// Each device holds its own copy until the process ends; host code uses only
// the per-device address hipGetSymbolAddress returns (in host code the
// array's name is a stand-in, not a device address).
static constexpr int kScratchKeys = 4096;  // 32 KiB per device
static __device__ __align__(256) unsigned long long scratch[kScratchKeys];

namespace {
thread_local std::string g_last_error;

std::mutex g_scratch_mu;
std::vector<unsigned long long*> g_scratch_dev;  // by device ordinal

int scratch_keys_for(int device, unsigned long long** out) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if ((int)g_scratch_dev.size() <= device) g_scratch_dev.resize((size_t)device + 1, nullptr);
    if (!g_scratch_dev[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return vgx_hip_fail(e, "hipGetSymbolAddress(scratch)");
        g_scratch_dev[device] = static_cast<unsigned long long*>(p);
    }
    *out = g_scratch_dev[device];
    return VGX_OK;
}
}  // namespace

int vgx_fail(int status, const std::string& msg) {
    g_last_error = msg;
    return status;
}

int vgx_hip_fail(hipError_t e, const char* what) {
    g_last_error = std::string(what) + ": " + hipGetErrorString(e);
    return e == hipErrorOutOfMemory ? VGX_ENOMEM : VGX_EHIP;
}

extern "C" {

int vgx_abi_version(void) { return VGX_ABI_VERSION; }

const char* vgx_strerror(int status) {
    switch (status) {
        case VGX_OK: return "ok";
        case VGX_EINVAL: return "invalid argument";
        case VGX_EHIP: return "HIP runtime error";
        case VGX_ENOMEM: return "out of device memory";
        case VGX_ESTATE: return "call out of order";
        case VGX_ERANGE: return "out of range";
    }
    return "unknown status";
}

const char* vgx_last_error(void) { return g_last_error.c_str(); }

// ---------------------------------------------------------------------------
// context

int vgx_ctx_create(int device, vgx_ctx** out) {
    if (!out) return vgx_fail(VGX_EINVAL, "vgx_ctx_create: out is NULL");
    *out = nullptr;
    int n = 0;
    VGX_HIP(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return vgx_fail(VGX_EINVAL, "vgx_ctx_create: no such device");
    VGX_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    VGX_HIP(hipGetDeviceProperties(&prop, device));
    unsigned long long* keys = nullptr;
    const int st = scratch_keys_for(device, &keys);  // with the device current
    if (st != VGX_OK) return st;
    vgx_ctx* c = new vgx_ctx();
    c->device = device;
    c->num_cu = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    c->scratch_keys = keys;
    hipError_t e = hipStreamCreate(&c->own);
    if (e != hipSuccess) {
        delete c;
        return vgx_hip_fail(e, "hipStreamCreate");
    }
    c->stream = c->own;
    *out = c;
    return VGX_OK;
}

int vgx_ctx_destroy(vgx_ctx* ctx) {
    if (!ctx) return VGX_OK;
    if (ctx->ws) {
        (void)hipStreamSynchronize(ctx->stream);
        (void)hipFree(ctx->ws);
    }
    if (ctx->own) {
        (void)hipStreamSynchronize(ctx->own);
        (void)hipStreamDestroy(ctx->own);
    }
    delete ctx;
    return VGX_OK;
}

int vgx_ctx_set_stream(vgx_ctx* ctx, void* stream) {
    if (!ctx) return vgx_fail(VGX_EINVAL, "vgx_ctx_set_stream: ctx is NULL");
    ctx->stream = static_cast<hipStream_t>(stream);
    return VGX_OK;
}

void* vgx_ctx_stream(vgx_ctx* ctx) { return ctx ? static_cast<void*>(ctx->stream) : nullptr; }

int vgx_ctx_sync(vgx_ctx* ctx) {
    if (!ctx) return vgx_fail(VGX_EINVAL, "vgx_ctx_sync: ctx is NULL");
    VGX_HIP(hipSetDevice(ctx->device));
    VGX_HIP(hipStreamSynchronize(ctx->stream));
    return VGX_OK;
}

// ---------------------------------------------------------------------------
// weights

// The per-row scale every q8/t3 kernel multiplies by: the part-3 plane is
// re-quantised to 16 bits at upload (engine/src/gpu_upload.cpp:46-50: lrint in
// double, clamped to [0, 65535]) and the shader rebuilds (p16*ws)*(1/65536) in
// fp32 (wrow_scale, engine/src/shaders.cpp:364-371).  No plane: every row
// uses ws.
static void row_scales(int rows, float ws, const float* plane, std::vector<float>& wsr) {
    wsr.resize((size_t)rows);
    for (int r = 0; r < rows; ++r) {
        if (!plane) { wsr[r] = ws; continue; }
        long q = lrint((double)plane[r] * 65536.0);
        if (q < 0) q = 0;
        if (q > 65535) q = 65535;
        const float p16 = (float)q;
        const float t = p16 * ws;
        wsr[r] = t * (1.0f / 65536.0f);
    }
}

static int mat_finish(vgx_ctx* ctx, vgx_mat* m) {
    VGX_HIP(hipMalloc(&m->d_dev, sizeof(MatDev)));
    VGX_HIP(hipMemcpy(m->d_dev, &m->d, sizeof(MatDev), hipMemcpyHostToDevice));
    m->ctx = ctx;
    return VGX_OK;
}

int vgx_mat_upload(vgx_ctx* ctx, const vgx_weight_desc* w, vgx_mat** out) {
    if (!ctx || !w || !out) return vgx_fail(VGX_EINVAL, "vgx_mat_upload: NULL argument");
    *out = nullptr;
    const int rows = w->rows, cols = w->cols;
    if (rows <= 0 || cols <= 0) return vgx_fail(VGX_EINVAL, "vgx_mat_upload: empty shape");
    if (cols > 32768) return vgx_fail(VGX_EINVAL, "vgx_mat_upload: cols > 32768");
    if (!w->body) return vgx_fail(VGX_EINVAL, "vgx_mat_upload: body is NULL");
    const float mul = (w->scale_mul == 0.0f) ? 1.0f : w->scale_mul;
    VGX_HIP(hipSetDevice(ctx->device));

    size_t need = 0;
    switch (w->kind) {
        case VGX_Q8:
            if (cols % 16) return vgx_fail(VGX_EINVAL, "vgx_mat_upload: q8 cols must be a multiple of 16");
            need = (size_t)rows * cols;
            break;
        case VGX_Q4:
            if (cols % 32) return vgx_fail(VGX_EINVAL, "vgx_mat_upload: q4 cols must be a multiple of 32");
            if (!w->q4_scale || !w->q4_min) return vgx_fail(VGX_EINVAL, "vgx_mat_upload: q4 needs scale and min planes");
            need = (size_t)rows * cols / 2;
            break;
        case VGX_T3:
            // the packer pads a row to a multiple of 8 columns
            // (engine/tools/mmcf_hf.py:151-156): cols/8 texels a row pair
            if (cols % 8) return vgx_fail(VGX_EINVAL, "vgx_mat_upload: t3 cols must be a multiple of 8");
            if (!w->row_plane) return vgx_fail(VGX_EINVAL, "vgx_mat_upload: t3 needs its part-3 row plane");
            need = (size_t)((rows + 1) / 2) * (size_t)(cols / 8) * 4;
            break;
        default:
            return vgx_fail(VGX_EINVAL, "vgx_mat_upload: unknown kind");
    }
    if (w->body_bytes != need)
        return vgx_fail(VGX_EINVAL, "vgx_mat_upload: body is " + std::to_string(w->body_bytes) +
                                        " bytes, the shape needs " + std::to_string(need));

    vgx_mat* m = new vgx_mat();
    m->d.kind = w->kind;
    m->d.rows = rows;
    m->d.cols = cols;
    m->body_bytes = need;
    // t3 texel rows padded to whole 32-column chunks (t3_rstride)
    const size_t t3_src = (size_t)(cols / 8) * 4, t3_dst = w->kind == VGX_T3 ? (size_t)t3_rstride(cols) : 0;
    m->body_alloc_bytes = w->kind == VGX_T3 ? (size_t)((rows + 1) / 2) * t3_dst : need;
    hipError_t e = hipMalloc(&m->body_alloc, m->body_alloc_bytes);
    if (e != hipSuccess) { delete m; return vgx_hip_fail(e, "hipMalloc(body)"); }
    m->d.body = static_cast<const uint8_t*>(m->body_alloc);

    if (w->kind == VGX_Q8 && !w->prebiased) {
        // q8i8 bodies are biased to q8u8 once here, as the reference did for its
        // legacy signed checkpoints at upload time.
        std::vector<uint8_t> tmp(need);
        const uint8_t* src = static_cast<const uint8_t*>(w->body);
        for (size_t i = 0; i < need; ++i) tmp[i] = src[i] ^ 0x80u;
        e = hipMemcpy(m->body_alloc, tmp.data(), need, hipMemcpyHostToDevice);
    } else if (w->kind == VGX_T3 && t3_dst != t3_src) {
        e = hipMemset(m->body_alloc, 0, m->body_alloc_bytes);
        if (e == hipSuccess)
            e = hipMemcpy2D(m->body_alloc, t3_dst, w->body, t3_src, t3_src, (size_t)((rows + 1) / 2),
                            hipMemcpyHostToDevice);
    } else {
        e = hipMemcpy(m->body_alloc, w->body, need, hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) { vgx_mat_free(m); return vgx_hip_fail(e, "hipMemcpy(body)"); }
    m->body_bytes = m->body_alloc_bytes;  // the bytes in HBM a kernel reads

    if (w->kind == VGX_Q4) {
        const size_t groups = (size_t)rows * (cols / 32);
        std::vector<uint32_t> sm(groups);
        for (size_t i = 0; i < groups; ++i)
            sm[i] = (uint32_t)(uint16_t)w->q4_scale[i] | ((uint32_t)(uint16_t)w->q4_min[i] << 16);
        m->plane_bytes = groups * 4;
        e = hipMalloc(&m->plane_alloc, m->plane_bytes);
        if (e == hipSuccess) e = hipMemcpy(m->plane_alloc, sm.data(), m->plane_bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) { vgx_mat_free(m); return vgx_hip_fail(e, "q4 planes"); }
        m->d.sm = static_cast<const uint32_t*>(m->plane_alloc);
        m->d.ps = w->scale * mul;
    } else {
        // t3: a +-1 level carries 127 steps (engine/src/model.cpp:927)
        const float ws = (w->kind == VGX_T3 ? w->scale * 127.0f : w->scale) * mul;
        std::vector<float> wsr;
        row_scales(rows, ws, w->row_plane, wsr);
        m->plane_bytes = (size_t)rows * 4;
        e = hipMalloc(&m->plane_alloc, m->plane_bytes);
        if (e == hipSuccess) e = hipMemcpy(m->plane_alloc, wsr.data(), m->plane_bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) { vgx_mat_free(m); return vgx_hip_fail(e, "row scales"); }
        m->d.wsr = static_cast<const float*>(m->plane_alloc);
    }
    int st = mat_finish(ctx, m);
    if (st != VGX_OK) { vgx_mat_free(m); return st; }
    *out = m;
    return VGX_OK;
}

int vgx_mat_clone(vgx_ctx* ctx, const vgx_mat* src, vgx_mat** out) {
    if (!ctx || !src || !out) return vgx_fail(VGX_EINVAL, "vgx_mat_clone: NULL argument");
    *out = nullptr;
    VGX_HIP(hipSetDevice(ctx->device));
    vgx_mat* m = new vgx_mat();
    m->d = src->d;
    m->body_bytes = src->body_bytes;
    m->body_alloc_bytes = src->body_alloc_bytes;
    m->plane_bytes = src->plane_bytes;
    hipError_t e = hipMalloc(&m->body_alloc, m->body_alloc_bytes);
    if (e == hipSuccess)
        e = hipMemcpyAsync(m->body_alloc, src->body_alloc, m->body_alloc_bytes, hipMemcpyDeviceToDevice, ctx->stream);
    if (e == hipSuccess) e = hipMalloc(&m->plane_alloc, m->plane_bytes);
    if (e == hipSuccess) e = hipMemcpyAsync(m->plane_alloc, src->plane_alloc, m->plane_bytes, hipMemcpyDeviceToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) { vgx_mat_free(m); return vgx_hip_fail(e, "vgx_mat_clone"); }
    m->d.body = static_cast<const uint8_t*>(m->body_alloc);
    if (m->d.kind == VGX_Q4) m->d.sm = static_cast<const uint32_t*>(m->plane_alloc);
    else m->d.wsr = static_cast<const float*>(m->plane_alloc);
    int st = mat_finish(ctx, m);
    if (st != VGX_OK) { vgx_mat_free(m); return st; }
    *out = m;
    return VGX_OK;
}

int vgx_mat_concat(vgx_ctx* ctx, int n, vgx_mat* const* mats, vgx_mat** out) {
    if (!ctx || !mats || !out || n <= 0) return vgx_fail(VGX_EINVAL, "vgx_mat_concat: NULL argument or n <= 0");
    *out = nullptr;
    const MatDev& a = mats[0]->d;
    if (a.kind == VGX_Q4) return vgx_fail(VGX_EINVAL, "vgx_mat_concat: q4 scales are per matrix; q8 and t3 only");
    size_t body = 0, plane = 0;
    long long rows = 0;
    for (int i = 0; i < n; ++i) {
        if (!mats[i]) return vgx_fail(VGX_EINVAL, "vgx_mat_concat: NULL matrix");
        const MatDev& d = mats[i]->d;
        if (d.kind != a.kind || d.cols != a.cols) return vgx_fail(VGX_EINVAL, "vgx_mat_concat: kinds or cols differ");
        if (d.kind == VGX_T3 && (d.rows % 2) && i != n - 1)
            return vgx_fail(VGX_EINVAL, "vgx_mat_concat: a t3 matrix before the last has an odd row count");
        body += mats[i]->body_bytes;
        plane += mats[i]->plane_bytes;
        rows += d.rows;
    }
    if (rows > (1 << 30)) return vgx_fail(VGX_EINVAL, "vgx_mat_concat: too many rows");
    VGX_HIP(hipSetDevice(ctx->device));
    vgx_mat* m = new vgx_mat();
    m->d = a;
    m->d.rows = (int)rows;
    m->d.out_off = m->d.blk_off = 0;
    m->body_bytes = body;
    m->body_alloc_bytes = body;
    m->plane_bytes = plane;
    hipError_t e = hipMalloc(&m->body_alloc, body);
    if (e == hipSuccess) e = hipMalloc(&m->plane_alloc, plane);
    size_t bo = 0, po = 0;
    for (int i = 0; i < n && e == hipSuccess; ++i) {
        e = hipMemcpyAsync(static_cast<uint8_t*>(m->body_alloc) + bo, mats[i]->body_alloc, mats[i]->body_bytes,
                           hipMemcpyDeviceToDevice, ctx->stream);
        if (e == hipSuccess)
            e = hipMemcpyAsync(static_cast<uint8_t*>(m->plane_alloc) + po, mats[i]->plane_alloc,
                               mats[i]->plane_bytes, hipMemcpyDeviceToDevice, ctx->stream);
        bo += mats[i]->body_bytes;
        po += mats[i]->plane_bytes;
    }
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) { vgx_mat_free(m); return vgx_hip_fail(e, "vgx_mat_concat"); }
    m->d.body = static_cast<const uint8_t*>(m->body_alloc);
    m->d.wsr = static_cast<const float*>(m->plane_alloc);
    int st = mat_finish(ctx, m);
    if (st != VGX_OK) { vgx_mat_free(m); return st; }
    *out = m;
    return VGX_OK;
}

int vgx_mat_free(vgx_mat* m) {
    if (!m) return VGX_OK;
    if (m->body_alloc) (void)hipFree(m->body_alloc);
    if (m->plane_alloc) (void)hipFree(m->plane_alloc);
    if (m->d_dev) (void)hipFree(m->d_dev);
    delete m;
    return VGX_OK;
}

int vgx_mat_shape(const vgx_mat* m, int* kind, int* rows, int* cols) {
    if (!m) return vgx_fail(VGX_EINVAL, "vgx_mat_shape: NULL matrix");
    if (kind) *kind = m->d.kind;
    if (rows) *rows = m->d.rows;
    if (cols) *cols = m->d.cols;
    return VGX_OK;
}

size_t vgx_mat_weight_bytes(const vgx_mat* m) { return m ? m->body_bytes + m->plane_bytes : 0; }

int vgx_dequant(vgx_ctx* ctx, const vgx_mat* m, float* out) {
    if (!ctx || !m || !out) return vgx_fail(VGX_EINVAL, "vgx_dequant: NULL argument");
    VGX_HIP(hipSetDevice(ctx->device));
    return vgx_dequant_launch(m->d, out, ctx->stream);
}

// ---------------------------------------------------------------------------
// GEMV entry points

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Workgroups of a GEMV launch: one per row tile up to 4 per CU; past that each
// workgroup loops over tiles (x is staged once per workgroup).  4 per CU was
// the best of 2..16 on HBM-streamed q8 and q4 launches.  A launch of at most
// kGridOnePass tiles a CU still takes one workgroup per tile: capped, its
// last tiles were streamed by a few workgroups after all the others had
// finished (the 73,448-row LM head: 1148 tiles, 124 of them a second pass).
static constexpr int kGridOnePass = 5;
static int gemv_grid(const vgx_ctx* ctx, int tiles) {
    if (tiles <= kGridOnePass * ctx->num_cu) return tiles;
    return 4 * ctx->num_cu;
}

static int launch_single(vgx_ctx* ctx, const vgx_mat* W, const int16_t* x, const float* xf,
                         const int16_t* res, void* y, const vgx_mat* W3, int hs, int split,
                         const int16_t* rw = nullptr, float eps = 0.0f) {
    if (!ctx || !W || !y) return vgx_fail(VGX_EINVAL, "gemv: NULL argument");
    if (!x && !xf) return vgx_fail(VGX_EINVAL, "gemv: x is NULL");
    if (!aligned16(x ? (const void*)x : (const void*)xf))
        return vgx_fail(VGX_EINVAL, "gemv: x must be 16-byte aligned");
    if (rw && !aligned16(rw)) return vgx_fail(VGX_EINVAL, "gemv: the RMSNorm weight must be 16-byte aligned");
    if (rw && !(eps > 0.0f)) return vgx_fail(VGX_EINVAL, "gemv: the RMSNorm epsilon must be positive");
    VGX_HIP(hipSetDevice(ctx->device));
    GemvLaunch L{};
    int lpr, ri, rpb;
    vgx_gemv_plan(W->d.kind, W->d.rows, W->d.cols, ctx->num_cu, &lpr, &ri, &rpb);
    const int units = W->d.kind == VGX_T3 ? (W->d.rows + 1) / 2 : W->d.rows;
    L.md[0] = W->d;
    L.mats = W->d_dev;
    L.nmat = 1;
    L.blocks = (units + rpb - 1) / rpb;
    L.grid = gemv_grid(ctx, L.blocks);
    L.x = x;
    L.xf = xf;
    L.res = res;
    L.y = y;
    L.gate = W3 ? 1 : 0;
    if (W3) L.md3 = W3->d;
    L.hs = hs;
    L.split_chunk = split;
    L.kind = W->d.kind;
    L.cols = W->d.cols;
    L.lpr = lpr;
    L.ri = ri;
    L.rw = rw;
    L.eps = eps;
    return vgx_gemv_launch(L, ctx->stream);
}

int vgx_gemv(vgx_ctx* ctx, const vgx_mat* W, const int16_t* x, const int16_t* res, int16_t* y) {
    return launch_single(ctx, W, x, nullptr, res, y, nullptr, 0, 0);
}

int vgx_gemv_f32(vgx_ctx* ctx, const vgx_mat* W, const float* x, float* y) {
    return launch_single(ctx, W, nullptr, x, nullptr, y, nullptr, 0, 0);
}

int vgx_gemv_add_split(vgx_ctx* ctx, const vgx_mat* W, int split, const int16_t* x,
                       const int16_t* res, int16_t* y) {
    if (!W || !res) return vgx_fail(VGX_EINVAL, "vgx_gemv_add_split: NULL argument");
    const int unit = W->d.kind == VGX_Q8 ? 16 : 32;
    if (split <= 0 || split >= W->d.cols || split % unit)
        return vgx_fail(VGX_EINVAL, "vgx_gemv_add_split: split must be inside cols and a multiple of " +
                                        std::to_string(unit));
    return launch_single(ctx, W, x, nullptr, res, y, nullptr, 0, split / unit);
}

int vgx_ffn_gate(vgx_ctx* ctx, const vgx_mat* W1, const vgx_mat* W3, const int16_t* x, int hs,
                 int16_t* h) {
    if (!W1 || !W3) return vgx_fail(VGX_EINVAL, "vgx_ffn_gate: NULL matrix");
    if (W1->d.kind != W3->d.kind || W1->d.rows != W3->d.rows || W1->d.cols != W3->d.cols)
        return vgx_fail(VGX_EINVAL, "vgx_ffn_gate: W1 and W3 differ in kind or shape");
    if (hs < 0 || hs > 5) return vgx_fail(VGX_EINVAL, "vgx_ffn_gate: hs outside 0..5");
    return launch_single(ctx, W1, x, nullptr, nullptr, h, W3, hs, 0);
}

int vgx_gemv_rms(vgx_ctx* ctx, const vgx_mat* W, const int16_t* x, const int16_t* rms_w, float eps,
                 const int16_t* res, int16_t* y) {
    if (!rms_w) return vgx_fail(VGX_EINVAL, "vgx_gemv_rms: NULL RMSNorm weight");
    return launch_single(ctx, W, x, nullptr, res, y, nullptr, 0, 0, rms_w, eps);
}

int vgx_ffn_gate_rms(vgx_ctx* ctx, const vgx_mat* W1, const vgx_mat* W3, const int16_t* x,
                     const int16_t* rms_w, float eps, int hs, int16_t* h) {
    if (!W1 || !W3) return vgx_fail(VGX_EINVAL, "vgx_ffn_gate_rms: NULL matrix");
    if (!rms_w) return vgx_fail(VGX_EINVAL, "vgx_ffn_gate_rms: NULL RMSNorm weight");
    if (W1->d.kind != W3->d.kind || W1->d.rows != W3->d.rows || W1->d.cols != W3->d.cols)
        return vgx_fail(VGX_EINVAL, "vgx_ffn_gate_rms: W1 and W3 differ in kind or shape");
    if (hs < 0 || hs > 5) return vgx_fail(VGX_EINVAL, "vgx_ffn_gate_rms: hs outside 0..5");
    return launch_single(ctx, W1, x, nullptr, nullptr, h, W3, hs, 0, rms_w, eps);
}

// ---------------------------------------------------------------------------
// groups

int vgx_group_create(vgx_ctx* ctx, int n, const vgx_mat* const* mats, vgx_group** out) {
    if (!ctx || !mats || !out || n <= 0) return vgx_fail(VGX_EINVAL, "vgx_group_create: bad argument");
    *out = nullptr;
    const int kind = mats[0]->d.kind, cols = mats[0]->d.cols;
    int maxrows = 0;
    for (int i = 0; i < n; ++i) {
        if (!mats[i]) return vgx_fail(VGX_EINVAL, "vgx_group_create: NULL matrix");
        if (mats[i]->d.kind != kind || mats[i]->d.cols != cols)
            return vgx_fail(VGX_EINVAL, "vgx_group_create: matrices differ in kind or cols");
        if (mats[i]->d.rows > maxrows) maxrows = mats[i]->d.rows;
    }
    VGX_HIP(hipSetDevice(ctx->device));
    vgx_group* g = new vgx_group();
    g->ctx = ctx;
    g->n = n;
    g->kind = kind;
    g->cols = cols;
    long long total_rows = 0;
    for (int i = 0; i < n; ++i) total_rows += mats[i]->d.rows;
    int lpr, ri, rpb;
    // plan on the whole group: it is one launch
    vgx_gemv_plan(kind, (int)(total_rows > (1 << 30) ? (1 << 30) : total_rows), cols, ctx->num_cu, &lpr, &ri, &rpb);
    g->lpr = lpr;
    g->ri = ri;
    std::vector<MatDev> ds((size_t)n);
    int blk = 0, off = 0;
    for (int i = 0; i < n; ++i) {
        ds[i] = mats[i]->d;
        ds[i].out_off = off;
        ds[i].blk_off = blk;
        const int units = kind == VGX_T3 ? (ds[i].rows + 1) / 2 : ds[i].rows;
        blk += (units + rpb - 1) / rpb;
        off += ds[i].rows;
    }
    g->blocks = blk;
    g->rows = off;
    g->host = ds;
    // equal row counts: the tile -> matrix lookup is a division
    bool uniform = true;
    for (int i = 1; i < n; ++i) uniform = uniform && ds[i].rows == ds[0].rows;
    g->bpm = uniform ? blk / n : 0;
    hipError_t e = hipMalloc(&g->d_dev, sizeof(MatDev) * (size_t)n);
    if (e == hipSuccess) e = hipMemcpy(g->d_dev, ds.data(), sizeof(MatDev) * (size_t)n, hipMemcpyHostToDevice);
    // a key slot per workgroup of the largest grid a launch takes (gemv_grid)
    g->nkeys = kGridOnePass * (ctx->num_cu > 0 ? ctx->num_cu : 256);
    if (e == hipSuccess) e = hipMalloc(&g->keys, sizeof(unsigned long long) * (size_t)g->nkeys);
    if (e != hipSuccess) { vgx_group_free(g); return vgx_hip_fail(e, "vgx_group_create"); }
    *out = g;
    return VGX_OK;
}

int vgx_group_free(vgx_group* g) {
    if (!g) return VGX_OK;
    if (g->d_dev) (void)hipFree(g->d_dev);
    if (g->keys) (void)hipFree(g->keys);
    delete g;
    return VGX_OK;
}

int vgx_group_rows(const vgx_group* g) { return g ? g->rows : 0; }

int vgx_gemv_plan_info(vgx_ctx* ctx, const vgx_mat* W, int* lanes_per_row, int* rows_per_lane) {
    if (!ctx || !W) return vgx_fail(VGX_EINVAL, "vgx_gemv_plan_info: NULL argument");
    int lpr, ri, rpb;
    vgx_gemv_plan(W->d.kind, W->d.rows, W->d.cols, ctx->num_cu, &lpr, &ri, &rpb);
    if (lanes_per_row) *lanes_per_row = lpr;
    if (rows_per_lane) *rows_per_lane = ri;
    return VGX_OK;
}

int vgx_group_plan_info(const vgx_group* g, int* lanes_per_row, int* rows_per_lane) {
    if (!g) return vgx_fail(VGX_EINVAL, "vgx_group_plan_info: NULL group");
    if (lanes_per_row) *lanes_per_row = g->lpr;
    if (rows_per_lane) *rows_per_lane = g->ri;
    return VGX_OK;
}

static int launch_group(vgx_ctx* ctx, const vgx_group* g, const int16_t* x, const float* xf, void* y,
                        const int16_t* rw = nullptr, float eps = 0.0f, int* argmax_out = nullptr,
                        const StepTail* tail = nullptr, bool static_keys = false) {
    if (!ctx || !g || !y || (!x && !xf)) return vgx_fail(VGX_EINVAL, "gemv_group: NULL argument");
    if (!aligned16(x ? (const void*)x : (const void*)xf))
        return vgx_fail(VGX_EINVAL, "gemv_group: x must be 16-byte aligned");
    if (rw && !aligned16(rw)) return vgx_fail(VGX_EINVAL, "gemv_group: the RMSNorm weight must be 16-byte aligned");
    if (rw && !(eps > 0.0f)) return vgx_fail(VGX_EINVAL, "gemv_group: the RMSNorm epsilon must be positive");
    VGX_HIP(hipSetDevice(ctx->device));
    GemvLaunch L{};
    L.mats = g->d_dev;
    L.nmat = g->n;
    if (g->n <= kInlineMats)
        for (int i = 0; i < g->n; ++i) L.md[i] = g->host[i];
    L.blocks = g->blocks;
    L.grid = gemv_grid(ctx, g->blocks);
    L.bpm = g->bpm;
    L.x = x;
    L.xf = xf;
    L.y = y;
    L.kind = g->kind;
    L.cols = g->cols;
    L.lpr = g->lpr;
    L.ri = g->ri;
    L.rw = rw;
    L.eps = eps;
    L.argmax_out = argmax_out;
    L.argmax_key = static_keys ? ctx->scratch_keys : g->keys;
    L.nkeys = static_keys ? kScratchKeys : g->nkeys;
    if (static_keys && L.grid > kScratchKeys)
        return vgx_fail(VGX_ERANGE, "vgx_logits_argmax_rms_noalloc: the launch takes " + std::to_string(L.grid) +
                                        " workgroups, the static key slots hold " + std::to_string(kScratchKeys));
    L.total_rows = g->rows;
    if (tail) L.tail = *tail;
    return vgx_gemv_launch(L, ctx->stream);
}

int vgx_gemv_group(vgx_ctx* ctx, const vgx_group* g, const int16_t* x, int16_t* y) {
    return launch_group(ctx, g, x, nullptr, y);
}

int vgx_gemv_group_f32(vgx_ctx* ctx, const vgx_group* g, const float* x, float* y) {
    return launch_group(ctx, g, nullptr, x, y);
}

int vgx_logits_argmax(vgx_ctx* ctx, const vgx_group* g, const int16_t* x, int16_t* logits, int* token) {
    if (!token || !logits) return vgx_fail(VGX_EINVAL, "vgx_logits_argmax: NULL output");
    int st = launch_group(ctx, g, x, nullptr, logits);
    if (st != VGX_OK) return st;
    return vgx_argmax_launch(logits, g->rows, 1, token, ctx->stream);
}

int vgx_argmax_rows(vgx_ctx* ctx, int nrows, int n, const int16_t* v, int* tokens) {
    if (!ctx || !v || !tokens) return vgx_fail(VGX_EINVAL, "vgx_argmax_rows: NULL argument");
    if (nrows <= 0 || nrows > 65535 || n <= 0) return vgx_fail(VGX_EINVAL, "vgx_argmax_rows: empty or oversized shape");
    VGX_HIP(hipSetDevice(ctx->device));
    return vgx_argmax_launch(v, n, nrows, tokens, ctx->stream);
}

int vgx_gemv_group_rms(vgx_ctx* ctx, const vgx_group* g, const int16_t* x, const int16_t* rms_w, float eps,
                       int16_t* y) {
    if (!rms_w) return vgx_fail(VGX_EINVAL, "vgx_gemv_group_rms: NULL RMSNorm weight");
    return launch_group(ctx, g, x, nullptr, y, rms_w, eps);
}

int vgx_logits_argmax_rms(vgx_ctx* ctx, const vgx_group* g, const int16_t* x, const int16_t* rms_w, float eps,
                          int16_t* logits, int* token) {
    if (!token || !logits) return vgx_fail(VGX_EINVAL, "vgx_logits_argmax_rms: NULL output");
    if (!rms_w) return vgx_fail(VGX_EINVAL, "vgx_logits_argmax_rms: NULL RMSNorm weight");
    return launch_group(ctx, g, x, nullptr, logits, rms_w, eps, token);
}

int vgx_logits_argmax_rms_noalloc(vgx_ctx* ctx, const vgx_group* g, const int16_t* x, const int16_t* rms_w,
                                  float eps, int16_t* logits, int* token) {
    if (!token || !logits) return vgx_fail(VGX_EINVAL, "vgx_logits_argmax_rms_noalloc: NULL output");
    if (!rms_w) return vgx_fail(VGX_EINVAL, "vgx_logits_argmax_rms_noalloc: NULL RMSNorm weight");
    if (!ctx || !ctx->scratch_keys) return vgx_fail(VGX_EINVAL, "vgx_logits_argmax_rms_noalloc: no context");
    return launch_group(ctx, g, x, nullptr, logits, rms_w, eps, token, nullptr, true);
}

int vgx_logits_argmax_step(vgx_ctx* ctx, const vgx_group* g, const int16_t* x, const int16_t* rms_w, float eps,
                           int16_t* logits, int* token, int* pos, int* hist, int hist_len, const int8_t* emb,
                           const float* emb_scale, int vocab, int dim, int16_t* x_next) {
    if (!token || !logits) return vgx_fail(VGX_EINVAL, "vgx_logits_argmax_step: NULL output");
    if (!rms_w) return vgx_fail(VGX_EINVAL, "vgx_logits_argmax_step: NULL RMSNorm weight");
    if (!pos || !hist || !emb || !emb_scale || !x_next)
        return vgx_fail(VGX_EINVAL, "vgx_logits_argmax_step: NULL step argument");
    if (hist_len <= 0 || vocab <= 0 || dim <= 0) return vgx_fail(VGX_EINVAL, "vgx_logits_argmax_step: empty shape");
    const StepTail t{pos, hist, hist_len, emb, emb_scale, vocab, dim, x_next};
    return launch_group(ctx, g, x, nullptr, logits, rms_w, eps, token, &t);
}

// ---------------------------------------------------------------------------
// host helpers

void vgx_quantize_act(const float* v, int n, int16_t* q) {
    for (int i = 0; i < n; ++i) {
        long r = lrintf(v[i] * 256.0f);
        q[i] = (int16_t)(r < -32768 ? -32768 : r > 32767 ? 32767 : r);
    }
}

void vgx_x_pack_i16_2(const float* v, int n, uint8_t* out) {
    const int texels = (n + 1) / 2;
    for (int t = 0; t < texels; ++t) {
        int16_t q[2] = {0, 0};
        vgx_quantize_act(&v[2 * t], (2 * t + 1 < n) ? 2 : 1, q);
        for (int k = 0; k < 2; ++k) {
            const uint16_t u = (uint16_t)q[k];
            out[4 * t + 2 * k] = (uint8_t)(u >> 8);
            out[4 * t + 2 * k + 1] = (uint8_t)u;
        }
    }
}

}  // extern "C"
