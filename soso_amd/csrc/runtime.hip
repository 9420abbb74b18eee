// runtime.hip -- the C ABI of include/soso_hip.h: handle, resident-weight
// registry keyed by tensor name, host<->device staging, stats and errors.
//
// Mirrors the contract of soso-llm-core's GpuDispatch
// (crates/soso-llm-core/src/gpu.rs:338-737) as its CUDA implementor keeps it
// (crates/soso-llm-api/src/cuda.rs): upload on a key's first use, remember a
// declined key forever, synchronous results, never abort.
#include "internal.hpp"

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstring>
#include <new>


// The scratch of soso_hip_moe_ffn_dev_noalloc: one array per GPU for the
// life of the process.  Host code uses only the device address that
// soso_hip_create looks up for its GPU (h->fixed_scratch), never this name.
static __device__ __align__(256) unsigned char scratch[SOSO_HIP_MOE_NOALLOC_SCRATCH_BYTES];

int set_err(soso_hip *h, int code, const std::string &msg)
{
    if (h) h->err = msg;
    return code;
}

int hip_check(soso_hip *h, hipError_t e, const char *what)
{
    if (e == hipSuccess) return SOSO_HIP_OK;
    // hipGetLastError() reports the last failing runtime call of this thread,
    // not only launches: clear it so a later launch check sees its own status.
    (void)hipGetLastError();
    return set_err(h, SOSO_HIP_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

int hip_release(soso_hip *h, hipError_t e, const char *what)
{
    if (e == hipSuccess) return SOSO_HIP_OK;
    (void)hipGetLastError();
    if (h) h->err += (h->err.empty() ? "" : "; ") + std::string(what) + ": " + hipGetErrorString(e);
    return SOSO_HIP_ERR_DEVICE;
}

// the first failure of a sequence of release calls
static int first_fail(int a, int b) { return a != SOSO_HIP_OK ? a : b; }

static bool any_graph(const soso_hip *h)
{
    for (hipGraphExec_t g : h->graphs)
        if (g) return true;
    return false;
}

// Scratch slot `slot` of at least `bytes`, or null.  Growing it inside graph
// capture is refused (null): it would synchronise and allocate within the
// capture.  While any graph exists the outgrown buffer is retired instead of
// freed, since a graph may hold it as a kernel argument.
// Pinned host staging, grown on demand (hipHostMalloc: new pinned memory,
// never registration of existing memory); freed with the handle.
void *pinned_get(soso_hip *h, size_t bytes)
{
    if (bytes <= h->pinned_cap) return h->pinned;
    if (h->pinned && hip_release(h, hipHostFree(h->pinned), "free pinned staging") != SOSO_HIP_OK) {
        h->pinned = nullptr;
        h->pinned_cap = 0;
        return nullptr;
    }
    h->pinned = nullptr;
    h->pinned_cap = 0;
    const size_t cap = std::max<size_t>(bytes, 1u << 20);
    if (hipHostMalloc(&h->pinned, cap, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        h->pinned = nullptr;
        return nullptr;
    }
    h->pinned_cap = cap;
    return h->pinned;
}

void *scratch_get(soso_hip *h, int slot, size_t bytes)
{
    if (bytes == 0) bytes = 16;
    if (h->scratch_cap[slot] >= bytes) return h->scratch[slot];
    if (h->capturing) return nullptr;
    if (h->scratch[slot]) {
        if (any_graph(h)) {
            h->retired.push_back(h->scratch[slot]);
        } else {
            (void)hipStreamSynchronize(h->stream);
            (void)hipFree(h->scratch[slot]);
        }
        h->scratch[slot] = nullptr;
        h->scratch_cap[slot] = 0;
    }
    size_t cap = bytes + bytes / 4 + 4096;
    void *p = nullptr;
    if (hipMalloc(&p, cap) != hipSuccess) return nullptr;
    h->scratch[slot] = p;
    h->scratch_cap[slot] = cap;
    return p;
}

static void free_retired(soso_hip *h)
{
    if (h->retired.empty()) return;
    (void)hipStreamSynchronize(h->stream);
    for (void *p : h->retired) (void)hipFree(p);
    h->retired.clear();
}

namespace {

struct CallClock {
    soso_hip *h;
    std::chrono::steady_clock::time_point t0;
    explicit CallClock(soso_hip *hh) : h(hh), t0(std::chrono::steady_clock::now()) {}
    void done()
    {
        h->stats.launches++;
        h->stats.total_ns +=
            (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - t0)
                .count();
    }
};

bool dtype_ok(uint8_t d)
{
    return d == SOSO_HIP_DTYPE_F32 || d == SOSO_HIP_DTYPE_Q8_0 || d == SOSO_HIP_DTYPE_Q4_K || d == SOSO_HIP_DTYPE_Q6_K;
}

int make_current(soso_hip *h) { return hip_check(h, hipSetDevice(h->device), "hipSetDevice"); }

// Registers a weight from raw bytes already on the device (or uploads host
// bytes first).  Returns 1 and sets *out, 0 when declined, <0 on error.
int register_weight(soso_hip *h, const std::string &key, const void *raw, bool raw_on_device, size_t w_len,
                    uint8_t dtype, size_t rows, size_t cols, Weight **out)
{
    Weight w;
    w.dtype = dtype;
    w.rows = rows;
    w.cols = cols;
    const size_t kc = kernel_cols(dtype, cols);
    w.kcols = kc != cols ? kc : 0;
    const size_t rb = fmt_row_bytes(dtype, cols);
    if (!dtype_ok(dtype) || !upload_shape_ok(dtype, rows, cols) || rb == 0 || w_len != rows * rb || !raw) {
        w.declined = true;
        h->weights[key] = w;
        h->stats.weights_declined++;
        return set_err(h, SOSO_HIP_DECLINED, "weight " + key + ": dtype/shape not handled here");
    }
    const size_t bytes = rows * packed_row_stride(dtype, kc);
    if (h->used + bytes > h->budget) {
        w.declined = true;
        h->weights[key] = w;
        h->stats.weights_declined++;
        return set_err(h, SOSO_HIP_DECLINED, "weight " + key + ": over the memory budget");
    }
    void *dev = nullptr;
    if (hipMalloc(&dev, bytes) != hipSuccess) {
        w.declined = true;
        h->weights[key] = w;
        h->stats.weights_declined++;
        return set_err(h, SOSO_HIP_DECLINED, "weight " + key + ": device allocation failed");
    }
    const void *raw_dev = raw;
    void *tmp = nullptr;
    int rc = SOSO_HIP_OK;
    if (!raw_on_device) {
        if (hipMalloc(&tmp, w_len) != hipSuccess) {
            set_err(h, SOSO_HIP_ERR_NOMEM, "weight " + key + ": staging allocation failed");
            (void)hip_release(h, hipFree(dev), "free weight");
            return SOSO_HIP_ERR_NOMEM;
        }
        rc = hip_check(h, hipMemcpyAsync(tmp, raw, w_len, hipMemcpyHostToDevice, h->stream), "upload weight");
        raw_dev = tmp;
    }
    if (rc == SOSO_HIP_OK) rc = repack_weight(h, dtype, raw_dev, dev, rows, cols);
    if (rc == SOSO_HIP_OK) rc = hip_check(h, hipStreamSynchronize(h->stream), "repack sync");
    if (tmp) rc = first_fail(rc, hip_release(h, hipFree(tmp), "free staging"));
    if (rc != SOSO_HIP_OK) {
        (void)hip_release(h, hipFree(dev), "free weight");
        return rc;
    }
    w.dev = dev;
    w.bytes = bytes;
    h->used += bytes;
    h->stats.weight_bytes_resident += bytes;
    h->stats.weights_resident++;
    auto it = h->weights.emplace(key, w).first;
    *out = &it->second;
    return SOSO_HIP_OK;
}

// Finds or uploads the weight for `key`; same declines as cuda.rs:2365-2384.
int get_weight(soso_hip *h, const char *key, size_t key_len, const uint8_t *w, size_t w_len, uint8_t dtype,
               size_t rows, size_t cols, Weight **out)
{
    std::string k(key, key_len);
    auto it = h->weights.find(k);
    if (it != h->weights.end()) {
        Weight &e = it->second;
        if (e.declined) return SOSO_HIP_DECLINED;
        if (e.rows != rows || e.cols != cols || (dtype != 0 && e.dtype != dtype))
            return set_err(h, SOSO_HIP_DECLINED, "weight " + k + ": shape/dtype differs from the resident copy");
        *out = &e;
        return SOSO_HIP_OK;
    }
    if (!w || dtype == 0) return set_err(h, SOSO_HIP_DECLINED, "weight " + k + ": not resident and no bytes given");
    return register_weight(h, k, w, false, w_len, dtype, rows, cols, out);
}

Weight *find_weight(soso_hip *h, const char *key, size_t key_len)
{
    auto it = h->weights.find(std::string(key, key_len));
    if (it == h->weights.end() || it->second.declined) return nullptr;
    return &it->second;
}

int moe_free(soso_hip *h, MoeLayer &m)
{
    int rc = hip_release(h, hipStreamSynchronize(h->stream), "moe free sync");
    if (m.tab) rc = first_fail(rc, hip_release(h, hipFree(m.tab), "free expert table"));
    if (m.tiled) rc = first_fail(rc, hip_release(h, hipFree(m.tiled), "free tiled table"));
    if (m.tiled_mem) {
        rc = first_fail(rc, hip_release(h, hipFree(m.tiled_mem), "free tiled experts"));
        h->used -= m.tiled_bytes;
    }
    m.tab = m.tiled = nullptr;
    m.tiled_mem = nullptr;
    m.tiled_bytes = 0;
    return rc;
}

int decode_free(soso_hip *h, DecodeModel &m)
{
    int rc = hip_release(h, hipStreamSynchronize(h->stream), "decode free sync");
    for (Weight &w : m.owned) {
        if (w.dev) {
            rc = first_fail(rc, hip_release(h, hipFree(w.dev), "free fused weight"));
            h->used -= w.bytes;
        }
    }
    m.owned.clear();
    if (m.kcache) rc = first_fail(rc, hip_release(h, hipFree(m.kcache), "free KV cache"));
    if (m.mem) rc = first_fail(rc, hip_release(h, hipFree(m.mem), "free step buffers"));
    if (m.moe_mem) rc = first_fail(rc, hip_release(h, hipFree(m.moe_mem), "free MoE scratch"));
    m.kcache = m.vcache = nullptr;
    m.mem = m.moe_mem = nullptr;
    return rc;
}

// Unregisters the decode models that read MoE layer `key` (it is being
// replaced or unregistered).
int drop_models_using_moe(soso_hip *h, const std::string &key)
{
    int rc = SOSO_HIP_OK;
    for (auto d = h->decode_models.begin(); d != h->decode_models.end();) {
        if (std::find(d->second.moe_uses.begin(), d->second.moe_uses.end(), key) != d->second.moe_uses.end()) {
            rc = first_fail(rc, decode_free(h, d->second));
            d = h->decode_models.erase(d);
        } else {
            ++d;
        }
    }
    return rc;
}

} // namespace

extern "C" {

int soso_hip_create(int device, uint64_t vram_budget, soso_hip **out)
{
    if (!out) return SOSO_HIP_ERR_ARG;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) return SOSO_HIP_ERR_DEVICE;
    if (device < 0 || device >= count) return SOSO_HIP_ERR_ARG;
    soso_hip *h = new (std::nothrow) soso_hip();
    if (!h) return SOSO_HIP_ERR_NOMEM;
    h->device = device;
    hipDeviceProp_t prop;
    if (hipSetDevice(device) != hipSuccess || hipGetDeviceProperties(&prop, device) != hipSuccess ||
        hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreate(&h->ev0) != hipSuccess || hipEventCreate(&h->ev1) != hipSuccess) {
        delete h;
        return SOSO_HIP_ERR_DEVICE;
    }
    if (hipMalloc((void **)&h->ticket, SOSO_TICKET_BYTES) != hipSuccess ||
        hipMemset(h->ticket, 0, SOSO_TICKET_BYTES) != hipSuccess) {
        // a failed create has no handle to report through: teardown results are moot
        (void)hipGetLastError();
        if (h->ticket) (void)hipFree(h->ticket);
        (void)hipStreamDestroy(h->stream);
        delete h;
        return SOSO_HIP_ERR_DEVICE;
    }
    // this GPU's copy of the fixed scratch array (with the device current)
    if (hipGetSymbolAddress(&h->fixed_scratch, HIP_SYMBOL(scratch)) != hipSuccess || !h->fixed_scratch) {
        (void)hipGetLastError();
        (void)hipFree(h->ticket);
        (void)hipStreamDestroy(h->stream);
        delete h;
        return SOSO_HIP_ERR_DEVICE;
    }
    h->num_cu = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    h->max_lds = prop.sharedMemPerBlock > 0 ? prop.sharedMemPerBlock : 65536;
    size_t free_b = 0, total_b = 0;
    if (!vram_budget && hipMemGetInfo(&free_b, &total_b) != hipSuccess) {
        (void)hipGetLastError();
        soso_hip_destroy(h);
        return SOSO_HIP_ERR_DEVICE;
    }
    h->budget = vram_budget ? vram_budget : (uint64_t)(free_b * 0.9);
    *out = h;
    return 0;
}

void soso_hip_destroy(soso_hip *h)
{
    if (!h) return;
    // the handle is gone when this returns, and with it any channel to report
    // a failed release: every result here is deliberately dropped
    (void)hipSetDevice(h->device);
    (void)hipStreamSynchronize(h->stream);
    for (auto &kv : h->weights)
        if (kv.second.dev) (void)hipFree(kv.second.dev);
    for (auto &kv : h->f32_tensors) (void)hipFree(kv.second);
    for (int i = 0; i < soso_hip::N_SCRATCH; i++)
        if (h->scratch[i]) (void)hipFree(h->scratch[i]);
    for (void *p : h->retired) (void)hipFree(p);
    if (h->pinned) (void)hipHostFree(h->pinned);
    for (auto &kv : h->moe_layers) (void)moe_free(h, kv.second);
    for (auto &kv : h->decode_models) (void)decode_free(h, kv.second);
    if (h->ticket) (void)hipFree(h->ticket);
    for (hipEvent_t e : h->events)
        if (e) (void)hipEventDestroy(e);
    for (hipGraphExec_t g : h->graphs)
        if (g) (void)hipGraphExecDestroy(g);
    (void)hipEventDestroy(h->ev0);
    (void)hipEventDestroy(h->ev1);
    (void)hipStreamDestroy(h->stream);
    (void)hipGetLastError();
    delete h;
}

int soso_hip_available(const soso_hip *h) { return h ? 1 : 0; }

int soso_hip_dtype_supported(const soso_hip *h, uint8_t dtype) { return h && dtype_ok(dtype) ? 1 : 0; }

void soso_hip_stats(const soso_hip *h, soso_hip_stats_t *out)
{
    if (h && out) *out = h->stats;
}

const char *soso_hip_last_error(const soso_hip *h) { return h ? h->err.c_str() : "null handle"; }

int soso_hip_matmul(soso_hip *h, const char *key, size_t key_len, const uint8_t *w, size_t w_len, uint8_t dtype,
                    size_t rows, size_t cols, size_t n, const float *x, float *y)
{
    if (!h) return SOSO_HIP_ERR_ARG;
    if (!key || !x || !y || rows == 0 || cols == 0 || n == 0) return set_err(h, SOSO_HIP_ERR_ARG, "matmul: args");
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    CallClock clk(h);
    Weight *wt = nullptr;
    rc = get_weight(h, key, key_len, w, w_len, dtype, rows, cols, &wt);
    if (rc != SOSO_HIP_OK) return rc;
    float *xd = (float *)scratch_get(h, 0, n * cols * 4);
    // x and y pass through the pinned staging buffer (the caller's buffers are
    // pageable: copies from and to them are staged by the runtime, slowly)
    float *hx = (float *)pinned_get(h, (n * cols + n * rows) * 4);
    if (!xd || !hx) return set_err(h, SOSO_HIP_ERR_NOMEM, "matmul: scratch");
    float *hy = hx + n * cols;
    memcpy(hx, x, n * cols * 4);
    rc = hip_check(h, hipMemcpyAsync(xd, hx, n * cols * 4, hipMemcpyHostToDevice, h->stream), "x upload");
    // the kernel writes y straight into the pinned buffer (host memory the
    // device addresses), so no download follows it.  Measured on MI355X
    // (median per call, host wall clock): Q8_0 4096 x 4096 38.5 us from and to
    // the caller's pageable buffers, 22.7 with a pinned upload and download,
    // 21.5 with y written by the kernel; Q4_K 14336 x 4096 34.6 / 34.0 / 26.2.
    // (x read from the pinned buffer by a copy kernel instead of the upload:
    // the same.)
    float *hyd = nullptr;
    if (rc == SOSO_HIP_OK) rc = hip_check(h, hipHostGetDevicePointer((void **)&hyd, hy, 0), "pinned y address");
    if (rc == SOSO_HIP_OK) rc = launch_matvec(h, *wt, xd, hyd, n);
    if (rc != SOSO_HIP_OK) {
        (void)hip_release(h, hipStreamSynchronize(h->stream), "matmul drain");
        return rc;
    }
    rc = hip_check(h, hipStreamSynchronize(h->stream), "matmul sync");
    if (rc != SOSO_HIP_OK) return rc;
    memcpy(y, hy, n * rows * 4);
    h->stats.bytes_up += n * cols * 4;
    h->stats.bytes_down += n * rows * 4;
    clk.done();
    return SOSO_HIP_OK;
}

int soso_hip_matvec(soso_hip *h, const char *key, size_t key_len, const uint8_t *w, size_t w_len, uint8_t dtype,
                    size_t rows, size_t cols, const float *x, float *y)
{
    return soso_hip_matmul(h, key, key_len, w, w_len, dtype, rows, cols, 1, x, y);
}

int soso_hip_matvec_batch(soso_hip *h, const soso_hip_op *ops, size_t n_ops, uint8_t *done)
{
    if (!h) return SOSO_HIP_ERR_ARG;
    if ((!ops || !done) && n_ops) return set_err(h, SOSO_HIP_ERR_ARG, "matvec_batch: args");
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    CallClock clk(h);
    size_t xs = 0, ys = 0;
    for (size_t i = 0; i < n_ops; i++) {
        done[i] = 0;
        xs += ops[i].cols;
        ys += ops[i].rows;
    }
    if (n_ops == 0) return SOSO_HIP_OK;
    // every x and every y pass through one pinned staging buffer: one upload,
    // the launches (writing y into it), one wait (Lote's single synchronisation)
    float *xd = (float *)scratch_get(h, 0, xs * 4);
    float *hx = (float *)pinned_get(h, (xs + ys) * 4);
    if (!xd || !hx) return set_err(h, SOSO_HIP_ERR_NOMEM, "matvec_batch: staging");
    float *hy = hx + xs;
    size_t xo = 0;
    for (size_t i = 0; i < n_ops; i++) {
        if (ops[i].x) memcpy(hx + xo, ops[i].x, ops[i].cols * 4);
        xo += ops[i].cols;
    }
    rc = hip_check(h, hipMemcpyAsync(xd, hx, xs * 4, hipMemcpyHostToDevice, h->stream), "x upload");
    // the kernels write y straight into the pinned buffer (as soso_hip_matmul)
    float *hyd = nullptr;
    if (rc == SOSO_HIP_OK) rc = hip_check(h, hipHostGetDevicePointer((void **)&hyd, hy, 0), "pinned y address");
    if (rc != SOSO_HIP_OK) return rc;
    std::vector<uint8_t> launched(n_ops, 0);
    size_t yo = 0;
    int worst = SOSO_HIP_OK;
    xo = 0;
    for (size_t i = 0; i < n_ops; i++) {
        const soso_hip_op &op = ops[i];
        Weight *wt = nullptr;
        int r = (op.key && op.x && op.y && op.rows && op.cols)
                    ? get_weight(h, op.key, op.key_len, op.w, op.w_len, op.dtype, op.rows, op.cols, &wt)
                    : SOSO_HIP_DECLINED;
        if (r == SOSO_HIP_OK) r = launch_matvec(h, *wt, xd + xo, hyd + yo, 1);
        if (r == SOSO_HIP_OK) launched[i] = 1;
        else if (r < worst) worst = r;
        else if (r == SOSO_HIP_DECLINED && worst == SOSO_HIP_OK) worst = SOSO_HIP_DECLINED;
        xo += op.cols;
        yo += op.rows;
    }
    rc = hip_check(h, hipStreamSynchronize(h->stream), "matvec_batch sync");
    if (rc != SOSO_HIP_OK) {
        (void)hip_release(h, hipStreamSynchronize(h->stream), "matvec_batch drain");
        return rc;
    }
    yo = 0;
    for (size_t i = 0; i < n_ops; i++) {
        if (launched[i]) {
            memcpy(ops[i].y, hy + yo, ops[i].rows * 4);
            done[i] = 1;
            h->stats.bytes_up += ops[i].cols * 4;
            h->stats.bytes_down += ops[i].rows * 4;
        }
        yo += ops[i].rows;
    }
    clk.done();
    return worst;
}

// ---------------------------------------------------------------------------
// Gated DeltaNet block (GpuDispatch::gdn_bloque, gpu.rs:577-599)
// ---------------------------------------------------------------------------
static int gdn_args_ok(soso_hip *h, const void *hist, const void *conv, const void *z, const void *decay,
                       const void *beta, const void *norm, const void *state, const void *out, size_t n, size_t n_k,
                       size_t n_v, size_t d, size_t kernel)
{
    if (!hist || !conv || !z || !decay || !beta || !norm || !state || !out)
        return set_err(h, SOSO_HIP_ERR_ARG, "gdn_block: null buffer");
    if (const char *why = gdn_unsupported(n, n_k, n_v, d, kernel)) return set_err(h, SOSO_HIP_DECLINED, why);
    return SOSO_HIP_OK;
}

int soso_hip_gdn_block(soso_hip *h, const float *hist, const float *conv, const float *z, const float *decay,
                       const float *beta, const float *norm, float *state, float *out, size_t n, size_t n_k,
                       size_t n_v, size_t d, size_t kernel, float eps)
{
    if (!h) return SOSO_HIP_ERR_ARG;
    int rc = gdn_args_ok(h, hist, conv, z, decay, beta, norm, state, out, n, n_k, n_v, d, kernel);
    if (rc != SOSO_HIP_OK) return rc;
    rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    CallClock clk(h);
    const size_t C = (2 * n_k + n_v) * d, vd = n_v * d;
    // one device buffer, 256-byte aligned pieces: the inputs, the state, the
    // output and the conv/normalisation result u
    const size_t sz[] = {(kernel - 1 + n) * C, C * kernel, n * vd, n * n_v, n * n_v, d, n_v * d * d, n * vd, n * C};
    size_t off[9], total = 0;
    for (int i = 0; i < 9; i++) {
        off[i] = total;
        total += (sz[i] * 4 + 255) & ~(size_t)255;
    }
    char *dev = (char *)scratch_get(h, 7, total);
    if (!dev) return set_err(h, SOSO_HIP_ERR_NOMEM, "gdn_block: scratch");
    float *p[9];
    for (int i = 0; i < 9; i++) p[i] = (float *)(dev + off[i]);
    const float *src[7] = {hist, conv, z, decay, beta, norm, state};
    for (int i = 0; i < 7 && rc == SOSO_HIP_OK; i++)
        rc = hip_check(h, hipMemcpyAsync(p[i], src[i], sz[i] * 4, hipMemcpyHostToDevice, h->stream), "gdn upload");
    if (rc == SOSO_HIP_OK)
        rc = launch_gdn_block(h, p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7], p[8], (int)n, (int)n_k, (int)n_v,
                              (int)kernel, eps);
    if (rc == SOSO_HIP_OK)
        rc = hip_check(h, hipMemcpyAsync(out, p[7], sz[7] * 4, hipMemcpyDeviceToHost, h->stream), "gdn out");
    if (rc == SOSO_HIP_OK)
        rc = hip_check(h, hipMemcpyAsync(state, p[6], sz[6] * 4, hipMemcpyDeviceToHost, h->stream), "gdn state");
    if (rc == SOSO_HIP_OK) rc = hip_check(h, hipStreamSynchronize(h->stream), "gdn sync");
    if (rc != SOSO_HIP_OK) {
        (void)hip_release(h, hipStreamSynchronize(h->stream), "gdn drain");
        return rc;
    }
    for (int i = 0; i < 7; i++) h->stats.bytes_up += sz[i] * 4;
    h->stats.bytes_down += (sz[6] + sz[7]) * 4;
    clk.done();
    return SOSO_HIP_OK;
}

int soso_hip_gdn_block_dev(soso_hip *h, const float *hist, const float *conv, const float *z, const float *decay,
                           const float *beta, const float *norm, float *state, float *out, size_t n, size_t n_k,
                           size_t n_v, size_t d, size_t kernel, float eps)
{
    if (!h) return SOSO_HIP_ERR_ARG;
    int rc = gdn_args_ok(h, hist, conv, z, decay, beta, norm, state, out, n, n_k, n_v, d, kernel);
    if (rc != SOSO_HIP_OK) return rc;
    rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    float *u = (float *)scratch_get(h, 4, n * (2 * n_k + n_v) * d * 4);
    if (!u) return set_err(h, SOSO_HIP_ERR_NOMEM, "gdn_block_dev: scratch (or growing it during capture)");
    return launch_gdn_block(h, hist, conv, z, decay, beta, norm, state, out, u, (int)n, (int)n_k, (int)n_v,
                            (int)kernel, eps);
}

int soso_hip_router_topk(soso_hip *h, const char *key, size_t key_len, const float *w, const float *xs, size_t n,
                         size_t hdim, size_t n_exp, size_t top_k, int32_t *idx, float *wgt)
{
    if (!h) return SOSO_HIP_ERR_ARG;
    // cuda.rs:1668-1670: shapes it cannot do are declined, not errors
    if (!key || !xs || !idx || !wgt || n == 0 || hdim == 0 || hdim % 4 || n_exp == 0 || n_exp > 256 || top_k == 0 ||
        top_k > n_exp || top_k > 64)
        return set_err(h, SOSO_HIP_DECLINED, "router_topk: shape not handled here");
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    CallClock clk(h);
    std::string k(key, key_len);
    void *wd = nullptr;
    auto it = h->f32_tensors.find(k);
    if (it != h->f32_tensors.end()) {
        wd = it->second;
    } else {
        if (!w) return set_err(h, SOSO_HIP_DECLINED, "router_topk: weights not resident and not given");
        if (hipMalloc(&wd, n_exp * hdim * 4) != hipSuccess) return set_err(h, SOSO_HIP_DECLINED, "router: alloc");
        rc = hip_check(h, hipMemcpy(wd, w, n_exp * hdim * 4, hipMemcpyHostToDevice), "router upload");
        if (rc != SOSO_HIP_OK) {
            (void)hip_release(h, hipFree(wd), "free router weights");
            return rc;
        }
        h->f32_tensors[k] = wd;
    }
    // blocks of at most moe_block_tokens(top_k) tokens per route launch, each
    // block's routing copied out before the next overwrites the scratch
    const size_t nb = std::min(n, moe_block_tokens(top_k));
    float *xd = (float *)scratch_get(h, 0, n * hdim * 4);
    // x, idx and wgt pass through the pinned staging buffer (the caller's
    // buffers are pageable: the runtime's own staging of each copy is slow)
    float *hx = (float *)pinned_get(h, (n * hdim + 2 * n * top_k) * 4);
    MoeScratch ms;
    if (!xd || !hx || !moe_scratch(h, nb, n_exp, top_k, 0, 0, ms))
        return set_err(h, SOSO_HIP_ERR_NOMEM, "router: scratch");
    int32_t *hidx = (int32_t *)(hx + n * hdim);
    float *hwgt = (float *)(hidx + n * top_k);
    memcpy(hx, xs, n * hdim * 4);
    rc = hip_check(h, hipMemcpyAsync(xd, hx, n * hdim * 4, hipMemcpyHostToDevice, h->stream), "x upload");
    for (size_t t0 = 0; t0 < n && rc == SOSO_HIP_OK; t0 += nb) {
        const size_t m = std::min(nb, n - t0);
        rc = launch_moe_route(h, (const float *)wd, xd + t0 * hdim, m, hdim, n_exp, top_k, ms);
        if (rc == SOSO_HIP_OK)
            rc = hip_check(h, hipMemcpyAsync(hidx + t0 * top_k, ms.idx, m * top_k * 4, hipMemcpyDeviceToHost, h->stream),
                           "idx");
        if (rc == SOSO_HIP_OK)
            rc = hip_check(h, hipMemcpyAsync(hwgt + t0 * top_k, ms.wgt, m * top_k * 4, hipMemcpyDeviceToHost, h->stream),
                           "wgt");
    }
    if (rc == SOSO_HIP_OK) rc = hip_check(h, hipStreamSynchronize(h->stream), "router sync");
    if (rc != SOSO_HIP_OK) {
        (void)hip_release(h, hipStreamSynchronize(h->stream), "router drain");
        return rc;
    }
    memcpy(idx, hidx, n * top_k * 4);
    memcpy(wgt, hwgt, n * top_k * 4);
    h->stats.bytes_up += n * hdim * 4;
    h->stats.bytes_down += n * top_k * 8;
    clk.done();
    return SOSO_HIP_OK;
}

int soso_hip_experts_block(soso_hip *h, const float *xs, size_t n, size_t hdim, size_t ffn, size_t top_k,
                           const float *wgt, const soso_hip_expert *exps, size_t n_exps, float *sum, uint8_t *done)
{
    if (!h) return SOSO_HIP_ERR_ARG;
    if (!xs || !wgt || !sum || !done || (!exps && n_exps) || n == 0 || hdim == 0 || ffn == 0 || top_k == 0)
        return set_err(h, SOSO_HIP_ERR_ARG, "experts_block: args");
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    CallClock clk(h);
    const bool pending = h->shared_pending;
    h->shared_pending = false;
    if (pending && (h->shared_n != n || h->shared_hdim != hdim))
        return set_err(h, SOSO_HIP_ERR_ARG, "experts_block: the pending shared expert was computed for another block");
    const size_t dims[3][2] = {{ffn, hdim}, {ffn, hdim}, {hdim, ffn}};
    const size_t slots = n * top_k;
    // Resolvable experts: the three matrices resident (or uploadable), one
    // dtype for all gate/up and one for all down (the first resolvable expert
    // fixes them), valid token/slot indices.  Shared experts are left to the
    // caller (they are summed through moe_compartido in the reference).
    std::vector<const Weight *> wts(n_exps * 3, nullptr);
    std::vector<uint8_t> ok(n_exps, 0), use(slots, 0);
    uint8_t dt_gu = 0, dt_dn = 0;
    bool all = true;
    for (size_t e = 0; e < n_exps; e++) {
        done[e] = 0;
        const soso_hip_expert &x = exps[e];
        bool good = x.n_tokens > 0 && !x.shared && x.tokens && x.targets;
        for (int k = 0; k < 3 && good; k++) {
            Weight *wt = nullptr;
            if (!x.keys[k]) {
                good = false;
                break;
            }
            int r = get_weight(h, x.keys[k], x.key_lens[k], x.w[k], x.w_len[k], x.dtype[k], dims[k][0], dims[k][1], &wt);
            if (r < 0) return r;
            if (r != SOSO_HIP_OK || wt->dtype == SOSO_HIP_DTYPE_F32 || weight_kcols(*wt) != wt->cols) good = false;
            else wts[3 * e + k] = wt;
        }
        if (good) {
            if (!dt_gu) {
                dt_gu = wts[3 * e]->dtype;
                dt_dn = wts[3 * e + 2]->dtype;
            }
            good = wts[3 * e]->dtype == dt_gu && wts[3 * e + 1]->dtype == dt_gu && wts[3 * e + 2]->dtype == dt_dn;
        }
        for (size_t t = 0; good && t < x.n_tokens; t++)
            if (x.tokens[t] >= n || x.targets[t] >= slots || x.targets[t] / top_k != x.tokens[t]) good = false;
        ok[e] = good ? 1 : 0;
        if (!good && x.n_tokens > 0) all = false;
    }
    // groups = resolvable experts; their slots sorted by group
    std::vector<size_t> gid;
    for (size_t e = 0; e < n_exps; e++)
        if (ok[e]) gid.push_back(e);
    const size_t G = gid.size();
    // [cnt G | offs G+1 | list slots | active groups G | their count], as moe_scratch lays it out
    // [cnt G | offs G + 1 | list slots | work items 4 x max_items | item count | records 4G | record count]
    const size_t max_items = moe_max_items(h, slots, G ? G : 1);
    std::vector<int> ints(2 * G + 2 + slots + 4 * max_items + 4 * G + 1, 0);
    std::vector<const uint8_t *> tab(3 * G);
    int o = 0;
    for (size_t g = 0; g < G; g++) {
        const soso_hip_expert &x = exps[gid[g]];
        ints[g] = (int)x.n_tokens;
        ints[G + g] = o;
        for (size_t t = 0; t < x.n_tokens; t++) {
            ints[2 * G + 1 + o++] = (int)x.targets[t];
            use[x.targets[t]] = 1;
        }
        for (int k = 0; k < 3; k++) tab[k * G + g] = (const uint8_t *)wts[3 * gid[g] + k]->dev;
    }
    ints[2 * G] = o;
    // work items as k_moe_route writes them: group g with c slots gets
    // max(1, round(c * target / slots)) row chunks
    {
        const int target = moe_item_target(h);
        size_t ni = 0;
        for (size_t g = 0; g < G; g++) {
            const int c = ints[g];
            const int nx = c > 0 ? std::min(0xFFFF, std::max(1, (int)((c * (long)target + (long)slots / 2) / (long)slots))) : 0;
            for (int j = 0; j < nx && ni < max_items; j++, ni++) {
                int *r = &ints[2 * G + 1 + slots + 4 * ni];
                r[0] = (int)g;
                r[1] = c;
                r[2] = ints[G + g];
                r[3] = j | (nx << 16);
            }
        }
        ints[2 * G + 1 + slots + 4 * max_items] = (int)ni;
        int *rec = &ints[2 * G + 2 + slots + 4 * max_items];
        for (size_t g = 0; g < G; g++) {
            rec[4 * g] = (int)g;
            rec[4 * g + 1] = ints[g];
            rec[4 * g + 2] = ints[G + g];
        }
        rec[4 * G] = (int)G;
    }
    float *xd = (float *)scratch_get(h, 0, n * hdim * 4);
    float *sd = (float *)scratch_get(h, 5, n * hdim * 4);
    // the weights, tables and slot marks sit together in aux (one upload)
    const size_t tab_off = (slots * 4 + 15) & ~(size_t)15, aux_bytes = tab_off + 3 * G * sizeof(void *) + slots;
    char *aux = (char *)scratch_get(h, 11, aux_bytes + 64);
    // every host-side buffer passes through the pinned staging buffer: x, the
    // groups, aux's image, then the sum on its way back
    const size_t x_b = (n * hdim * 4 + 15) & ~(size_t)15, ints_b = (ints.size() * 4 + 15) & ~(size_t)15,
                 aux_b = (aux_bytes + 15) & ~(size_t)15;
    char *hs = (char *)pinned_get(h, x_b + ints_b + aux_b + n * hdim * 4);
    MoeScratch ms;
    if (!xd || !sd || !aux || !hs || !moe_scratch(h, n, G, top_k, hdim, ffn, ms))
        return set_err(h, SOSO_HIP_ERR_NOMEM, "experts_block: scratch");
    float *wd = (float *)aux;
    const uint8_t **tabd = (const uint8_t **)(aux + tab_off);
    uint8_t *used = (uint8_t *)(tabd + 3 * G);
    char *hints = hs + x_b, *haux = hints + ints_b;
    float *hsum = (float *)(haux + aux_b);
    memcpy(hs, xs, n * hdim * 4);
    if (G) memcpy(hints, ints.data(), ints.size() * 4);
    memcpy(haux, wgt, slots * 4);
    if (G) memcpy(haux + tab_off, tab.data(), tab.size() * sizeof(void *));
    memcpy(haux + tab_off + 3 * G * sizeof(void *), use.data(), slots);
    rc = hip_check(h, hipMemcpyAsync(xd, hs, n * hdim * 4, hipMemcpyHostToDevice, h->stream), "x upload");
    if (rc == SOSO_HIP_OK && G)
        rc = hip_check(h, hipMemcpyAsync(ms.cnt, hints, ints.size() * 4, hipMemcpyHostToDevice, h->stream),
                       "groups upload");
    if (rc == SOSO_HIP_OK)
        rc = hip_check(h, hipMemcpyAsync(aux, haux, aux_bytes, hipMemcpyHostToDevice, h->stream), "aux upload");
    if (rc == SOSO_HIP_OK) {
        if (G)
            rc = launch_moe_experts(h, xd, n, hdim, ffn, top_k, dt_gu, dt_dn, tabd, G, wd, used, nullptr, ms, sd);
        else
            rc = hip_check(h, hipMemsetAsync(sd, 0, n * hdim * 4, h->stream), "zero sum");
    }
    // the shared expert of the same block (moe_shared, gpu.rs:518-521) joins
    // the sum after the ranked experts, as soso adds it last (bloque35.rs:1000-1005)
    if (rc == SOSO_HIP_OK && pending) rc = launch_vec_add(h, sd, (const float *)h->scratch[12], n * hdim);
    if (rc == SOSO_HIP_OK) rc = hip_check(h, hipMemcpyAsync(hsum, sd, n * hdim * 4, hipMemcpyDeviceToHost, h->stream), "sum");
    if (rc == SOSO_HIP_OK) rc = hip_check(h, hipStreamSynchronize(h->stream), "experts sync");
    if (rc != SOSO_HIP_OK) {
        (void)hip_release(h, hipStreamSynchronize(h->stream), "experts drain");
        return rc;
    }
    memcpy(sum, hsum, n * hdim * 4);
    for (size_t e = 0; e < n_exps; e++) done[e] = ok[e];
    h->stats.bytes_up += n * hdim * 4 + slots * 4;
    h->stats.bytes_down += n * hdim * 4;
    clk.done();
    return all ? SOSO_HIP_OK : SOSO_HIP_DECLINED;
}

// ---- shared expert of an MoE block (GpuDispatch::moe_compartido) -------------
int soso_hip_moe_shared(soso_hip *h, const char *const *keys, const size_t *key_lens, const uint8_t *const *w,
                        const size_t *w_len, const uint8_t *dtype, const float *pg_w, const float *xs, size_t n,
                        size_t hdim, size_t ffn)
{
    if (!h) return SOSO_HIP_ERR_ARG;
    if (!keys || !key_lens || !w || !w_len || !dtype || !pg_w || !xs || n == 0 || hdim == 0 || ffn == 0)
        return set_err(h, SOSO_HIP_ERR_ARG, "moe_shared: args");
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    CallClock clk(h);
    h->shared_pending = false;
    const size_t dims[3][2] = {{ffn, hdim}, {ffn, hdim}, {hdim, ffn}};
    Weight *wt[3] = {};
    for (int k = 0; k < 3; k++) {
        if (!keys[k]) return set_err(h, SOSO_HIP_ERR_ARG, "moe_shared: key");
        rc = get_weight(h, keys[k], key_lens[k], w[k], w_len[k], dtype[k], dims[k][0], dims[k][1], &wt[k]);
        if (rc != SOSO_HIP_OK) return rc;
        if (wt[k]->dtype == SOSO_HIP_DTYPE_F32) return set_err(h, SOSO_HIP_DECLINED, "moe_shared: f32 expert");
    }
    float *xd = (float *)scratch_get(h, 2, (n * hdim + hdim) * 4);
    float *gu = (float *)scratch_get(h, 3, 2 * n * ffn * 4);
    float *out = (float *)scratch_get(h, 12, n * hdim * 4);
    if (!xd || !gu || !out) return set_err(h, SOSO_HIP_ERR_NOMEM, "moe_shared: scratch");
    float *pgd = xd + n * hdim;
    rc = hip_check(h, hipMemcpyAsync(xd, xs, n * hdim * 4, hipMemcpyHostToDevice, h->stream), "x upload");
    if (rc == SOSO_HIP_OK)
        rc = hip_check(h, hipMemcpyAsync(pgd, pg_w, hdim * 4, hipMemcpyHostToDevice, h->stream), "gate upload");
    // gate, up, SwiGLU, down (each a matmul over the n tokens), then the gate
    if (rc == SOSO_HIP_OK) rc = launch_matvec(h, *wt[0], xd, gu, n);
    if (rc == SOSO_HIP_OK) rc = launch_matvec(h, *wt[1], xd, gu + n * ffn, n);
    if (rc == SOSO_HIP_OK) rc = launch_shared_swiglu(h, gu, gu + n * ffn, n * ffn);
    if (rc == SOSO_HIP_OK) rc = launch_matvec(h, *wt[2], gu + n * ffn, out, n);
    if (rc == SOSO_HIP_OK) rc = launch_shared_gate(h, xd, pgd, out, n, hdim);
    if (rc != SOSO_HIP_OK) return rc;
    h->shared_pending = true;
    h->shared_n = n;
    h->shared_hdim = hdim;
    h->stats.bytes_up += (n * hdim + hdim) * 4;
    clk.done();
    return SOSO_HIP_OK;
}

// ---- MoE FFN resident on the device ----------------------------------------
// want_tiled = false: no tile-major copies (a layer only the single-token
// kernels read, such as soso_hip_moe_capa's).
static int moe_register_impl(soso_hip *h, const char *layer_key, size_t layer_key_len, const char *router_key,
                             size_t router_key_len, const char *const *expert_keys, const size_t *expert_key_lens,
                             size_t n_exp, size_t hdim, size_t ffn, size_t top_k, bool want_tiled)
{
    if (!h) return SOSO_HIP_ERR_ARG;
    if (!layer_key || !router_key || (expert_keys && !expert_key_lens) || n_exp == 0 || n_exp > 256 || top_k == 0 ||
        top_k > n_exp || top_k > 64 || hdim == 0 || hdim % 4 || ffn == 0)
        return set_err(h, SOSO_HIP_ERR_ARG, "moe_register: args");
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    MoeLayer m;
    m.router = find_weight(h, router_key, router_key_len);
    if (!m.router || m.router->dtype != SOSO_HIP_DTYPE_F32 || m.router->rows != n_exp || m.router->cols != hdim)
        return set_err(h, SOSO_HIP_DECLINED, "moe_register: router not resident as f32 [n_exp x hdim]");
    m.n_exp = n_exp;
    m.hdim = hdim;
    m.ffn = ffn;
    m.top_k = top_k;
    if (!expert_keys) { // the router alone: experts stay on the host (decode_token's cpu_moe)
        std::string k(layer_key, layer_key_len);
        auto it = h->moe_layers.find(k);
        if (it != h->moe_layers.end()) {
            rc = first_fail(drop_models_using_moe(h, k), moe_free(h, it->second));
            h->moe_layers.erase(it);
        }
        h->moe_layers.emplace(k, m);
        return rc;
    }
    std::vector<const uint8_t *> tab(3 * n_exp);
    const size_t dims[3][2] = {{ffn, hdim}, {ffn, hdim}, {hdim, ffn}};
    for (size_t e = 0; e < n_exp; e++)
        for (int k = 0; k < 3; k++) {
            const Weight *w = find_weight(h, expert_keys[3 * e + k], expert_key_lens[3 * e + k]);
            if (!w || w->rows != dims[k][0] || w->cols != dims[k][1] || weight_kcols(*w) != w->cols ||
                w->dtype == SOSO_HIP_DTYPE_F32)
                return set_err(h, SOSO_HIP_DECLINED, "moe_register: expert matrix missing or of the wrong shape");
            const uint8_t want = k < 2 ? m.dt_gu : m.dt_down;
            if (want && w->dtype != want) return set_err(h, SOSO_HIP_DECLINED, "moe_register: mixed expert dtypes");
            if (k < 2) m.dt_gu = w->dtype;
            else m.dt_down = w->dtype;
            tab[k * n_exp + e] = (const uint8_t *)w->dev;
        }
    m.host_tab.assign(tab.begin(), tab.end());
    if (hipMalloc((void **)&m.tab, tab.size() * sizeof(void *)) != hipSuccess)
        return set_err(h, SOSO_HIP_ERR_NOMEM, "moe_register: table");
    rc = hip_check(h, hipMemcpy(m.tab, tab.data(), tab.size() * sizeof(void *), hipMemcpyHostToDevice), "table upload");
    // Tile-major copies of the Q4_K experts for the matrix-core path (the
    // row-major ones stay for the single-token kernels); skipped, with the
    // row-major matrix-core path as fallback, when the budget has no room.
    const bool tgu = want_tiled && m.dt_gu == SOSO_HIP_DTYPE_Q4_K && tiled_q4k_ok(m.dt_gu, ffn, hdim);
    const bool tdn = want_tiled && m.dt_down == SOSO_HIP_DTYPE_Q4_K && tiled_q4k_ok(m.dt_down, hdim, ffn);
    const size_t b_gu = ffn * packed_row_stride(SOSO_HIP_DTYPE_Q4_K, hdim);
    const size_t b_dn = hdim * packed_row_stride(SOSO_HIP_DTYPE_Q4_K, ffn);
    const size_t tbytes = n_exp * ((tgu ? 2 * b_gu : 0) + (tdn ? b_dn : 0));
    if (rc == SOSO_HIP_OK && tbytes > 0 && h->used + tbytes <= h->budget &&
        hipMalloc(&m.tiled_mem, tbytes) == hipSuccess) {
        h->used += tbytes;
        m.tiled_bytes = tbytes;
        std::vector<const uint8_t *> tt(3 * n_exp, nullptr);
        uint8_t *p = (uint8_t *)m.tiled_mem;
        for (size_t e = 0; e < n_exp && rc == SOSO_HIP_OK; e++)
            for (int k = 0; k < 3 && rc == SOSO_HIP_OK; k++) {
                if (k < 2 ? !tgu : !tdn) continue;
                rc = launch_tile_q4k(h, tab[k * n_exp + e], p, dims[k][0], dims[k][1]);
                tt[k * n_exp + e] = p;
                p += k < 2 ? b_gu : b_dn;
            }
        if (rc == SOSO_HIP_OK && hipMalloc((void **)&m.tiled, tt.size() * sizeof(void *)) != hipSuccess)
            rc = set_err(h, SOSO_HIP_ERR_NOMEM, "moe_register: tiled table");
        if (rc == SOSO_HIP_OK)
            rc = hip_check(h, hipMemcpyAsync(m.tiled, tt.data(), tt.size() * sizeof(void *), hipMemcpyHostToDevice,
                                             h->stream), "tiled table upload");
        if (rc == SOSO_HIP_OK) rc = hip_check(h, hipStreamSynchronize(h->stream), "tiled copies");
        m.tiled_gu = tgu;
        m.tiled_down = tdn;
    }
    if (rc != SOSO_HIP_OK) {
        (void)moe_free(h, m);
        return rc;
    }
    std::string k(layer_key, layer_key_len);
    auto it = h->moe_layers.find(k);
    if (it != h->moe_layers.end()) {
        rc = first_fail(drop_models_using_moe(h, k), moe_free(h, it->second));
        h->moe_layers.erase(it);
    }
    h->moe_layers.emplace(k, m);
    return rc;
}

int soso_hip_moe_register(soso_hip *h, const char *layer_key, size_t layer_key_len, const char *router_key,
                          size_t router_key_len, const char *const *expert_keys, const size_t *expert_key_lens,
                          size_t n_exp, size_t hdim, size_t ffn, size_t top_k)
{
    return moe_register_impl(h, layer_key, layer_key_len, router_key, router_key_len, expert_keys, expert_key_lens,
                             n_exp, hdim, ffn, top_k, true);
}

// A registered layer over n tokens with its scratch in ms (sized for
// min(n, moe_block_tokens(top_k)) tokens): one token takes the single-token
// path; more run route + experts in blocks of moe_block_tokens(top_k).
static int moe_ffn_run(soso_hip *h, const MoeLayer &m, const float *x_dev, size_t n, float *out_dev, int32_t *idx_dev,
                       float *wgt_dev, const MoeScratch &ms)
{
    if (n == 1) {
        MoeScratch s = ms;
        if (idx_dev) s.idx = idx_dev;
        if (wgt_dev) s.wgt = wgt_dev;
        const int rc = launch_moe_ffn1(h, m, x_dev, s, out_dev);
        if (rc != SOSO_HIP_DECLINED) return rc;
    }
    const size_t nb = moe_block_tokens(m.top_k);
    int rc = SOSO_HIP_OK;
    for (size_t t0 = 0; t0 < n && rc == SOSO_HIP_OK; t0 += nb) {
        const size_t c = std::min(nb, n - t0);
        MoeScratch s = ms;
        if (idx_dev) s.idx = idx_dev + t0 * m.top_k;
        if (wgt_dev) s.wgt = wgt_dev + t0 * m.top_k;
        const float *xc = x_dev + t0 * m.hdim;
        // experts that scan the ranking themselves spare the route its slot sort
        const bool scan = mfma_moe_scan_ok(c, m.top_k, m.n_exp, m.dt_gu, m.dt_down, m.hdim, m.ffn);
        rc = launch_moe_route(h, (const float *)m.router->dev, xc, c, m.hdim, m.n_exp, m.top_k, s, !scan);
        if (rc == SOSO_HIP_OK)
            rc = launch_moe_experts(h, xc, c, m.hdim, m.ffn, m.top_k, m.dt_gu, m.dt_down, m.tab, m.n_exp, s.wgt,
                                    nullptr, s.idx, s, out_dev + t0 * m.hdim, &m, scan);
    }
    return rc;
}

int soso_hip_moe_ffn_dev(soso_hip *h, const char *layer_key, size_t layer_key_len, const float *x_dev, size_t n,
                         float *out_dev, int32_t *idx_dev, float *wgt_dev)
{
    if (!h) return SOSO_HIP_ERR_ARG;
    if (!layer_key || !x_dev || !out_dev || n == 0) return set_err(h, SOSO_HIP_ERR_ARG, "moe_ffn_dev: args");
    auto it = h->moe_layers.find(std::string(layer_key, layer_key_len));
    if (it == h->moe_layers.end()) return set_err(h, SOSO_HIP_DECLINED, "moe_ffn_dev: layer not registered");
    const MoeLayer &m = it->second;
    if (!m.tab) return set_err(h, SOSO_HIP_DECLINED, "moe_ffn_dev: the layer's experts stay on the host");
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    MoeScratch ms;
    if (!moe_scratch(h, std::min(n, moe_block_tokens(m.top_k)), m.n_exp, m.top_k, m.hdim, m.ffn, ms))
        return h->capturing ? set_err(h, SOSO_HIP_DECLINED,
                                      "moe_ffn_dev: its scratch would have to grow inside graph capture (make one call "
                                      "with this token count outside capture first)")
                            : set_err(h, SOSO_HIP_ERR_NOMEM, "moe_ffn_dev: scratch");
    return moe_ffn_run(h, m, x_dev, n, out_dev, idx_dev, wgt_dev, ms);
}

// The allocation-free form of soso_hip_moe_ffn_dev: the same kernels, with
// the scratch carved out of this GPU's fixed array.
int soso_hip_moe_ffn_dev_noalloc(soso_hip *h, const char *layer_key, size_t layer_key_len, const float *x_dev, size_t n,
                                 float *out_dev, int32_t *idx_dev, float *wgt_dev)
{
    if (!h) return SOSO_HIP_ERR_ARG;
    if (!layer_key || !x_dev || !out_dev || n == 0) return set_err(h, SOSO_HIP_ERR_ARG, "moe_ffn_dev_noalloc: args");
    auto it = h->moe_layers.find(std::string(layer_key, layer_key_len));
    if (it == h->moe_layers.end()) return set_err(h, SOSO_HIP_DECLINED, "moe_ffn_dev_noalloc: layer not registered");
    const MoeLayer &m = it->second;
    if (!m.tab) return set_err(h, SOSO_HIP_DECLINED, "moe_ffn_dev_noalloc: the layer's experts stay on the host");
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    MoeScratch ms;
    const size_t need = moe_scratch_fixed(h, std::min(n, moe_block_tokens(m.top_k)), m.n_exp, m.top_k, m.hdim, m.ffn,
                                          h->fixed_scratch, SOSO_HIP_MOE_NOALLOC_SCRATCH_BYTES, ms);
    if (need > SOSO_HIP_MOE_NOALLOC_SCRATCH_BYTES)
        return set_err(h, SOSO_HIP_ERR_ARG, "moe_ffn_dev_noalloc: " + std::to_string(n) + " tokens need " +
                                                std::to_string(need) + " bytes of scratch; the fixed array holds " +
                                                std::to_string((size_t)SOSO_HIP_MOE_NOALLOC_SCRATCH_BYTES));
    return moe_ffn_run(h, m, x_dev, n, out_dev, idx_dev, wgt_dev, ms);
}

// ---- dense decode step -------------------------------------------------------
// decode_create / decode_create_moe: moe_keys (n_layers entries, null for a
// dense model) names the registered MoE layer that is layer l's FFN, or null
// for a dense FFN.
// layers_only: a stack of layers without the output norm and head (the keys
// end with the last layer's; cfg->vocab is ignored): soso_hip_moe_capa's
// per-layer steps, hidden state in and out.
static int decode_create_impl(soso_hip *h, const char *model_key, size_t model_key_len, const soso_hip_decode_cfg *cfg,
                              uint32_t flags, const char *const *keys, const size_t *key_lens,
                              const char *const *moe_keys, const size_t *moe_key_lens, int drop_sources,
                              bool layers_only = false)
{
    if (!h) return SOSO_HIP_ERR_ARG;
    if (!model_key || !cfg || !keys || !key_lens || cfg->n_layers == 0 || cfg->hidden == 0 || cfg->hidden % 4 ||
        cfg->n_kv_heads == 0 || cfg->n_heads % cfg->n_kv_heads || cfg->head_dim == 0 || cfg->ffn == 0 ||
        (cfg->vocab == 0 && !layers_only) || cfg->ctx_max == 0)
        return set_err(h, SOSO_HIP_ERR_ARG, "decode_create: config");
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    const size_t L = cfg->n_layers, H = cfg->hidden, qd = (size_t)cfg->n_heads * cfg->head_dim,
                 kvd = (size_t)cfg->n_kv_heads * cfg->head_dim, F = cfg->ffn;
    if (cfg->head_dim != 128) return set_err(h, SOSO_HIP_DECLINED, "decode_create: head_dim must be 128");
    {
        const uint32_t G = cfg->n_heads / cfg->n_kv_heads;
        if (G != 1 && G != 2 && G != 4 && G != 8)
            return set_err(h, SOSO_HIP_DECLINED, "decode_create: query heads per KV head must be 1, 2, 4 or 8");
    }
    DecodeModel m;
    m.n_layers = L;
    m.hidden = H;
    m.n_heads = cfg->n_heads;
    m.n_kv_heads = cfg->n_kv_heads;
    m.head_dim = cfg->head_dim;
    m.ffn = F;
    m.vocab = layers_only ? 0 : cfg->vocab;
    m.ctx_max = cfg->ctx_max;
    m.theta = cfg->rope_theta;
    m.eps = cfg->rms_eps;
    m.kv_f16 = cfg->kv_f16 != 0;
    if (flags & ~(SOSO_HIP_DECODE_QK_NORM | SOSO_HIP_DECODE_ROPE_NEOX))
        return set_err(h, SOSO_HIP_ERR_ARG, "decode_create: unknown flags");
    m.qk_norm = (flags & SOSO_HIP_DECODE_QK_NORM) != 0;
    m.rope_neox = (flags & SOSO_HIP_DECODE_ROPE_NEOX) != 0;
    const size_t kpl = m.qk_norm ? 11 : 9;      // keys per layer
    auto get = [&](size_t i, size_t rows, size_t cols, bool f32, const Weight **out) -> bool {
        const Weight *w = find_weight(h, keys[i], key_lens[i]);
        // (a padded Q8_0 copy is for launch_matvec's callers only)
        if (!w || w->rows != rows || w->cols != cols || weight_kcols(*w) != cols ||
            (f32 != (w->dtype == SOSO_HIP_DTYPE_F32)))
            return false;
        *out = w;
        return true;
    };
    std::vector<const Weight *> q(L), k(L), v(L), g(L), u(L);
    m.layers.resize(L);
    size_t moe_need = 0, n_moe = 0; // MoE scratch bytes (the largest layer's) and layers
    for (size_t l = 0; l < L; l++) {
        const Weight *an, *fn, *qn = nullptr, *kn = nullptr;
        const size_t b = kpl * l;
        const bool is_moe = moe_keys && moe_keys[l];
        if (is_moe) {
            const std::string mk(moe_keys[l], moe_key_lens[l]);
            auto mit = h->moe_layers.find(mk);
            if (mit == h->moe_layers.end())
                return set_err(h, SOSO_HIP_DECLINED, "decode_create: layer " + std::to_string(l) + ": MoE layer " +
                                                         mk + " is not registered");
            const MoeLayer &ml = mit->second;
            if (ml.hdim != H)
                return set_err(h, SOSO_HIP_DECLINED, "decode_create: layer " + std::to_string(l) +
                                                         ": the MoE layer's width is not hidden");
            // a layer registered without experts runs them on the host (decode_token's cpu_moe)
            if (!ml.tab) m.n_host_moe++;
            else if (const char *why = moe_ffn1_unsupported(h, ml))
                return set_err(h, SOSO_HIP_DECLINED, "decode_create: layer " + std::to_string(l) + " MoE: " + why);
            if (H > 8192) return set_err(h, SOSO_HIP_DECLINED, "decode_create: MoE layers take hidden <= 8192");
            m.layers[l].moe = &ml;
            MoeScratch probe;
            moe_need = std::max(moe_need, moe_scratch_fixed(h, 1, ml.n_exp, ml.top_k, ml.hdim, ml.ffn, nullptr, 0,
                                                            probe));
            n_moe++;
            m.moe_uses.push_back(mk);
        }
        if (!get(b, 1, H, true, &an) || !get(b + 1, qd, H, false, &q[l]) || !get(b + 2, kvd, H, false, &k[l]) ||
            !get(b + 3, kvd, H, false, &v[l]) || !get(b + 4, H, qd, false, &m.layers[l].o) ||
            !get(b + 5, 1, H, true, &fn) ||
            (!is_moe && (!get(b + 6, F, H, false, &g[l]) || !get(b + 7, F, H, false, &u[l]) ||
                         !get(b + 8, H, F, false, &m.layers[l].down))))
            return set_err(h, SOSO_HIP_DECLINED, "decode_create: layer " + std::to_string(l) +
                                                     ": a weight is missing or has the wrong shape");
        if (m.qk_norm && (!get(b + 9, 1, cfg->head_dim, true, &qn) || !get(b + 10, 1, cfg->head_dim, true, &kn)))
            return set_err(h, SOSO_HIP_DECLINED, "decode_create: layer " + std::to_string(l) +
                                                     ": q_norm / k_norm missing or not F32 [head_dim]");
        if (q[l]->dtype != k[l]->dtype || q[l]->dtype != v[l]->dtype || (!is_moe && g[l]->dtype != u[l]->dtype))
            return set_err(h, SOSO_HIP_DECLINED, "decode_create: q/k/v or gate/up dtypes differ");
        // every launch of the step, checked here so that a step never declines
        // halfway through a token
        const struct {
            const Weight *w;
            size_t rows, cols;
            int xs, epi;
            const char *role;
        } roles[] = {{q[l], qd + 2 * kvd, H, XS_RMSNORM, EPI_STORE, "q/k/v"},
                     {m.layers[l].o, H, qd, XS_PLAIN, EPI_RESID, "o"},
                     {g[l], 2 * F, H, XS_RMSNORM, EPI_SWIGLU, "gate/up"},
                     {m.layers[l].down, H, F, XS_PLAIN, EPI_RESID, "down"}};
        for (const auto &r : roles)
            if (r.w && (!is_moe || r.w == q[l] || r.w == m.layers[l].o)) {
                const char *why = matvec_ex_unsupported(h, r.w->dtype, r.rows, r.cols, r.xs, r.epi);
                // a down projection the split-row form does not take may still
                // run as column segments (whose consumer is checked below)
                if (why && r.w == m.layers[l].down &&
                    !matvec_ex_unsupported(h, r.w->dtype, r.rows, r.cols, XS_PLAIN, EPI_PARTS))
                    why = nullptr;
                if (why)
                    return set_err(h, SOSO_HIP_DECLINED,
                                   "decode_create: layer " + std::to_string(l) + " " + r.role + ": " + why);
            }
        m.layers[l].attn_norm = (const float *)an->dev;
        m.layers[l].ffn_norm = (const float *)fn->dev;
        // a segmented down projection where it is built; whether its
        // consumer (the next q/k/v or the head) sums the partials is settled
        // once the whole stack is known
        m.layers[l].down_parts = !is_moe && !matvec_ex_unsupported(h, m.layers[l].down->dtype, H, F, XS_PLAIN, EPI_PARTS);
        m.layers[l].q_norm = qn ? (const float *)qn->dev : nullptr;
        m.layers[l].k_norm = kn ? (const float *)kn->dev : nullptr;
    }
    if (!layers_only) {
        const Weight *on;
        if (!get(kpl * L, 1, H, true, &on) || !get(kpl * L + 1, cfg->vocab, H, false, &m.head))
            return set_err(h, SOSO_HIP_DECLINED, "decode_create: output_norm/head missing or of the wrong shape");
        if (const char *why = matvec_ex_unsupported(h, m.head->dtype, cfg->vocab, H, XS_RMSNORM, EPI_STORE))
            return set_err(h, SOSO_HIP_DECLINED, std::string("decode_create: head: ") + why);
        m.out_norm = (const float *)on->dev;
    }
    // the consumer of each segmented down projection must take the partials;
    // where it cannot, the split-row form runs the projection, if it can
    for (size_t l = 0; l < L; l++) {
        DecodeLayer &dl = m.layers[l];
        if (!dl.down_parts) continue;
        if (l + 1 < L)
            dl.down_parts = !matvec_ex_unsupported(h, q[l + 1]->dtype, qd + 2 * kvd, H, XS_RMSNORM_P4, EPI_STORE);
        else dl.down_parts = m.head && !matvec_ex_unsupported(h, m.head->dtype, cfg->vocab, H, XS_RMSNORM_P4, EPI_STORE);
        if (!dl.down_parts)
            if (const char *why = matvec_ex_unsupported(h, dl.down->dtype, H, F, XS_PLAIN, EPI_RESID))
                return set_err(h, SOSO_HIP_DECLINED, "decode_create: layer " + std::to_string(l) + " down: " + why);
    }
    // what stays in use (dropping one of these unregisters the model)
    for (size_t l = 0; l < L; l++) {
        for (size_t j : {0, 4, 5, 8})
            if (!(j == 8 && m.layers[l].moe)) m.uses.emplace_back(keys[kpl * l + j], key_lens[kpl * l + j]);
        if (m.qk_norm)
            for (size_t j : {9, 10}) m.uses.emplace_back(keys[kpl * l + j], key_lens[kpl * l + j]);
    }
    if (!layers_only) {
        m.uses.emplace_back(keys[kpl * L], key_lens[kpl * L]);
        m.uses.emplace_back(keys[kpl * L + 1], key_lens[kpl * L + 1]);
    }
    // fused copies
    m.owned.resize(2 * L);
    for (size_t l = 0; l < L && rc == SOSO_HIP_OK; l++) {
        const bool dense = !m.layers[l].moe; // an MoE layer fuses q/k/v only
        const size_t st_qkv = packed_row_stride(q[l]->dtype, H), st_gu = dense ? packed_row_stride(g[l]->dtype, H) : 0;
        Weight &wq = m.owned[2 * l], &wg = m.owned[2 * l + 1];
        wq.dtype = q[l]->dtype;
        wq.rows = qd + 2 * kvd;
        wq.cols = H;
        wq.bytes = wq.rows * st_qkv;
        if (dense) {
            wg.dtype = g[l]->dtype;
            wg.rows = 2 * F;
            wg.cols = H;
            wg.bytes = wg.rows * st_gu;
        }
        // each allocation is counted as it succeeds, so decode_free's release
        // of whatever was allocated keeps h->used exact on a failure
        bool got = h->used + wq.bytes + wg.bytes <= h->budget && hipMalloc(&wq.dev, wq.bytes) == hipSuccess;
        if (got) h->used += wq.bytes;
        else wq.dev = nullptr;
        got = got && (!dense || hipMalloc(&wg.dev, wg.bytes) == hipSuccess);
        if (got) h->used += wg.bytes;
        else wg.dev = nullptr;
        if (!got) {
            rc = set_err(h, SOSO_HIP_DECLINED, "decode_create: no memory for the fused weights");
            break;
        }
        char *dq = (char *)wq.dev;
        rc = hip_check(h, hipMemcpyAsync(dq, q[l]->dev, qd * st_qkv, hipMemcpyDeviceToDevice, h->stream), "qkv copy");
        if (rc == SOSO_HIP_OK)
            rc = hip_check(h, hipMemcpyAsync(dq + qd * st_qkv, k[l]->dev, kvd * st_qkv, hipMemcpyDeviceToDevice,
                                             h->stream), "qkv copy");
        if (rc == SOSO_HIP_OK)
            rc = hip_check(h, hipMemcpyAsync(dq + (qd + kvd) * st_qkv, v[l]->dev, kvd * st_qkv,
                                             hipMemcpyDeviceToDevice, h->stream), "qkv copy");
        if (rc == SOSO_HIP_OK && dense)
            rc = hip_check(h, hipMemcpy2DAsync(wg.dev, 2 * st_gu, g[l]->dev, st_gu, st_gu, F, hipMemcpyDeviceToDevice,
                                               h->stream), "gate copy");
        if (rc == SOSO_HIP_OK && dense)
            rc = hip_check(h, hipMemcpy2DAsync((char *)wg.dev + st_gu, 2 * st_gu, u[l]->dev, st_gu, st_gu, F,
                                               hipMemcpyDeviceToDevice, h->stream), "up copy");
        m.layers[l].qkv = &wq;
        m.layers[l].gu = &wg;
    }
    // KV cache and step buffers
    const size_t kv_bytes = L * cfg->ctx_max * kvd * (m.kv_f16 ? 2 : 4);
    const size_t chunks = 1 + (cfg->ctx_max + ATT_CHUNK - 1) / ATT_CHUNK; // attention partials per head, at most
    const size_t act_floats = H + (qd + 2 * kvd) + qd + F + (size_t)cfg->n_heads * chunks * (cfg->head_dim + 2) +
                              m.vocab + 64 + cfg->head_dim / 2 + H + H + (size_t)MV_SEG * H;
    // MoE scratch (shared by the MoE layers, which run one after another) and
    // each layer's routing of the last step (256-byte slots)
    const size_t moe_route_bytes = 512;
    const size_t moe_bytes = n_moe ? moe_need + n_moe * moe_route_bytes : 0;
    const size_t mem_bytes = act_floats * 4;
    if (rc == SOSO_HIP_OK) {
        if (hipMalloc(&m.kcache, 2 * kv_bytes) != hipSuccess || hipMalloc(&m.mem, mem_bytes) != hipSuccess ||
            (moe_bytes && hipMalloc(&m.moe_mem, moe_bytes) != hipSuccess))
            rc = set_err(h, SOSO_HIP_DECLINED, "decode_create: no memory for the KV cache");
    }
    if (rc == SOSO_HIP_OK) rc = hip_check(h, hipMemsetAsync(m.kcache, 0, 2 * kv_bytes, h->stream), "kv zero");
    if (rc == SOSO_HIP_OK) rc = hip_check(h, hipMemsetAsync(m.mem, 0, mem_bytes, h->stream), "step buffers zero");
    if (rc == SOSO_HIP_OK) rc = hip_check(h, hipStreamSynchronize(h->stream), "decode_create sync");
    if (rc != SOSO_HIP_OK) {
        (void)decode_free(h, m);
        return rc;
    }
    m.vcache = (char *)m.kcache + kv_bytes;
    float *f = (float *)m.mem;
    m.hid = f;
    m.qkv_raw = f + H;
    m.att = m.qkv_raw + qd + 2 * kvd;
    m.act = m.att + qd;
    m.part = m.act + F;
    m.logits = m.part + (size_t)cfg->n_heads * chunks * (cfg->head_dim + 2);
    m.rope_freq = m.logits + m.vocab + 64;
    m.xn = m.rope_freq + cfg->head_dim / 2;
    m.hid2 = m.xn + H;
    m.dpart = m.hid2 + H;
    for (size_t l = 0, j = 0; l < L; l++) {
        DecodeLayer &dl = m.layers[l];
        if (!dl.moe) continue;
        const MoeLayer &ml = *dl.moe;
        moe_scratch_fixed(h, 1, ml.n_exp, ml.top_k, ml.hdim, ml.ffn, m.moe_mem, moe_need, dl.moe_s);
        char *r = (char *)m.moe_mem + moe_need + j++ * moe_route_bytes; // top_k <= 8: 32 + 32 bytes
        dl.moe_s.idx = (int32_t *)r;
        dl.moe_s.wgt = (float *)(r + 256);
    }
    {
        // rope_cabezas (gemm.rs:1468-1470): freq_i = powf(theta, -2 i / head_dim) in f32
        std::vector<float> fr(cfg->head_dim / 2);
        const float n_f = (float)cfg->head_dim;
        for (size_t i = 0; i < fr.size(); i++) fr[i] = powf(cfg->rope_theta, -2.0f * (float)i / n_f);
        rc = hip_check(h, hipMemcpy(m.rope_freq, fr.data(), fr.size() * 4, hipMemcpyHostToDevice), "rope table");
        if (rc != SOSO_HIP_OK) {
            (void)decode_free(h, m);
            return rc;
        }
    }
    std::string key(model_key, model_key_len);
    auto old = h->decode_models.find(key);
    if (old != h->decode_models.end()) {
        rc = decode_free(h, old->second);
        h->decode_models.erase(old);
    }
    DecodeModel &dm = h->decode_models.emplace(key, std::move(m)).first->second;
    for (size_t l = 0; l < L; l++) { // the owned vector moved: re-point the layers at it
        dm.layers[l].qkv = &dm.owned[2 * l];
        dm.layers[l].gu = &dm.owned[2 * l + 1];
    }
    if (drop_sources)
        for (size_t l = 0; l < L; l++)
            for (size_t j : {1, 2, 3, 6, 7})
                if (!(j >= 6 && dm.layers[l].moe)) soso_hip_weight_drop(h, keys[kpl * l + j], key_lens[kpl * l + j]);
    return SOSO_HIP_OK;
}

int soso_hip_decode_create(soso_hip *h, const char *model_key, size_t model_key_len, const soso_hip_decode_cfg *cfg,
                           const char *const *keys, const size_t *key_lens, int drop_sources)
{
    return decode_create_impl(h, model_key, model_key_len, cfg, 0, keys, key_lens, nullptr, nullptr, drop_sources);
}

int soso_hip_decode_create_moe(soso_hip *h, const char *model_key, size_t model_key_len,
                               const soso_hip_decode_cfg *cfg, const char *const *keys, const size_t *key_lens,
                               const char *const *moe_layer_keys, const size_t *moe_layer_key_lens, int drop_sources)
{
    if (h && (!moe_layer_keys || !moe_layer_key_lens)) return set_err(h, SOSO_HIP_ERR_ARG, "decode_create_moe: args");
    return decode_create_impl(h, model_key, model_key_len, cfg, 0, keys, key_lens, moe_layer_keys, moe_layer_key_lens,
                              drop_sources);
}

int soso_hip_decode_create_ex(soso_hip *h, const char *model_key, size_t model_key_len,
                              const soso_hip_decode_cfg *cfg, uint32_t flags, const char *const *keys,
                              const size_t *key_lens, const char *const *moe_layer_keys,
                              const size_t *moe_layer_key_lens, int drop_sources)
{
    if (h && moe_layer_keys && !moe_layer_key_lens) return set_err(h, SOSO_HIP_ERR_ARG, "decode_create_ex: args");
    return decode_create_impl(h, model_key, model_key_len, cfg, flags, keys, key_lens, moe_layer_keys,
                              moe_layer_key_lens, drop_sources);
}

int soso_hip_decode_moe_routing_dev(soso_hip *h, const char *model_key, size_t model_key_len, uint32_t layer,
                                    int32_t **idx_dev, float **wgt_dev)
{
    if (!h || !model_key || !idx_dev || !wgt_dev) return SOSO_HIP_ERR_ARG;
    auto it = h->decode_models.find(std::string(model_key, model_key_len));
    if (it == h->decode_models.end()) return set_err(h, SOSO_HIP_DECLINED, "decode_moe_routing: no such model");
    if (layer >= it->second.n_layers || !it->second.layers[layer].moe)
        return set_err(h, SOSO_HIP_ERR_ARG, "decode_moe_routing: not an MoE layer");
    *idx_dev = it->second.layers[layer].moe_s.idx;
    *wgt_dev = it->second.layers[layer].moe_s.wgt;
    return SOSO_HIP_OK;
}

int soso_hip_decode_kv_dev(soso_hip *h, const char *model_key, size_t model_key_len, uint32_t layer, void **k_dev,
                           void **v_dev)
{
    if (!h || !model_key || !k_dev || !v_dev) return SOSO_HIP_ERR_ARG;
    auto it = h->decode_models.find(std::string(model_key, model_key_len));
    if (it == h->decode_models.end()) return set_err(h, SOSO_HIP_DECLINED, "decode_kv: model not registered");
    const DecodeModel &m = it->second;
    if (layer >= m.n_layers) return set_err(h, SOSO_HIP_ERR_ARG, "decode_kv: layer");
    const size_t per = m.ctx_max * m.n_kv_heads * m.head_dim * (m.kv_f16 ? 2 : 4);
    *k_dev = (char *)m.kcache + layer * per;
    *v_dev = (char *)m.vcache + layer * per;
    return SOSO_HIP_OK;
}

int soso_hip_decode_kv_upload(soso_hip *h, const char *model_key, size_t model_key_len, uint32_t layer, uint32_t row0,
                              uint32_t n_rows, const void *k_rows, const void *v_rows, int rows_f32)
{
    if (!h) return SOSO_HIP_ERR_ARG;
    if (!model_key || (n_rows && (!k_rows || !v_rows))) return set_err(h, SOSO_HIP_ERR_ARG, "decode_kv_upload: args");
    if (h->capturing) return set_err(h, SOSO_HIP_ERR_ARG, "decode_kv_upload: not inside graph capture");
    auto it = h->decode_models.find(std::string(model_key, model_key_len));
    if (it == h->decode_models.end()) return set_err(h, SOSO_HIP_DECLINED, "decode_kv_upload: model not registered");
    const DecodeModel &m = it->second;
    if (layer >= m.n_layers) return set_err(h, SOSO_HIP_ERR_ARG, "decode_kv_upload: layer");
    if ((size_t)row0 + n_rows > m.ctx_max) return set_err(h, SOSO_HIP_ERR_ARG, "decode_kv_upload: rows beyond ctx_max");
    if (n_rows == 0) return SOSO_HIP_OK;
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    const size_t kvd = m.n_kv_heads * m.head_dim;
    const bool src_f32 = rows_f32 != 0 || !m.kv_f16;
    const size_t bytes = (size_t)n_rows * kvd * (src_f32 ? 4 : 2);
    void *stage = scratch_get(h, 11, bytes);
    if (!stage) return set_err(h, SOSO_HIP_DECLINED, "decode_kv_upload: no memory for staging");
    const size_t per = m.ctx_max * kvd * (m.kv_f16 ? 2 : 4);
    for (int which = 0; which < 2 && rc == SOSO_HIP_OK; which++) {
        const void *src = which ? v_rows : k_rows;
        void *cache = (char *)(which ? m.vcache : m.kcache) + layer * per;
        // host or device source: the runtime tells them apart (unified addressing)
        rc = hip_check(h, hipMemcpyAsync(stage, src, bytes, hipMemcpyDefault, h->stream), "kv rows copy");
        if (rc == SOSO_HIP_OK)
            rc = launch_kv_scatter(h, stage, src_f32, cache, m.kv_f16, (int)kvd, (int)m.head_dim, (int)m.ctx_max,
                                   (int)row0, (int)n_rows);
        // the staging buffer is reused for V: K's scatter must have read it
        if (rc == SOSO_HIP_OK) rc = hip_check(h, hipStreamSynchronize(h->stream), "kv upload sync");
    }
    if (rc == SOSO_HIP_OK) h->stats.bytes_up += 2 * bytes;
    return rc;
}

int soso_hip_decode_step_dev(soso_hip *h, const char *model_key, size_t model_key_len, const float *x_dev, uint32_t pos,
                             float *logits_dev, uint32_t *token_dev, void *kv_rows_dev)
{
    if (!h) return SOSO_HIP_ERR_ARG;
    if (!model_key || !x_dev) return set_err(h, SOSO_HIP_ERR_ARG, "decode_step: args");
    auto it = h->decode_models.find(std::string(model_key, model_key_len));
    if (it == h->decode_models.end()) return set_err(h, SOSO_HIP_DECLINED, "decode_step: model not registered");
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    if (it->second.n_host_moe)
        return set_err(h, SOSO_HIP_DECLINED,
                       "decode_step: the model has MoE layers whose experts stay on the host (soso_hip_decode_token)");
    return decode_step(h, it->second, x_dev, pos, logits_dev, token_dev, kv_rows_dev);
}

int soso_hip_decode_token(soso_hip *h, const char *model_key, size_t model_key_len, const float *embed, uint32_t pos,
                          soso_hip_cpu_moe_fn cpu_moe, void *cpu_moe_ctx, float *logits, void *kv_rows,
                          uint32_t *token)
{
    if (!h) return SOSO_HIP_ERR_ARG;
    if (!model_key || !embed) return set_err(h, SOSO_HIP_ERR_ARG, "decode_token: args");
    if (h->capturing) return set_err(h, SOSO_HIP_DECLINED, "decode_token: synchronous, not inside graph capture");
    auto it = h->decode_models.find(std::string(model_key, model_key_len));
    if (it == h->decode_models.end()) return set_err(h, SOSO_HIP_DECLINED, "decode_token: model not registered");
    DecodeModel &m = it->second;
    if (m.n_host_moe && !cpu_moe)
        return set_err(h, SOSO_HIP_DECLINED, "decode_token: the model's host-side experts need cpu_moe");
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    CallClock clk(h);
    const size_t H = m.hidden, esz = m.kv_f16 ? 2 : 4;
    const size_t kv_bytes = m.n_layers * 2 * m.n_kv_heads * m.head_dim * esz;
    // device staging: the step's KV rows, then its token
    char *dev = (char *)scratch_get(h, 6, kv_bytes + 256);
    if (!dev) return set_err(h, SOSO_HIP_ERR_NOMEM, "decode_token: staging");
    uint32_t *tok_dev = (uint32_t *)(dev + ((kv_bytes + 255) & ~(size_t)255));
    // the embedding row becomes the hidden state (layer 0 reads it in place)
    rc = hip_check(h, hipMemcpyAsync(m.hid, embed, H * 4, hipMemcpyHostToDevice, h->stream), "embed upload");
    HostMoe hm;
    hm.fn = cpu_moe;
    hm.ctx = cpu_moe_ctx;
    if (rc == SOSO_HIP_OK) rc = decode_step(h, m, m.hid, pos, nullptr, tok_dev, kv_rows ? dev : nullptr, &hm);
    if (rc == SOSO_HIP_OK && logits)
        rc = hip_check(h, hipMemcpyAsync(logits, m.logits, m.vocab * 4, hipMemcpyDeviceToHost, h->stream), "logits");
    if (rc == SOSO_HIP_OK && kv_rows)
        rc = hip_check(h, hipMemcpyAsync(kv_rows, dev, kv_bytes, hipMemcpyDeviceToHost, h->stream), "kv rows");
    if (rc == SOSO_HIP_OK && token)
        rc = hip_check(h, hipMemcpyAsync(token, tok_dev, 4, hipMemcpyDeviceToHost, h->stream), "token");
    if (rc == SOSO_HIP_OK) rc = hip_check(h, hipStreamSynchronize(h->stream), "decode_token sync");
    if (rc != SOSO_HIP_OK) return rc;
    h->stats.decode_embed_up += H * 4;
    h->stats.decode_logits_down += logits ? m.vocab * 4 : 0;
    h->stats.decode_kv_down += kv_rows ? kv_bytes : 0;
    h->stats.decode_steps++;
    clk.done();
    return SOSO_HIP_OK;
}

int soso_hip_decode_destroy(soso_hip *h, const char *model_key, size_t model_key_len)
{
    if (!h || !model_key) return SOSO_HIP_ERR_ARG;
    auto it = h->decode_models.find(std::string(model_key, model_key_len));
    if (it == h->decode_models.end()) return SOSO_HIP_DECLINED;
    const int rc = decode_free(h, it->second);
    h->decode_models.erase(it);
    return rc;
}

// ---- one GQA-MoE layer at a time (GpuDispatch::moe_capa) ---------------------
// The layer runs as a one-layer device step without a head (decode_step over a
// layers_only model: the attention with its f16 KV cache, then the MoE FFN of
// the layer registered from the caller's experts), token by token.  The
// output of a chained call (encadenar) stays in the step's hidden buffer, or,
// for several tokens, in scratch slot 15, until the next layer reads it
// (continuar) or soso_hip_moe_capa_flush brings it down.
static bool moe_capa_is_discarded(const soso_hip *h, uint32_t layer)
{
    return std::find(h->moe_capa_discarded.begin(), h->moe_capa_discarded.end(), layer) !=
           h->moe_capa_discarded.end();
}

static int moe_capa_drop(soso_hip *h, uint32_t layer)
{
    auto it = h->moe_capas.find(layer);
    if (it == h->moe_capas.end()) return SOSO_HIP_OK;
    int rc = SOSO_HIP_OK;
    auto dm = h->decode_models.find(it->second.model);
    if (dm != h->decode_models.end()) {
        rc = decode_free(h, dm->second);
        h->decode_models.erase(dm);
    }
    // the library's own keys (dropping the router also unregisters the MoE layer)
    for (const std::string &k : it->second.own_keys) {
        const int r = soso_hip_weight_drop(h, k.data(), k.size());
        if (r < 0) rc = first_fail(rc, r);
    }
    if (h->moe_pend.valid && h->moe_pend.layer == layer) h->moe_pend.valid = false;
    h->moe_capas.erase(it);
    return rc;
}

// First call of a layer: its norms and router become resident under the
// library's own keys, its MoE FFN is registered and its one-layer step built.
static int moe_capa_prepare(soso_hip *h, const soso_hip_moe_capa *c)
{
    const size_t H = c->hidden_dim, hd = c->head_dim;
    if (!c->attn_norm || !c->ffn_norm || !c->router || (c->qk_norm && (!c->q_norm || !c->k_norm)))
        return set_err(h, SOSO_HIP_ERR_ARG, "moe_capa: the layer's first call needs its norms and router (MoeNormas)");
    soso_hip::MoeCapaLayer st;
    const std::string base = "moe_capa.L" + std::to_string(c->layer);
    st.model = base;
    st.moe_key = base + ".moe";
    st.theta = c->theta;
    st.eps = c->eps;
    st.qk_norm = c->qk_norm ? 1 : 0;
    int rc = SOSO_HIP_OK;
    auto put = [&](const std::string &k, const float *v, size_t rows, size_t cols) {
        if (rc != SOSO_HIP_OK) return;
        Weight *w = nullptr;
        (void)soso_hip_weight_drop(h, k.data(), k.size()); // a stale copy from an earlier life of the layer
        rc = get_weight(h, k.data(), k.size(), (const uint8_t *)v, rows * cols * 4, SOSO_HIP_DTYPE_F32, rows, cols, &w);
        if (rc == SOSO_HIP_OK) st.own_keys.push_back(k);
    };
    put(base + ".attn_norm", c->attn_norm, 1, H);
    put(base + ".ffn_norm", c->ffn_norm, 1, H);
    if (c->qk_norm) {
        put(base + ".q_norm", c->q_norm, 1, hd);
        put(base + ".k_norm", c->k_norm, 1, hd);
    }
    put(base + ".router", c->router, c->n_exp, H);
    std::vector<std::string> ek;
    std::vector<const char *> ep;
    std::vector<size_t> el;
    if (rc == SOSO_HIP_OK) {
        static const char *const part[3] = {"ffn_gate", "ffn_up", "ffn_down"};
        ek.reserve(3 * c->n_exp);
        for (size_t e = 0; e < c->n_exp; e++)
            for (int j = 0; j < 3; j++) {
                char num[24];
                snprintf(num, sizeof num, "%02zu", e);
                ek.push_back(std::string(c->prefix) + ".E" + num + "." + part[j]);
            }
        for (const std::string &k : ek) {
            ep.push_back(k.data());
            el.push_back(k.size());
        }
        const std::string rk = base + ".router";
        rc = moe_register_impl(h, st.moe_key.data(), st.moe_key.size(), rk.data(), rk.size(), ep.data(), el.data(),
                               c->n_exp, H, c->ffn, c->top_k, false);
    }
    if (rc == SOSO_HIP_OK) {
        soso_hip_decode_cfg cfg{};
        cfg.n_layers = 1;
        cfg.hidden = (uint32_t)H;
        cfg.n_heads = (uint32_t)c->heads;
        cfg.n_kv_heads = (uint32_t)c->kv_heads;
        cfg.head_dim = (uint32_t)hd;
        cfg.ffn = 1; // the layer's FFN is the MoE layer
        cfg.vocab = 0;
        cfg.ctx_max = (uint32_t)c->ctx_max;
        cfg.rope_theta = c->theta;
        cfg.rms_eps = c->eps;
        cfg.kv_f16 = 1; // soso's device MoE layers keep an f16 KV (moe_gpu.rs:47)
        const std::string an = base + ".attn_norm", fn = base + ".ffn_norm", qn = base + ".q_norm",
                          kn = base + ".k_norm";
        const char *keys[11] = {an.data(), c->key_q, c->key_k, c->key_v, c->key_o, fn.data(), nullptr, nullptr,
                                nullptr, qn.data(), kn.data()};
        size_t lens[11] = {an.size(), strlen(c->key_q), strlen(c->key_k), strlen(c->key_v), strlen(c->key_o),
                           fn.size(), 0, 0, 0, qn.size(), kn.size()};
        const char *mk[1] = {st.moe_key.data()};
        const size_t ml[1] = {st.moe_key.size()};
        const uint32_t flags = SOSO_HIP_DECODE_ROPE_NEOX | (c->qk_norm ? SOSO_HIP_DECODE_QK_NORM : 0u);
        rc = decode_create_impl(h, st.model.data(), st.model.size(), &cfg, flags, keys, lens, mk, ml, 0, true);
    }
    const std::string err = h->err;
    h->moe_capas[c->layer] = st;
    if (rc != SOSO_HIP_OK) {
        (void)moe_capa_drop(h, c->layer);
        h->err = err;
    }
    return rc;
}

int soso_hip_moe_capa_run(soso_hip *h, const soso_hip_moe_capa *c, float *hidden)
{
    if (!h) return SOSO_HIP_ERR_ARG;
    if (!c || !c->key_q || !c->key_k || !c->key_v || !c->key_o || !c->prefix || c->n == 0 || c->hidden_dim == 0 ||
        c->heads == 0 || c->kv_heads == 0 || c->n_exp == 0 || c->top_k == 0 || (!hidden && !c->encadenar) ||
        (!hidden && !c->continuar))
        return set_err(h, SOSO_HIP_ERR_ARG, "moe_capa: args");
    if (h->capturing) return set_err(h, SOSO_HIP_ERR_ARG, "moe_capa: not inside graph capture");
    if (moe_capa_is_discarded(h, c->layer)) return set_err(h, SOSO_HIP_DECLINED, "moe_capa: layer discarded");
    // what the device step does not run: the CPU keeps the layer
    if (c->ventana > 0) return set_err(h, SOSO_HIP_DECLINED, "moe_capa: sliding-window attention");
    if (c->rope_factors || c->rope_mscale != 1.0f) return set_err(h, SOSO_HIP_DECLINED, "moe_capa: YaRN RoPE");
    if (c->head_dim == 0 || c->escala != 1.0f / sqrtf((float)c->head_dim))
        return set_err(h, SOSO_HIP_DECLINED, "moe_capa: attention scale other than 1/sqrt(head_dim)");
    if (c->pos0 + c->n > c->ctx_max) return set_err(h, SOSO_HIP_DECLINED, "moe_capa: positions beyond ctx_max");
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    CallClock clk(h);
    auto it = h->moe_capas.find(c->layer);
    if (it != h->moe_capas.end() &&
        (it->second.theta != c->theta || it->second.eps != c->eps || it->second.qk_norm != (c->qk_norm ? 1 : 0) ||
         !h->decode_models.count(it->second.model))) {
        // the layer's configuration changed, or a weight its step read was
        // dropped: built again (from the norms this call must then carry)
        rc = moe_capa_drop(h, c->layer);
        if (rc < 0) return rc;
        it = h->moe_capas.end();
    }
    if (it == h->moe_capas.end()) {
        rc = moe_capa_prepare(h, c);
        if (rc != SOSO_HIP_OK) return rc;
        it = h->moe_capas.find(c->layer);
    }
    soso_hip::MoeCapaLayer &st = it->second;
    auto dmi = h->decode_models.find(st.model);
    if (dmi == h->decode_models.end()) return set_err(h, SOSO_HIP_ERR, "moe_capa: the layer's step is gone");
    DecodeModel &m = dmi->second;
    const size_t H = c->hidden_dim;
    if (m.hidden != H || m.n_heads != c->heads || m.n_kv_heads != c->kv_heads || m.head_dim != c->head_dim ||
        !m.layers[0].moe || m.layers[0].moe->n_exp != c->n_exp || m.layers[0].moe->top_k != c->top_k ||
        m.layers[0].moe->ffn != c->ffn || m.ctx_max < c->ctx_max)
        return set_err(h, SOSO_HIP_ERR_ARG, "moe_capa: the layer's shape differs from its first call");
    // the positions before pos0 must be in this layer's device KV (computed here)
    if (c->pos0 > st.kv_pos)
        return set_err(h, SOSO_HIP_DECLINED, "moe_capa: earlier positions of the layer were not computed here");
    // input: the pending output of layer - 1 (continuar), or the caller's hidden
    const float *xin = nullptr;
    if (c->continuar) {
        if (!h->moe_pend.valid || h->moe_pend.layer + 1 != c->layer || h->moe_pend.pos0 != c->pos0 ||
            h->moe_pend.n != c->n || h->moe_pend.width != H)
            return set_err(h, SOSO_HIP_ERR_ARG, "moe_capa: continuar without the previous layer's pending output");
        xin = h->moe_pend.dev;
    } else {
        float *xd = (float *)scratch_get(h, 14, c->n * H * 4);
        if (!xd) return set_err(h, SOSO_HIP_ERR_NOMEM, "moe_capa: input staging");
        rc = hip_check(h, hipMemcpyAsync(xd, hidden, c->n * H * 4, hipMemcpyHostToDevice, h->stream), "hidden up");
        if (rc != SOSO_HIP_OK) return rc;
        h->stats.bytes_up += c->n * H * 4;
        xin = xd;
    }
    // several tokens: their outputs gather in scratch slot 15 (the previous
    // layer's, when it is the input, is copied aside first)
    float *outs = nullptr;
    if (c->n > 1) {
        if (c->continuar && h->moe_pend.dev != m.hid) {
            float *tmp = (float *)scratch_get(h, 14, c->n * H * 4);
            if (!tmp) return set_err(h, SOSO_HIP_ERR_NOMEM, "moe_capa: input staging");
            rc = hip_check(h, hipMemcpyAsync(tmp, xin, c->n * H * 4, hipMemcpyDeviceToDevice, h->stream), "pending");
            if (rc != SOSO_HIP_OK) return rc;
            xin = tmp;
        }
        outs = (float *)scratch_get(h, 15, c->n * H * 4);
        if (!outs) return set_err(h, SOSO_HIP_ERR_NOMEM, "moe_capa: output staging");
    }
    h->moe_pend.valid = false;
    for (size_t t = 0; t < c->n && rc == SOSO_HIP_OK; t++) {
        rc = decode_step(h, m, xin + t * H, (uint32_t)(c->pos0 + t), nullptr, nullptr, nullptr);
        if (rc == SOSO_HIP_OK && outs)
            rc = hip_check(h, hipMemcpyAsync(outs + t * H, m.hid, H * 4, hipMemcpyDeviceToDevice, h->stream),
                           "token output");
    }
    if (rc != SOSO_HIP_OK) {
        (void)hip_release(h, hipStreamSynchronize(h->stream), "moe_capa drain");
        return rc;
    }
    st.kv_pos = c->pos0 + c->n;
    const float *res = outs ? outs : m.hid;
    if (c->encadenar) {
        h->moe_pend.valid = true;
        h->moe_pend.layer = c->layer;
        h->moe_pend.pos0 = c->pos0;
        h->moe_pend.n = c->n;
        h->moe_pend.width = H;
        h->moe_pend.dev = res;
        clk.done();
        return SOSO_HIP_OK;
    }
    rc = hip_check(h, hipMemcpyAsync(hidden, res, c->n * H * 4, hipMemcpyDeviceToHost, h->stream), "hidden down");
    if (rc == SOSO_HIP_OK) rc = hip_check(h, hipStreamSynchronize(h->stream), "moe_capa sync");
    if (rc != SOSO_HIP_OK) return rc;
    h->stats.bytes_down += c->n * H * 4;
    clk.done();
    return SOSO_HIP_OK;
}

int soso_hip_moe_capa_can(const soso_hip *h, uint32_t layer)
{
    return h && !moe_capa_is_discarded(h, layer) ? 1 : 0;
}

int soso_hip_moe_capa_ready(const soso_hip *h, uint32_t layer)
{
    if (!h) return 0;
    auto it = h->moe_capas.find(layer);
    return it != h->moe_capas.end() && h->decode_models.count(it->second.model) ? 1 : 0;
}

int soso_hip_moe_capa_pending(const soso_hip *h, uint32_t layer, size_t pos0, size_t n)
{
    return h && h->moe_pend.valid && h->moe_pend.layer == layer && h->moe_pend.pos0 == pos0 && h->moe_pend.n == n
               ? 1
               : 0;
}

int soso_hip_moe_capa_flush(soso_hip *h, float *hidden)
{
    if (!h) return SOSO_HIP_ERR_ARG;
    if (!h->moe_pend.valid) return SOSO_HIP_OK;
    if (!hidden) return set_err(h, SOSO_HIP_ERR_ARG, "moe_capa_flush: args");
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    const size_t bytes = h->moe_pend.n * h->moe_pend.width * 4;
    rc = hip_check(h, hipMemcpyAsync(hidden, h->moe_pend.dev, bytes, hipMemcpyDeviceToHost, h->stream), "pending down");
    if (rc == SOSO_HIP_OK) rc = hip_check(h, hipStreamSynchronize(h->stream), "moe_capa_flush sync");
    if (rc != SOSO_HIP_OK) return rc;
    h->stats.bytes_down += bytes;
    h->moe_pend.valid = false;
    return SOSO_HIP_OK;
}

void soso_hip_moe_capa_discard(soso_hip *h, uint32_t layer)
{
    if (!h) return;
    if (make_current(h) == SOSO_HIP_OK) (void)moe_capa_drop(h, layer);
    if (!moe_capa_is_discarded(h, layer)) h->moe_capa_discarded.push_back(layer);
}

int soso_hip_moe_capa_kv_dev(soso_hip *h, uint32_t layer, void **k_dev, void **v_dev)
{
    if (!h || !k_dev || !v_dev) return SOSO_HIP_ERR_ARG;
    auto it = h->moe_capas.find(layer);
    if (it == h->moe_capas.end()) return set_err(h, SOSO_HIP_DECLINED, "moe_capa_kv: layer not prepared");
    return soso_hip_decode_kv_dev(h, it->second.model.data(), it->second.model.size(), 0, k_dev, v_dev);
}

int soso_hip_moe_capa_routing_dev(soso_hip *h, uint32_t layer, int32_t **idx_dev, float **wgt_dev)
{
    if (!h || !idx_dev || !wgt_dev) return SOSO_HIP_ERR_ARG;
    auto it = h->moe_capas.find(layer);
    if (it == h->moe_capas.end()) return set_err(h, SOSO_HIP_DECLINED, "moe_capa_routing: layer not prepared");
    return soso_hip_decode_moe_routing_dev(h, it->second.model.data(), it->second.model.size(), 0, idx_dev, wgt_dev);
}

int soso_hip_weight_upload(soso_hip *h, const char *key, size_t key_len, const uint8_t *w, size_t w_len,
                           uint8_t dtype, size_t rows, size_t cols)
{
    if (!h) return SOSO_HIP_ERR_ARG;
    if (!key || !w || rows == 0 || cols == 0) return set_err(h, SOSO_HIP_ERR_ARG, "weight_upload: args");
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    Weight *wt = nullptr;
    return get_weight(h, key, key_len, w, w_len, dtype, rows, cols, &wt);
}

int soso_hip_weight_resident(const soso_hip *h, const char *key, size_t key_len)
{
    if (!h || !key) return 0;
    auto it = h->weights.find(std::string(key, key_len));
    return it != h->weights.end() && !it->second.declined ? 1 : 0;
}

// ---- device-resident API ----------------------------------------------------
int soso_hip_dev_alloc(soso_hip *h, size_t bytes, void **dptr)
{
    if (!h || !dptr) return SOSO_HIP_ERR_ARG;
    *dptr = nullptr;
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    return hip_check(h, hipMalloc(dptr, bytes ? bytes : 16), "hipMalloc");
}

int soso_hip_dev_free(soso_hip *h, void *dptr)
{
    if (!h) return SOSO_HIP_ERR_ARG;
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    rc = hip_check(h, hipStreamSynchronize(h->stream), "dev_free sync");
    return first_fail(rc, hip_check(h, hipFree(dptr), "hipFree"));
}

int soso_hip_h2d(soso_hip *h, void *dst, const void *src, size_t bytes)
{
    if (!h || !dst || !src) return SOSO_HIP_ERR_ARG;
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    rc = hip_check(h, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, h->stream), "h2d");
    return rc == SOSO_HIP_OK ? hip_check(h, hipStreamSynchronize(h->stream), "h2d sync") : rc;
}

int soso_hip_d2h(soso_hip *h, void *dst, const void *src, size_t bytes)
{
    if (!h || !dst || !src) return SOSO_HIP_ERR_ARG;
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    rc = hip_check(h, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, h->stream), "d2h");
    return rc == SOSO_HIP_OK ? hip_check(h, hipStreamSynchronize(h->stream), "d2h sync") : rc;
}

int soso_hip_sync(soso_hip *h)
{
    if (!h) return SOSO_HIP_ERR_ARG;
    int rc = make_current(h);
    return rc == SOSO_HIP_OK ? hip_check(h, hipStreamSynchronize(h->stream), "sync") : rc;
}

int soso_hip_d2d(soso_hip *h, void *dst, const void *src, size_t bytes)
{
    if (!h || !dst || !src) return SOSO_HIP_ERR_ARG;
    int rc = make_current(h);
    return rc == SOSO_HIP_OK ? hip_check(h, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, h->stream), "d2d")
                             : rc;
}

int soso_hip_weight_from_dev(soso_hip *h, const char *key, size_t key_len, const void *raw_dev, size_t w_len,
                             uint8_t dtype, size_t rows, size_t cols)
{
    if (!h || !key || !raw_dev) return SOSO_HIP_ERR_ARG;
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    std::string k(key, key_len);
    if (h->weights.count(k)) return set_err(h, SOSO_HIP_ERR_ARG, "weight " + k + " already registered");
    Weight *w = nullptr;
    return register_weight(h, k, raw_dev, true, w_len, dtype, rows, cols, &w);
}

int soso_hip_synth_raw(soso_hip *h, void *dst, uint8_t dtype, size_t rows, size_t cols, uint64_t seed,
                       uint64_t stream)
{
    if (!h || !dst) return SOSO_HIP_ERR_ARG;
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    return launch_synth_raw(h, dst, dtype, rows, cols, seed, stream);
}

int soso_hip_synth_normal(soso_hip *h, float *dst, size_t n, float sigma, uint64_t seed, uint64_t stream)
{
    if (!h || !dst) return SOSO_HIP_ERR_ARG;
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    return launch_synth_normal(h, dst, n, sigma, seed, stream);
}

int soso_hip_read_probe(soso_hip *h, const void *src_dev, size_t bytes, uint32_t wg_per_cu, uint32_t threads,
                        uint32_t loads, uint32_t chunked, uint32_t *out_dev, size_t out_len)
{
    if (!h) return SOSO_HIP_ERR_ARG;
    if (!src_dev || !out_dev || bytes < 16 || wg_per_cu == 0 || wg_per_cu > 32 || threads == 0 || threads > 1024 ||
        threads % 64 || !(loads == 1 || loads == 2 || loads == 4 || loads == 8 || loads == 16) ||
        (chunked && (bytes < 1024 || bytes >= (1ull << 31))))
        return set_err(h, SOSO_HIP_ERR_ARG, "read_probe: args");
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    return launch_read_probe(h, src_dev, bytes, wg_per_cu, threads, loads, chunked & 1u, (chunked & 2u) != 0, out_dev,
                             out_len);
}

int soso_hip_weight_synth(soso_hip *h, const char *key, size_t key_len, uint8_t dtype, size_t rows, size_t cols,
                          uint64_t seed, uint64_t stream)
{
    if (!h || !key) return SOSO_HIP_ERR_ARG;
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    const size_t rb = fmt_row_bytes(dtype, cols);
    if (rb == 0 || dtype == SOSO_HIP_DTYPE_F32) return set_err(h, SOSO_HIP_ERR_ARG, "weight_synth: dtype/shape");
    void *raw = nullptr;
    if (hipMalloc(&raw, rows * rb) != hipSuccess) return set_err(h, SOSO_HIP_ERR_NOMEM, "weight_synth: alloc");
    rc = launch_synth_raw(h, raw, dtype, rows, cols, seed, stream);
    if (rc == SOSO_HIP_OK) rc = soso_hip_weight_from_dev(h, key, key_len, raw, rows * rb, dtype, rows, cols);
    rc = first_fail(rc, hip_release(h, hipStreamSynchronize(h->stream), "weight_synth sync"));
    return first_fail(rc, hip_release(h, hipFree(raw), "free synth staging"));
}

int soso_hip_weight_drop(soso_hip *h, const char *key, size_t key_len)
{
    if (!h || !key) return SOSO_HIP_ERR_ARG;
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    auto it = h->weights.find(std::string(key, key_len));
    if (it == h->weights.end()) return SOSO_HIP_DECLINED;
    rc = hip_release(h, hipStreamSynchronize(h->stream), "weight_drop sync");
    // a registered MoE layer that reads this weight is unregistered with it
    for (auto m = h->moe_layers.begin(); m != h->moe_layers.end();) {
        bool uses = m->second.router == &it->second;
        for (const void *p : m->second.host_tab) uses = uses || (p && p == it->second.dev);
        if (uses) {
            rc = first_fail(rc, drop_models_using_moe(h, m->first));
            rc = first_fail(rc, moe_free(h, m->second));
            m = h->moe_layers.erase(m);
        } else {
            ++m;
        }
    }
    // ... and so is a decode model that reads it
    for (auto m = h->decode_models.begin(); m != h->decode_models.end();) {
        if (std::find(m->second.uses.begin(), m->second.uses.end(), it->first) != m->second.uses.end()) {
            rc = first_fail(rc, decode_free(h, m->second));
            m = h->decode_models.erase(m);
        } else {
            ++m;
        }
    }
    if (it->second.dev) {
        rc = first_fail(rc, hip_release(h, hipFree(it->second.dev), "free weight"));
        h->used -= it->second.bytes;
        h->stats.weight_bytes_resident -= it->second.bytes;
        h->stats.weights_resident--;
    }
    h->weights.erase(it);
    return rc;
}

int soso_hip_matvec_dev(soso_hip *h, const char *key, size_t key_len, const float *x_dev, float *y_dev)
{
    return soso_hip_matmul_dev(h, key, key_len, 1, x_dev, y_dev);
}

int soso_hip_matmul_dev(soso_hip *h, const char *key, size_t key_len, size_t n, const float *x_dev, float *y_dev)
{
    if (!h || !key || !x_dev || !y_dev || n == 0) return SOSO_HIP_ERR_ARG;
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    Weight *w = find_weight(h, key, key_len);
    if (!w) return set_err(h, SOSO_HIP_DECLINED, "matvec_dev: key not resident");
    return launch_matvec(h, *w, x_dev, y_dev, n);
}

int soso_hip_dequant_dev(soso_hip *h, const char *key, size_t key_len, float *out_dev)
{
    if (!h || !key || !out_dev) return SOSO_HIP_ERR_ARG;
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    Weight *w = find_weight(h, key, key_len);
    if (!w) return set_err(h, SOSO_HIP_DECLINED, "dequant_dev: key not resident");
    return launch_dequant(h, *w, out_dev);
}

int soso_hip_argmax_dev(soso_hip *h, const float *x_dev, size_t n, uint32_t *idx_dev)
{
    if (!h || !x_dev || !idx_dev || n == 0) return SOSO_HIP_ERR_ARG;
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    return launch_argmax(h, x_dev, n, idx_dev);
}

int soso_hip_timer_start(soso_hip *h)
{
    if (!h) return SOSO_HIP_ERR_ARG;
    int rc = make_current(h);
    return rc == SOSO_HIP_OK ? hip_check(h, hipEventRecord(h->ev0, h->stream), "event record") : rc;
}

int soso_hip_timer_stop(soso_hip *h, float *ms)
{
    if (!h || !ms) return SOSO_HIP_ERR_ARG;
    int rc = make_current(h);
    if (rc == SOSO_HIP_OK) rc = hip_check(h, hipEventRecord(h->ev1, h->stream), "event record");
    if (rc == SOSO_HIP_OK) rc = hip_check(h, hipEventSynchronize(h->ev1), "event sync");
    if (rc == SOSO_HIP_OK) rc = hip_check(h, hipEventElapsedTime(ms, h->ev0, h->ev1), "event elapsed");
    return rc;
}

int soso_hip_event_record(soso_hip *h, int slot)
{
    if (!h || slot < 0 || slot > 65535) return SOSO_HIP_ERR_ARG;
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    if ((size_t)slot >= h->events.size()) h->events.resize((size_t)slot + 1, nullptr);
    if (!h->events[slot] && hipEventCreate(&h->events[slot]) != hipSuccess) {
        h->events[slot] = nullptr;
        return set_err(h, SOSO_HIP_ERR_DEVICE, "hipEventCreate");
    }
    return hip_check(h, hipEventRecord(h->events[slot], h->stream), "event record");
}

int soso_hip_event_elapsed(soso_hip *h, int a, int b, float *ms)
{
    if (!h || !ms || a < 0 || b < 0 || (size_t)a >= h->events.size() || (size_t)b >= h->events.size() ||
        !h->events[a] || !h->events[b])
        return SOSO_HIP_ERR_ARG;
    int rc = make_current(h);
    if (rc == SOSO_HIP_OK) rc = hip_check(h, hipEventSynchronize(h->events[b]), "event sync");
    if (rc == SOSO_HIP_OK) rc = hip_check(h, hipEventElapsedTime(ms, h->events[a], h->events[b]), "event elapsed");
    return rc;
}

int soso_hip_graph_begin(soso_hip *h)
{
    if (!h || h->capturing) return SOSO_HIP_ERR_ARG;
    int rc = make_current(h);
    if (rc == SOSO_HIP_OK)
        rc = hip_check(h, hipStreamBeginCapture(h->stream, hipStreamCaptureModeThreadLocal), "begin capture");
    if (rc == SOSO_HIP_OK) h->capturing = true;
    return rc;
}

int soso_hip_graph_end(soso_hip *h, int *graph_id)
{
    if (!h || !graph_id || !h->capturing) return SOSO_HIP_ERR_ARG;
    h->capturing = false;
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    hipGraph_t g = nullptr;
    rc = hip_check(h, hipStreamEndCapture(h->stream, &g), "end capture");
    if (rc != SOSO_HIP_OK) return rc;
    hipGraphExec_t ex = nullptr;
    rc = hip_check(h, hipGraphInstantiate(&ex, g, nullptr, nullptr, 0), "graph instantiate");
    // the captured template is not needed once instantiated (nor after a failure)
    (void)hip_release(h, hipGraphDestroy(g), "graph destroy");
    if (rc != SOSO_HIP_OK) return rc;
    h->graphs.push_back(ex);
    *graph_id = (int)h->graphs.size() - 1;
    return SOSO_HIP_OK;
}

int soso_hip_graph_launch(soso_hip *h, int id)
{
    if (!h || id < 0 || (size_t)id >= h->graphs.size() || !h->graphs[id]) return SOSO_HIP_ERR_ARG;
    int rc = make_current(h);
    return rc == SOSO_HIP_OK ? hip_check(h, hipGraphLaunch(h->graphs[id], h->stream), "graph launch") : rc;
}

int soso_hip_graph_destroy(soso_hip *h, int id)
{
    if (!h || id < 0 || (size_t)id >= h->graphs.size() || !h->graphs[id]) return SOSO_HIP_ERR_ARG;
    int rc = make_current(h);
    if (rc != SOSO_HIP_OK) return rc;
    (void)hipStreamSynchronize(h->stream);
    (void)hipGraphExecDestroy(h->graphs[id]);
    h->graphs[id] = nullptr;
    if (!any_graph(h)) free_retired(h); // no graph can hold them any more
    return SOSO_HIP_OK;
}

} // extern "C"
