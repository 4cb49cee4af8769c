// hymt_hip.cpp -- the C ABI of libhymt_hip.so (declared in include/hymt_hip.h).
//
// Owns one HIP device and stream per context, the paged K/V cache of every
// layer, the RoPE table and the kernels' workspaces.  Plays the role of the
// reference backends' device state (VulkanBackend.cs:275-294,
// MetalBackend.cs:160-197) for the attention path only.
#include "../../include/hymt_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "attn_kernels.hpp"
#include "ktimer.hpp"
#include "kv_pages.hpp"
#include "weights.hpp"

using namespace hymt;

namespace {

thread_local std::string g_err;

int fail(int code, const std::string &msg) {
    g_err = msg;
    return code;
}

struct HipError {
    hipError_t e;
    const char *what;
};

#define HIP_TRY(call)                                        \
    do {                                                     \
        hipError_t e_ = (call);                              \
        if (e_ != hipSuccess) throw HipError{e_, #call};     \
    } while (0)

// A device buffer that grows on demand and never shrinks.  A buffer that
// belongs to a context bumps the context's generation when it moves, so that
// recordings holding its old address can be refused (hymt_graph_launch).
struct DevBuf {
    void *p = nullptr;
    size_t bytes = 0;
    uint64_t *gen = nullptr;
    void reserve(size_t n) {
        if (n <= bytes) return;
        if (p) HIP_TRY(hipFree(p));
        p = nullptr;
        bytes = 0;
        if (gen) ++*gen;
        HIP_TRY(hipMalloc(&p, n));
        bytes = n;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
    }
};

// Pinned host staging for calls with host pointers.
struct HostBuf {
    void *p = nullptr;
    size_t bytes = 0;
    void reserve(size_t n) {
        if (n <= bytes) return;
        if (p) HIP_TRY(hipHostFree(p));
        p = nullptr;
        bytes = 0;
        HIP_TRY(hipHostMalloc(&p, n, hipHostMallocDefault));
        bytes = n;
    }
    void release() {
        if (p) (void)hipHostFree(p);
        p = nullptr;
        bytes = 0;
    }
};

size_t dtype_bytes(int dt) { return dt == HYMT_F32 ? 4 : 2; }

}  // namespace

struct hymt_ctx {
    int device = HYMT_DEVICE_NONE;
    hipStream_t stream = nullptr;

    // attention config (ModelConfig)
    bool configured = false;
    int heads = 0, kv_heads = 0, head_dim = 0, rope_dim = 0;
    float rope_base = 10000.f, eps = 1e-6f;

    // paged KV
    bool kv_ready = false;
    int layers = 0, kv_dtype = HYMT_BF16;
    KvPages pages;
    DevBuf kpool, vpool, tab;
    size_t layer_elems = 0;  // elements per layer pool

    // RoPE table rows [0, rope_cap)
    int rope_cap = 0;
    DevBuf rope_cos, rope_sin;
    // 128 ones: the gamma of an absent QK norm and the table row of rope_dim
    // 0, so that the decode kernel's loads never depend on a branch
    DevBuf ones;

    // decode workspace: split partials (m, l) and acc
    DevBuf dec_ml, dec_acc;
    // prefill workspace: split partials; q prepared by prefill_kv for the flash kernel
    DevBuf part_o, part_ml, qready;
    // staging for host-pointer calls
    DevBuf in_q, in_k, in_v, in_qnw, in_knw, out_o, up_k, up_v;
    DevBuf rows_idx;  // token ids of hymt_embed_rows
    HostBuf h_in, h_out;
    // the prefill GEMMs' hipBLASLt state (created on the first GEMM)
    GemmState *gemm = nullptr;
    // per-kernel timing (HYMT_HIP_TIMING at creation, hymt_timing_enable):
    // the timer once created, and whether calls are timed now
    KernelTimer *timer = nullptr;
    bool timing_on = false;

    // stream capture (hymt_graph_begin .. hymt_graph_end)
    bool capturing = false;
    bool capture_failed = false;
    // bumped whenever a buffer above is reallocated: a recording replays the
    // addresses it captured, so it is only valid for the generation it was
    // recorded in
    uint64_t gen = 0;

    hymt_ctx() {
        for (DevBuf *b : {&kpool, &vpool, &tab, &rope_cos, &rope_sin, &ones, &dec_ml, &dec_acc, &part_o, &part_ml,
                          &qready, &in_q, &in_k, &in_v, &in_qnw, &in_knw, &out_o, &up_k, &up_v, &rows_idx})
            b->gen = &gen;
    }

    bool has_device() const { return device >= 0; }
    void *klayer(int l) const { return (char *)kpool.p + (size_t)l * layer_elems * dtype_bytes(kv_dtype); }
    void *vlayer(int l) const { return (char *)vpool.p + (size_t)l * layer_elems * dtype_bytes(kv_dtype); }
};

struct hymt_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    uint64_t gen = 0;  // the context's buffer generation at recording
};

namespace {

int map_hip(const HipError &e) {
    if (e.e == hipErrorOutOfMemory || e.e == hipErrorMemoryAllocation)
        return fail(HYMT_E_OOM, std::string("device allocation failed: ") + e.what);
    return fail(HYMT_E_DEVICE, std::string(e.what) + ": " + hipGetErrorString(e.e));
}

// Mirror changed page-table entries to the device table.
void flush_table(hymt_ctx *c) {
    if (!c->pages.has_dirty()) return;
    std::vector<int> idx = c->pages.take_dirty();
    std::vector<int> val(idx.size());
    for (size_t i = 0; i < idx.size(); i++) val[i] = c->pages.phys(idx[i]);
    HIP_TRY(launch_tab_update((int32_t *)c->tab.p, idx.data(), val.data(), (int)idx.size(), c->stream));
}

// Map [pos, pos+len) for writing: pages for unmapped blocks, fresh pages for
// blocks pinned by the block store, whose leading rows are copied over first
// (MetalBackend.cs ExecCopies, :320-332), then the table mirror.
void map_write(hymt_ctx *c, int pos, int len) {
    c->pages.ensure_written(pos, len);
    const std::vector<KvPages::Copy> copies = c->pages.take_copies();
    if (!c->has_device()) return;
    const size_t page_bytes = (size_t)c->kv_heads * kPage * c->head_dim * dtype_bytes(c->kv_dtype);
    const size_t layer_bytes = c->layer_elems * dtype_bytes(c->kv_dtype);
    for (const KvPages::Copy &x : copies)
        HIP_TRY(launch_kv_copy_page(c->kpool.p, c->vpool.p, layer_bytes, page_bytes, x.src, x.dst,
                                    c->layers, c->stream));
    flush_table(c);
}

// Ops.EnsureRopeTable (Ops.cs:170-195): freq_i = 1 / base^(i/half), angle =
// pos * freq in fp32; rows [0, max(needed, 4096)).  The reference grows its
// table on demand; here it is built once for the cache's capacity when the
// cache is created (a row's values do not depend on the table's size), so
// no attention call ever reallocates it.
void ensure_rope(hymt_ctx *c, int needed) {
    if (needed <= c->rope_cap) return;
    int cap = std::max(needed, 4096);
    if (c->rope_cap > 0) cap = std::max(cap, 2 * c->rope_cap);
    const int half = c->rope_dim / 2;
    if (half == 0) {  // rope_dim 0: nothing rotates, the kernels read no table
        c->rope_cap = cap;
        return;
    }
    std::vector<float> freqs(half), cs((size_t)cap * half), sn((size_t)cap * half);
    for (int i = 0; i < half; i++) freqs[i] = 1.0f / powf(c->rope_base, (float)i / (float)half);
    for (int pos = 0; pos < cap; pos++)
        for (int i = 0; i < half; i++) {
            float angle = (float)pos * freqs[i];
            cs[(size_t)pos * half + i] = cosf(angle);
            sn[(size_t)pos * half + i] = sinf(angle);
        }
    HIP_TRY(hipStreamSynchronize(c->stream));  // kernels may still read the old table
    c->rope_cos.reserve(cs.size() * 4);
    c->rope_sin.reserve(sn.size() * 4);
    HIP_TRY(hipMemcpy(c->rope_cos.p, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(c->rope_sin.p, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
    c->rope_cap = cap;
}

// Copy host tensors into device staging through one pinned buffer.
struct Upload {
    const void *src;
    size_t bytes;
    DevBuf *dst;
};
void stage_in(hymt_ctx *c, std::initializer_list<Upload> ups) {
    size_t total = 0;
    for (auto &u : ups) total += (u.src ? (u.bytes + 255) & ~(size_t)255 : 0);
    HIP_TRY(hipStreamSynchronize(c->stream));  // pinned buffer may still feed a copy
    c->h_in.reserve(total);
    size_t off = 0;
    for (auto &u : ups) {
        if (!u.src) continue;
        u.dst->reserve(u.bytes);
        std::memcpy((char *)c->h_in.p + off, u.src, u.bytes);
        HIP_TRY(hipMemcpyAsync(u.dst->p, (char *)c->h_in.p + off, u.bytes, hipMemcpyHostToDevice, c->stream));
        off += (u.bytes + 255) & ~(size_t)255;
    }
}

void stage_out(hymt_ctx *c, const void *dsrc, void *hdst, size_t bytes) {
    c->h_out.reserve(bytes);
    HIP_TRY(hipMemcpyAsync(c->h_out.p, dsrc, bytes, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    std::memcpy(hdst, c->h_out.p, bytes);
}

// The kernels read q/k/v/gamma rows and write outputs as 16-byte vectors.
bool aligned16(std::initializer_list<const void *> ptrs) {
    for (const void *p : ptrs)
        if (((uintptr_t)p & 15u) != 0) return false;
    return true;
}

int check_ctx(hymt_ctx *c, bool need_kv, bool need_dev) {
    if (!c) return fail(HYMT_E_ARG, "null context");
    if (need_kv && !c->kv_ready) return fail(HYMT_E_STATE, "KV cache not created (hymt_kv_create)");
    if (need_dev && !c->has_device()) return fail(HYMT_E_NO_DEVICE, "context has no device");
    return HYMT_OK;
}

// The timer of a call on `c`: none without timing, and none while recording
// (a recording holds no events of ours, and waiting on one would fail).
KernelTimer *call_timer(const hymt_ctx *c) { return c && c->timing_on && !c->capturing ? c->timer : nullptr; }

// Calls that synchronise or copy host memory cannot be recorded.
int refuse_in_capture(hymt_ctx *c, const char *what) {
    if (!c->capturing) return HYMT_OK;
    c->capture_failed = true;
    return fail(HYMT_E_STATE, std::string(what) + " cannot run while the stream is being recorded");
}

// A device-pointer call being recorded fails if it would have to allocate.
int fail_capture(hymt_ctx *c, const std::string &msg) {
    c->capture_failed = true;
    return fail(HYMT_E_STATE, msg + " during recording; run the call once before hymt_graph_begin");
}

}  // namespace

extern "C" {

const char *hymt_last_error(void) { return g_err.c_str(); }

int hymt_abi_version(void) { return HYMT_ABI_VERSION; }

int hymt_device_count(int *count) {
    if (!count) return fail(HYMT_E_ARG, "null count");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    *count = (e == hipSuccess) ? n : 0;
    return HYMT_OK;
}

int hymt_create(int device, hymt_ctx **out) {
    if (!out) return fail(HYMT_E_ARG, "null out");
    *out = nullptr;
    hymt_ctx *c = new (std::nothrow) hymt_ctx();
    if (!c) return fail(HYMT_E_OOM, "host allocation failed");
    if (device == HYMT_DEVICE_NONE) {
        *out = c;
        return HYMT_OK;
    }
    int n = 0;
    if (device < 0 || hipGetDeviceCount(&n) != hipSuccess || device >= n) {
        delete c;
        return fail(HYMT_E_NO_DEVICE, "HIP device " + std::to_string(device) + " not available (" +
                                          std::to_string(n) + " devices)");
    }
    try {
        HIP_TRY(hipSetDevice(device));
        hipDeviceProp_t prop;
        HIP_TRY(hipGetDeviceProperties(&prop, device));
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
            delete c;
            return fail(HYMT_E_NO_DEVICE, std::string("built for gfx950, device is ") + prop.gcnArchName);
        }
        HIP_TRY(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
        c->device = device;
        // the no-allocation decode's static workspace: its address on this
        // device, resolved once per device while the device is current
        HIP_TRY(decode_scratch_init(device));
        c->timer = timer_from_env();
        c->timing_on = c->timer != nullptr;
    } catch (const HipError &e) {
        delete c;
        return map_hip(e);
    }
    *out = c;
    return HYMT_OK;
}

int hymt_destroy(hymt_ctx *c) {
    if (!c) return HYMT_OK;
    if (c->has_device()) {
        (void)hipSetDevice(c->device);
        if (c->capturing) {
            hipGraph_t g = nullptr;
            (void)hipStreamEndCapture(c->stream, &g);
            if (g) (void)hipGraphDestroy(g);
            c->capturing = false;
        }
        (void)hipStreamSynchronize(c->stream);
        for (DevBuf *b : {&c->kpool, &c->vpool, &c->tab, &c->rope_cos, &c->rope_sin, &c->ones, &c->dec_ml,
                          &c->dec_acc, &c->part_o, &c->part_ml, &c->qready, &c->in_q,
                          &c->in_k, &c->in_v, &c->in_qnw, &c->in_knw, &c->out_o, &c->up_k, &c->up_v, &c->rows_idx})
            b->release();
        c->h_in.release();
        c->h_out.release();
        gemm_state_destroy(c->gemm);
        c->gemm = nullptr;
        timer_destroy(c->timer);
        c->timer = nullptr;
        (void)hipStreamDestroy(c->stream);
        decode_scratch_release(c->device, c);  // its work has drained (synchronised above)
    }
    delete c;
    return HYMT_OK;
}

int hymt_set_attn_config(hymt_ctx *c, int heads, int kv_heads, int head_dim, int rope_dim,
                         float rope_base, float eps) {
    if (int r = check_ctx(c, false, false)) return r;
    if (c->kv_ready) return fail(HYMT_E_STATE, "config must precede hymt_kv_create");
    if (heads <= 0 || kv_heads <= 0 || heads % kv_heads || head_dim <= 0 || rope_dim < 0 ||
        rope_dim > head_dim || (rope_dim & 1) || !(rope_base > 0.f) || !(eps >= 0.f))
        return fail(HYMT_E_ARG, "invalid attention config");
    if (head_dim != kHeadDim || heads / kv_heads != kGroup || 8 % kv_heads)
        return fail(HYMT_E_UNSUPPORTED, "built for head_dim 128, 4 q heads per kv head, kv_heads dividing 8");
    c->heads = heads;
    c->kv_heads = kv_heads;
    c->head_dim = head_dim;
    c->rope_dim = rope_dim;
    c->rope_base = rope_base;
    c->eps = eps;
    c->configured = true;
    return HYMT_OK;
}

int hymt_kv_create(hymt_ctx *c, int layers, int max_tokens, int kv_dtype) {
    if (int r = check_ctx(c, false, false)) return r;
    if (!c->configured) return fail(HYMT_E_STATE, "hymt_set_attn_config first");
    if (c->kv_ready) return fail(HYMT_E_STATE, "KV cache already created");
    if (int r = refuse_in_capture(c, "hymt_kv_create")) return r;
    if (layers <= 0 || max_tokens <= 0 || kv_dtype < HYMT_F32 || kv_dtype > HYMT_BF16)
        return fail(HYMT_E_ARG, "invalid KV cache arguments");
    c->layers = layers;
    c->kv_dtype = kv_dtype;
    c->pages = KvPages(max_tokens);
    const int P = c->pages.max_pages();
    c->layer_elems = (size_t)P * c->kv_heads * kPage * c->head_dim;
    if (c->has_device()) {
        try {
            HIP_TRY(hipSetDevice(c->device));
            const size_t bytes = (size_t)layers * c->layer_elems * dtype_bytes(kv_dtype);
            c->kpool.reserve(bytes);
            c->vpool.reserve(bytes);
            c->tab.reserve((size_t)P * 4);
            HIP_TRY(hipMemset(c->tab.p, 0xFF, (size_t)P * 4));
            c->dec_ml.reserve((size_t)c->heads * kMaxSplits * 2 * 4);
            c->dec_acc.reserve((size_t)c->heads * kMaxSplits * kHeadDim * 4);
            ensure_rope(c, c->pages.max_tokens());
            const std::vector<float> ones(kHeadDim, 1.0f);
            c->ones.reserve(kHeadDim * 4);
            HIP_TRY(hipMemcpy(c->ones.p, ones.data(), kHeadDim * 4, hipMemcpyHostToDevice));
        } catch (const HipError &e) {
            c->kpool.release();
            c->vpool.release();
            return map_hip(e);
        }
    }
    c->kv_ready = true;
    return HYMT_OK;
}

int hymt_kv_info(hymt_ctx *c, int *max_tokens, int *pages_total, int *pages_mapped) {
    if (int r = check_ctx(c, true, false)) return r;
    if (max_tokens) *max_tokens = c->pages.max_tokens();
    if (pages_total) *pages_total = c->pages.max_pages();
    if (pages_mapped) *pages_mapped = c->pages.mapped();
    return HYMT_OK;
}

int hymt_kv_map(hymt_ctx *c, int pos, int len) {
    if (int r = check_ctx(c, true, false)) return r;
    if (pos < 0 || len < 0) return fail(HYMT_E_ARG, "invalid range");
    if (c->capturing && c->pages.needs_copy(pos, len)) return fail_capture(c, "a write into a harvested block");
    try {
        if (c->has_device()) HIP_TRY(hipSetDevice(c->device));
        map_write(c, pos, len);
    } catch (const CapacityError &e) {
        return fail(HYMT_E_CAPACITY, e.what());
    } catch (const HipError &e) {
        return map_hip(e);
    }
    return HYMT_OK;
}

int hymt_kv_page(hymt_ctx *c, int block, int *phys) {
    if (int r = check_ctx(c, true, false)) return r;
    if (!phys || block < 0 || block >= c->pages.max_pages()) return fail(HYMT_E_ARG, "invalid block");
    *phys = c->pages.phys(block);
    return HYMT_OK;
}

int hymt_kv_set_len(hymt_ctx *c, int len) {
    if (int r = check_ctx(c, true, false)) return r;
    if (len < 0) return fail(HYMT_E_ARG, "negative cache length");
    c->pages.set_len(len);
    return HYMT_OK;
}

int hymt_kv_harvest(hymt_ctx *c, const int32_t *tokens, int n_tokens, int block_tokens) {
    if (int r = check_ctx(c, true, false)) return r;
    if (n_tokens < 0 || (n_tokens > 0 && !tokens)) return fail(HYMT_E_ARG, "invalid token list");
    if (int r = refuse_in_capture(c, "hymt_kv_harvest")) return r;
    try {
        c->pages.harvest(tokens, n_tokens, block_tokens);
    } catch (const BlockSizeError &e) {
        return fail(HYMT_E_UNSUPPORTED, e.what());
    }
    return HYMT_OK;
}

int hymt_kv_restore(hymt_ctx *c, const int32_t *tokens, int n_tokens, int block_tokens,
                    int *restored_tokens) {
    if (int r = check_ctx(c, true, false)) return r;
    if (!restored_tokens || n_tokens < 0 || (n_tokens > 0 && !tokens))
        return fail(HYMT_E_ARG, "invalid token list");
    if (int r = refuse_in_capture(c, "hymt_kv_restore")) return r;
    try {
        *restored_tokens = c->pages.restore(tokens, n_tokens, block_tokens);
        if (c->has_device()) {
            HIP_TRY(hipSetDevice(c->device));
            flush_table(c);
        }
    } catch (const BlockSizeError &e) {
        return fail(HYMT_E_UNSUPPORTED, e.what());
    } catch (const HipError &e) {
        return map_hip(e);
    }
    return HYMT_OK;
}

int hymt_kv_store_info(hymt_ctx *c, int *entries, int *pages_free) {
    if (int r = check_ctx(c, true, false)) return r;
    if (entries) *entries = c->pages.store_entries();
    if (pages_free) *pages_free = c->pages.pages_free();
    return HYMT_OK;
}

int hymt_kv_upload(hymt_ctx *c, int layer, int pos, int len, const uint16_t *k_bf16,
                   const uint16_t *v_bf16) {
    if (int r = check_ctx(c, true, false)) return r;
    if (layer < 0 || layer >= c->layers || pos < 0 || len < 0 || (len > 0 && (!k_bf16 || !v_bf16)))
        return fail(HYMT_E_ARG, "invalid upload arguments");
    if ((long)pos + len > c->pages.max_tokens())
        return fail(HYMT_E_CAPACITY, "KV capacity " + std::to_string(c->pages.max_tokens()) +
                                         " exceeded at " + std::to_string((long)pos + len));
    if (len == 0) return HYMT_OK;
    if (!c->has_device()) return fail(HYMT_E_NO_DEVICE, "context has no device");
    if (int r = refuse_in_capture(c, "hymt_kv_upload")) return r;
    try {
        HIP_TRY(hipSetDevice(c->device));
        map_write(c, pos, len);
        const size_t stride = (size_t)c->kv_heads * c->head_dim;
        const size_t bytes = (size_t)len * stride * 2;
        stage_in(c, {{k_bf16 + (size_t)pos * stride, bytes, &c->up_k},
                     {v_bf16 + (size_t)pos * stride, bytes, &c->up_v}});
        HIP_TRY(launch_kv_upload(c->kv_dtype, (const uint16_t *)c->up_k.p, (const uint16_t *)c->up_v.p,
                                 (const int32_t *)c->tab.p, c->klayer(layer), c->vlayer(layer), pos,
                                 len, c->kv_heads, c->stream));
        HIP_TRY(hipStreamSynchronize(c->stream));
    } catch (const HipError &e) {
        return map_hip(e);
    } catch (const CapacityError &e) {
        return fail(HYMT_E_CAPACITY, e.what());
    }
    return HYMT_OK;
}

int hymt_kv_read(hymt_ctx *c, int layer, int pos, int len, float *k_out, float *v_out) {
    if (int r = check_ctx(c, true, true)) return r;
    if (layer < 0 || layer >= c->layers || pos < 0 || len < 0 || (len > 0 && (!k_out || !v_out)))
        return fail(HYMT_E_ARG, "invalid read arguments");
    if (!c->pages.resident(pos + len)) return fail(HYMT_E_STATE, "rows not resident");
    if (len == 0) return HYMT_OK;
    if (int r = refuse_in_capture(c, "hymt_kv_read")) return r;
    try {
        HIP_TRY(hipSetDevice(c->device));
        const size_t n = (size_t)len * c->kv_heads * c->head_dim;
        c->out_o.reserve(2 * n * 4);
        float *dk = (float *)c->out_o.p, *dv = dk + n;
        HIP_TRY(launch_kv_read(c->kv_dtype, (const int32_t *)c->tab.p, c->klayer(layer), c->vlayer(layer),
                               dk, dv, pos, len, c->kv_heads, c->stream));
        stage_out(c, dk, k_out, n * 4);
        stage_out(c, dv, v_out, n * 4);
    } catch (const HipError &e) {
        return map_hip(e);
    }
    return HYMT_OK;
}

// scratch_ml / scratch_acc: the split partials of a no-allocation call (the
// static device workspace), or null for the context's own buffers
static int decode_impl(hymt_ctx *c, int layer, int pos, const float *q, const float *k, const float *v,
                       const float *qnw, const float *knw, float *out, unsigned flags, float *scratch_ml,
                       float *scratch_acc) {
    if (int r = check_ctx(c, true, false)) return r;
    if (layer < 0 || layer >= c->layers || pos < 0 || !q || !k || !v || !out)
        return fail(HYMT_E_ARG, "invalid decode arguments");
    if (pos >= c->pages.max_tokens())
        return fail(HYMT_E_CAPACITY, "KV capacity " + std::to_string(c->pages.max_tokens()) +
                                         " exceeded at " + std::to_string(pos + 1));
    if (!c->pages.resident(pos)) return fail(HYMT_E_STATE, "device KV must hold [0, pos) before decode");
    const bool dev = flags & HYMT_FLAG_DEVICE_PTRS;
    if (dev && !aligned16({q, k, v, qnw, knw, out}))
        return fail(HYMT_E_ARG, "device tensors must be 16-byte aligned");
    if (!c->has_device()) return fail(HYMT_E_NO_DEVICE, "context has no device");
    if (!dev)
        if (int r = refuse_in_capture(c, "a host-pointer decode")) return r;
    if (c->capturing && c->pages.needs_copy(pos, 1)) return fail_capture(c, "a write into a harvested block");
    try {
        HIP_TRY(hipSetDevice(c->device));
        map_write(c, pos, 1);  // the RoPE table already covers the capacity
        const size_t D = c->head_dim, qn = (size_t)c->heads * D, kn = (size_t)c->kv_heads * D;
        if (!dev) {
            stage_in(c, {{q, qn * 4, &c->in_q}, {k, kn * 4, &c->in_k}, {v, kn * 4, &c->in_v},
                         {qnw, D * 4, &c->in_qnw}, {knw, D * 4, &c->in_knw}});
            c->out_o.reserve(qn * 4);
        }
        DecodeArgs a;
        const float *ones = (const float *)c->ones.p;
        a.q = dev ? q : (const float *)c->in_q.p;
        a.knew = dev ? k : (const float *)c->in_k.p;
        a.vnew = dev ? v : (const float *)c->in_v.p;
        a.qnw = !qnw ? ones : dev ? qnw : (const float *)c->in_qnw.p;
        a.knw = !knw ? ones : dev ? knw : (const float *)c->in_knw.p;
        a.norm_q = qnw != nullptr;
        a.norm_k = knw != nullptr;
        const int half = c->rope_dim / 2;
        a.rope_cos = half ? (const float *)c->rope_cos.p + (size_t)pos * half : ones;
        a.rope_sin = half ? (const float *)c->rope_sin.p + (size_t)pos * half : ones;
        a.tab = (const int32_t *)c->tab.p;
        a.kpool = c->klayer(layer);
        a.vpool = c->vlayer(layer);
        a.part_ml = scratch_ml ? scratch_ml : (float *)c->dec_ml.p;
        a.part_acc = scratch_acc ? scratch_acc : (float *)c->dec_acc.p;
        a.out = dev ? out : (float *)c->out_o.p;
        a.L = pos + 1;
        a.kv_heads = c->kv_heads;
        a.rope_half = half;
        a.rope_dim = c->rope_dim;
        const int npages = (a.L + kPage - 1) / kPage;
        a.ppw = a.nsplit = 0;  // the work split is chosen by launch_decode
        a.eps = c->eps;
        a.qscale = 1.4426950408889634f / sqrtf((float)D);
        a.pages_in_args = npages <= kArgPages;
        if (a.pages_in_args) {
            // padded with the last page: the kernel clamps look-ahead page
            // indices to the list's end, not to L
            for (int b = 0; b < npages; b++) a.pages[b] = c->pages.phys(b);
            for (int b = npages; b < kArgPages; b++) a.pages[b] = a.pages[npages - 1];
        }
        HIP_TRY(launch_decode(c->kv_dtype, a, c->stream));
        if (!dev) stage_out(c, c->out_o.p, out, qn * 4);
    } catch (const HipError &e) {
        return map_hip(e);
    } catch (const CapacityError &e) {
        return fail(HYMT_E_CAPACITY, e.what());
    }
    return HYMT_OK;
}

int hymt_attn_decode(hymt_ctx *c, int layer, int pos, const float *q, const float *k, const float *v,
                     const float *qnw, const float *knw, float *out, unsigned flags) {
    TimedCall timed(call_timer(c), "attn_decode", pos);
    return decode_impl(c, layer, pos, q, k, v, qnw, knw, out, flags, nullptr, nullptr);
}

int hymt_attn_decode_noalloc(hymt_ctx *c, int layer, int pos, const float *q, const float *k, const float *v,
                             const float *qnw, const float *knw, float *out) {
    if (int r = check_ctx(c, true, false)) return r;
    if (!c->has_device()) return fail(HYMT_E_NO_DEVICE, "context has no device");
    float *ml = nullptr, *acc = nullptr;
    int max_heads = 0;
    const hipError_t e = decode_scratch(c->device, &ml, &acc, &max_heads);
    if (e != hipSuccess)
        return fail(HYMT_E_DEVICE, std::string("decode workspace not resolved on this device: ") + hipGetErrorString(e));
    if (c->heads > max_heads)
        return fail(HYMT_E_UNSUPPORTED, "the static decode workspace holds " + std::to_string(max_heads) +
                                            " q heads; the context has " + std::to_string(c->heads));
    if (!decode_scratch_claim(c->device, c))
        return fail(HYMT_E_STATE, "the static decode workspace of device " + std::to_string(c->device) +
                                      " is held by another live context (destroy it first)");
    TimedCall timed(call_timer(c), "attn_decode_noalloc", pos);
    return decode_impl(c, layer, pos, q, k, v, qnw, knw, out, HYMT_FLAG_DEVICE_PTRS, ml, acc);
}

// q_ld / kv_ld: elements from one q (k, v) row to the next; 0 = packed rows
// out_bf16 (the model's prefill): out receives bf16 bits, the o-projection
// GEMM's input, rounded as hymt_to_bf16 rounds the fp32 output
static int prefill_impl(hymt_ctx *c, int layer, int pos, int seq, const void *q, int q_ld, const void *k,
                        const void *v, int kv_ld, int io_dtype, const float *qnw, const float *knw, float *out,
                        unsigned flags, bool out_bf16 = false) {
    if (int r = check_ctx(c, true, false)) return r;
    if (layer < 0 || layer >= c->layers || pos < 0 || seq <= 0 || !q || !k || !v || !out ||
        (io_dtype != HYMT_F32 && io_dtype != HYMT_BF16))
        return fail(HYMT_E_ARG, "invalid prefill arguments");
    if (c->kv_dtype == HYMT_F32)
        return fail(HYMT_E_UNSUPPORTED, "prefill runs on bf16/f16 MFMA; f32 KV cache has no prefill path");
    if (c->rope_dim % 64)
        return fail(HYMT_E_UNSUPPORTED, "prefill built for rope_dim 0, 64 or 128");
    if ((long)pos + seq > c->pages.max_tokens())
        return fail(HYMT_E_CAPACITY, "KV capacity " + std::to_string(c->pages.max_tokens()) +
                                         " exceeded at " + std::to_string((long)pos + seq));
    if (!c->pages.resident(pos)) return fail(HYMT_E_STATE, "device KV must hold [0, pos) before prefill");
    const bool dev = flags & HYMT_FLAG_DEVICE_PTRS;
    // the kernels read q, k, v and the norm vectors and write out as 16-byte
    // vectors (rows q_ld / kv_ld elements apart stay aligned: multiples of 8)
    if (dev && !aligned16({q, k, v, qnw, knw, out}))
        return fail(HYMT_E_ARG, "device tensors must be 16-byte aligned");
    if (!c->has_device()) return fail(HYMT_E_NO_DEVICE, "context has no device");
    if (!dev)
        if (int r = refuse_in_capture(c, "a host-pointer prefill")) return r;
    if (out_bf16 && !dev) return fail(HYMT_E_ARG, "bf16 output needs device pointers");
    if (c->capturing && c->pages.needs_copy(pos, seq)) return fail_capture(c, "a write into a harvested block");
    try {
        HIP_TRY(hipSetDevice(c->device));
        map_write(c, pos, seq);  // the RoPE table already covers the capacity
        const size_t D = c->head_dim, es = dtype_bytes(io_dtype);
        const size_t qn = (size_t)seq * c->heads * D, kn = (size_t)seq * c->kv_heads * D;
        if (!dev) {
            stage_in(c, {{q, qn * es, &c->in_q}, {k, kn * es, &c->in_k}, {v, kn * es, &c->in_v},
                         {qnw, D * 4, &c->in_qnw}, {knw, D * 4, &c->in_knw}});
            c->out_o.reserve(qn * 4);
        }
        PrepArgs p;
        p.k = dev ? k : c->in_k.p;
        p.v = dev ? v : c->in_v.p;
        p.knw = !knw ? (const float *)c->ones.p : dev ? knw : (const float *)c->in_knw.p;
        p.norm_k = knw != nullptr;
        p.rope_cos = (const float *)c->rope_cos.p;
        p.rope_sin = (const float *)c->rope_sin.p;
        p.tab = (const int32_t *)c->tab.p;
        p.kpool = c->klayer(layer);
        p.vpool = c->vlayer(layer);
        p.pos0 = pos;
        p.seq = seq;
        p.kv_heads = c->kv_heads;
        p.rope_half = c->rope_dim / 2;
        p.rope_dim = c->rope_dim;
        p.io_bf16 = io_dtype == HYMT_BF16;
        p.eps = c->eps;
        p.kv_ld = kv_ld ? kv_ld : c->kv_heads * (int)D;
        p.q = dev ? q : c->in_q.p;
        p.qnw = !qnw ? (const float *)c->ones.p : dev ? qnw : (const float *)c->in_qnw.p;
        p.norm_q = qnw != nullptr;
        p.q_ld = q_ld ? q_ld : c->heads * (int)D;
        p.heads = c->heads;
        p.qscale = 1.4426950408889634f / sqrtf((float)D);
        p.qready = nullptr;

        FlashArgs f{};
        f.q = p.q;
        f.qnw = p.qnw;
        f.qready = nullptr;
        f.norm_q = qnw != nullptr;
        f.rope_cos = (const float *)c->rope_cos.p;
        f.rope_sin = (const float *)c->rope_sin.p;
        f.tab = (const int32_t *)c->tab.p;
        f.kpool = c->klayer(layer);
        f.vpool = c->vlayer(layer);
        f.out = dev ? out : (float *)c->out_o.p;
        f.pos0 = pos;
        f.seq = seq;
        f.heads = c->heads;
        f.kv_heads = c->kv_heads;
        f.rope_half = c->rope_dim / 2;
        f.rope_dim = c->rope_dim;
        f.io_bf16 = io_dtype == HYMT_BF16;
        f.eps = c->eps;
        f.qscale = p.qscale;
        f.q_ld = p.q_ld;
        f.out_bf16 = out_bf16;
        f.nb16 = (seq + 15) / 16;
        f.npairs = (f.nb16 + 1) / 2;
        const int npages = (pos + seq + kPage - 1) / kPage;
        f.pages_in_args = npages <= kArgPages;
        if (f.pages_in_args) {
            for (int b = 0; b < npages; b++) f.pages[b] = c->pages.phys(b);
            for (int b = npages; b < kArgPages; b++) f.pages[b] = f.pages[npages - 1];
        }
        // Work items: split the kv range of block pairs only when the (kv
        // head, pair) combinations fill less than half the GPU.  From half
        // up, the merge launch and its partials cost more than the idle CUs
        // (1531 rows, 192 pairs: 38.5 + 20.0 us split against 25 us whole).
        int max_tiles = 0;
        for (int pr = 0; pr < f.npairs; pr++) max_tiles = std::max(max_tiles, pair_tiles(pos, pr, f.nb16, seq));
        int cap = max_tiles;
        const int pairs = f.npairs * c->kv_heads;
        if (pairs < 128) {
            const int per = (256 + pairs - 1) / pairs;
            cap = std::max(4, (max_tiles + per - 1) / per);
        }
        cap = std::min(cap, kItemTiles);
        f.cap = cap;
        int items = 0, ns0 = -1;
        bool split = false, uniform = true;
        for (int pr = 0; pr < f.npairs; pr++) {
            const int ns = (pair_tiles(pos, pr, f.nb16, seq) + cap - 1) / cap;
            items += ns;
            split |= ns > 1;
            uniform &= ns0 < 0 || ns == ns0;
            ns0 = ns;
        }
        f.split_ns = split && uniform ? ns0 : 0;
        f.items_per_kvh = items;
        if (split) {
            const size_t slots = (size_t)c->kv_heads * items;
            // partial O / l in the 16-bit cache type, (m, l) in fp32; the q
            // rows prepared once by prefill_kv for the pair's split items
            // (each item would otherwise repeat the q prologue: config 4's
            // call 36.8 -> 33.2 us; unsplit, the 16 MB of q traffic cost what
            // the shorter flash prologue saves)
            if (c->capturing &&
                (slots * kGroup * 32 * D * 2 > c->part_o.bytes || slots * kGroup * 32 * 2 * 4 > c->part_ml.bytes ||
                 qn * 2 > c->qready.bytes))
                return fail_capture(c, "prefill workspace growth");
            c->part_o.reserve(slots * kGroup * 32 * D * 2);
            c->part_ml.reserve(slots * kGroup * 32 * 2 * 4);
            c->qready.reserve(qn * 2);
            p.qready = c->qready.p;
            f.qready = (const uint16_t *)c->qready.p;
        }
        f.part_o = c->part_o.p;
        f.part_ml = (float *)c->part_ml.p;
        HIP_TRY(launch_prefill_prep(c->kv_dtype, p, c->stream));
        HIP_TRY(launch_prefill_flash(c->kv_dtype, f, items * c->kv_heads, c->stream));
        if (split) HIP_TRY(launch_prefill_merge(c->kv_dtype, f, c->stream));
        if (!dev) stage_out(c, c->out_o.p, out, qn * 4);
    } catch (const HipError &e) {
        return map_hip(e);
    } catch (const CapacityError &e) {
        return fail(HYMT_E_CAPACITY, e.what());
    }
    return HYMT_OK;
}

int hymt_attn_prefill(hymt_ctx *c, int layer, int pos, int seq, const void *q, const void *k,
                      const void *v, int io_dtype, const float *qnw, const float *knw, float *out,
                      unsigned flags) {
    TimedCall timed(call_timer(c), "attn_prefill", seq);
    return prefill_impl(c, layer, pos, seq, q, 0, k, v, 0, io_dtype, qnw, knw, out, flags);
}

int hymt_attn_prefill_ld(hymt_ctx *c, int layer, int pos, int seq, const void *q, int q_ld, const void *k,
                         const void *v, int kv_ld, int io_dtype, const float *qnw, const float *knw,
                         float *out, unsigned flags) {
    if (int r = check_ctx(c, true, false)) return r;
    if (!(flags & HYMT_FLAG_DEVICE_PTRS))
        return fail(HYMT_E_ARG, "hymt_attn_prefill_ld takes device pointers (HYMT_FLAG_DEVICE_PTRS)");
    if (q_ld < c->heads * c->head_dim || kv_ld < c->kv_heads * c->head_dim || q_ld % 8 || kv_ld % 8)
        return fail(HYMT_E_ARG, "row strides must cover a row and be multiples of 8 elements");
    TimedCall timed(call_timer(c), "attn_prefill_ld", seq);
    return prefill_impl(c, layer, pos, seq, q, q_ld, k, v, kv_ld, io_dtype, qnw, knw, out, flags);
}

int hymt_sync(hymt_ctx *c) {
    if (int r = check_ctx(c, false, true)) return r;
    if (int r = refuse_in_capture(c, "hymt_sync")) return r;
    hipError_t e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) return fail(HYMT_E_DEVICE, std::string("hipStreamSynchronize: ") + hipGetErrorString(e));
    return HYMT_OK;
}

int hymt_timing_enable(hymt_ctx *c, int mode) {
    if (int r = check_ctx(c, false, true)) return r;
    if (mode < 0 || mode > 2) return fail(HYMT_E_ARG, "timing mode is 0 (off), 1 (print) or 2 (quiet)");
    if (mode == 0) {
        c->timing_on = false;
        return HYMT_OK;
    }
    if (!c->timer) c->timer = timer_create(mode == 1);
    if (!c->timer) return fail(HYMT_E_OOM, "timer allocation failed");
    timer_set_print(c->timer, mode == 1);
    c->timing_on = true;
    return HYMT_OK;
}

int hymt_timing_get(hymt_ctx *c, const char *kernel, long *count, double *us) {
    if (int r = check_ctx(c, false, false)) return r;
    if (!kernel || !count || !us) return fail(HYMT_E_ARG, "null argument");
    if (!c->timer) return fail(HYMT_E_STATE, "timing is off (HYMT_HIP_TIMING=1 or quiet at creation)");
    if (!timer_totals(c->timer, kernel, count, us))
        return fail(HYMT_E_ARG, std::string("no kernel named ") + kernel + " was timed");
    return HYMT_OK;
}

int hymt_timing_reset(hymt_ctx *c) {
    if (int r = check_ctx(c, false, false)) return r;
    if (!c->timer) return fail(HYMT_E_STATE, "timing is off (HYMT_HIP_TIMING=1 or quiet at creation)");
    timer_reset(c->timer);
    return HYMT_OK;
}

int hymt_get_stream(hymt_ctx *c, void **stream) {
    if (int r = check_ctx(c, false, true)) return r;
    if (!stream) return fail(HYMT_E_ARG, "null stream out");
    *stream = (void *)c->stream;
    return HYMT_OK;
}

int hymt_dev_alloc(hymt_ctx *c, size_t bytes, void **dptr) {
    if (int r = check_ctx(c, false, true)) return r;
    if (!dptr || bytes == 0) return fail(HYMT_E_ARG, "invalid allocation request");
    if (int r = refuse_in_capture(c, "hymt_dev_alloc")) return r;
    (void)hipSetDevice(c->device);
    hipError_t e = hipMalloc(dptr, bytes);
    if (e != hipSuccess) return fail(HYMT_E_OOM, std::string("hipMalloc: ") + hipGetErrorString(e));
    return HYMT_OK;
}

int hymt_dev_free(hymt_ctx *c, void *dptr) {
    if (int r = check_ctx(c, false, true)) return r;
    if (!dptr) return HYMT_OK;
    if (int r = refuse_in_capture(c, "hymt_dev_free")) return r;
    (void)hipStreamSynchronize(c->stream);
    hipError_t e = hipFree(dptr);
    if (e != hipSuccess) return fail(HYMT_E_DEVICE, std::string("hipFree: ") + hipGetErrorString(e));
    return HYMT_OK;
}

int hymt_memcpy(hymt_ctx *c, void *dst, const void *src, size_t bytes, int kind) {
    if (int r = check_ctx(c, false, true)) return r;
    if (!dst || !src || kind < 0 || kind > 2) return fail(HYMT_E_ARG, "invalid copy arguments");
    if (bytes == 0) return HYMT_OK;
    if (int r = refuse_in_capture(c, "hymt_memcpy")) return r;
    const hipMemcpyKind k = kind == 0 ? hipMemcpyHostToDevice
                            : kind == 1 ? hipMemcpyDeviceToHost
                                        : hipMemcpyDeviceToDevice;
    hipError_t e = hipMemcpyAsync(dst, src, bytes, k, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) return fail(HYMT_E_DEVICE, std::string("hipMemcpy: ") + hipGetErrorString(e));
    return HYMT_OK;
}

int hymt_graph_begin(hymt_ctx *c) {
    if (int r = check_ctx(c, false, true)) return r;
    if (c->capturing) return fail(HYMT_E_STATE, "a recording is already open");
    (void)hipSetDevice(c->device);
    // this thread's stream-unsafe HIP calls fail instead of joining the graph
    hipError_t e = hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return fail(HYMT_E_DEVICE, std::string("hipStreamBeginCapture: ") + hipGetErrorString(e));
    c->capturing = true;
    c->capture_failed = false;
    return HYMT_OK;
}

int hymt_graph_end(hymt_ctx *c, hymt_graph **out) {
    if (int r = check_ctx(c, false, true)) return r;
    if (!out) return fail(HYMT_E_ARG, "null graph out");
    *out = nullptr;
    if (!c->capturing) return fail(HYMT_E_STATE, "no recording is open");
    (void)hipSetDevice(c->device);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(c->stream, &g);
    c->capturing = false;
    if (c->capture_failed || e != hipSuccess || !g) {
        if (g) (void)hipGraphDestroy(g);
        if (e != hipSuccess)
            return fail(HYMT_E_DEVICE, std::string("hipStreamEndCapture: ") + hipGetErrorString(e));
        return fail(HYMT_E_STATE, "a call failed during recording; the recording is discarded");
    }
    hymt_graph *hg = new (std::nothrow) hymt_graph();
    if (!hg) {
        (void)hipGraphDestroy(g);
        return fail(HYMT_E_OOM, "host allocation failed");
    }
    hg->graph = g;
    hg->gen = c->gen;
    e = hipGraphInstantiate(&hg->exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        delete hg;
        return fail(HYMT_E_DEVICE, std::string("hipGraphInstantiate: ") + hipGetErrorString(e));
    }
    *out = hg;
    return HYMT_OK;
}

int hymt_graph_launch(hymt_ctx *c, hymt_graph *g) {
    if (int r = check_ctx(c, false, true)) return r;
    if (!g || !g->exec) return fail(HYMT_E_ARG, "null graph");
    if (c->capturing) return fail(HYMT_E_STATE, "cannot replay while recording");
    if (g->gen != c->gen)
        return fail(HYMT_E_STATE, "the recording holds addresses of context buffers that have since been "
                                  "reallocated (RoPE table or workspace growth); record it again");
    (void)hipSetDevice(c->device);
    TimedCall timed(call_timer(c), "graph_launch", 0);
    KernelSpan span("graph", c->stream);
    hipError_t e = hipGraphLaunch(g->exec, c->stream);
    if (e != hipSuccess) return fail(HYMT_E_DEVICE, std::string("hipGraphLaunch: ") + hipGetErrorString(e));
    return HYMT_OK;
}

int hymt_graph_destroy(hymt_ctx *c, hymt_graph *g) {
    if (int r = check_ctx(c, false, true)) return r;
    if (!g) return HYMT_OK;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);  // a replay may still be running
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
    return HYMT_OK;
}

}  // extern "C"

// ---- quantized weights ------------------------------------------------------

namespace {
// The GEMV and row kernels read activations and norm weights as float4.
bool misaligned16(const void *p) { return p && ((uintptr_t)p & 15u) != 0; }
}  // namespace

struct hymt_weight {
    hymt::WeightDev dev;
    void *mem = nullptr;
    size_t bytes = 0;
    uint16_t *dense = nullptr;  // bf16 [rows][cols] copy for the prefill GEMMs (hymt_weight_dense)
};

int hymt_weight_upload(hymt_ctx *c, int type, int rows, int cols, const void *data, size_t bytes,
                       hymt_weight **out) {
    if (int r = check_ctx(c, false, true)) return r;
    if (!out || !data) return fail(HYMT_E_ARG, "null weight data or out pointer");
    *out = nullptr;
    if (int r = refuse_in_capture(c, "hymt_weight_upload")) return r;
    const long rb = hymt::gguf_row_bytes(type, cols);
    if (rb < 0) return fail(HYMT_E_UNSUPPORTED, "weight type " + std::to_string(type) + " is not supported");
    if (rows < 1 || cols < 2048 || cols > 8192 || cols % 2048 != 0)
        return fail(HYMT_E_UNSUPPORTED, "weight shape " + std::to_string(rows) + " x " + std::to_string(cols) +
                                            ": cols must be a multiple of 2048 up to 8192");
    if (bytes != (size_t)rows * (size_t)rb)
        return fail(HYMT_E_ARG, "weight data is " + std::to_string(bytes) + " bytes, expected " +
                                    std::to_string((size_t)rows * (size_t)rb));
    hymt::PackedWeight pk;
    if (!hymt::pack_weight(type, rows, cols, (const uint8_t *)data, pk))
        return fail(HYMT_E_UNSUPPORTED, "weight type " + std::to_string(type) + " is not supported");
    hymt_weight *w = new (std::nothrow) hymt_weight();
    if (!w) return fail(HYMT_E_OOM, "host allocation failed");
    (void)hipSetDevice(c->device);
    hipError_t e = hipMalloc(&w->mem, pk.buf.size());
    if (e != hipSuccess) {
        delete w;
        return fail(HYMT_E_OOM, std::string("hipMalloc: ") + hipGetErrorString(e));
    }
    e = hipMemcpy(w->mem, pk.buf.data(), pk.buf.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(w->mem);
        delete w;
        return fail(HYMT_E_DEVICE, std::string("hipMemcpy: ") + hipGetErrorString(e));
    }
    uint8_t *base = (uint8_t *)w->mem;
    w->bytes = pk.buf.size();
    w->dev.type = type;
    w->dev.rows = rows;
    w->dev.cols = cols;
    w->dev.q = base + pk.off_q;
    w->dev.q2 = pk.off_q2 == SIZE_MAX ? nullptr : base + pk.off_q2;
    w->dev.d = pk.off_d == SIZE_MAX ? nullptr : (const float *)(base + pk.off_d);
    *out = w;
    return HYMT_OK;
}

int hymt_weight_free(hymt_ctx *c, hymt_weight *w) {
    if (int r = check_ctx(c, false, true)) return r;
    if (!w) return HYMT_OK;
    if (int r = refuse_in_capture(c, "hymt_weight_free")) return r;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    hipError_t e = hipFree(w->mem);
    if (w->dense) {
        const hipError_t e2 = hipFree(w->dense);
        if (e == hipSuccess) e = e2;
    }
    delete w;
    if (e != hipSuccess) return fail(HYMT_E_DEVICE, std::string("hipFree: ") + hipGetErrorString(e));
    return HYMT_OK;
}

int hymt_weight_info(const hymt_weight *w, int *type, int *rows, int *cols, size_t *device_bytes) {
    if (!w) return fail(HYMT_E_ARG, "null weight");
    if (type) *type = w->dev.type;
    if (rows) *rows = w->dev.rows;
    if (cols) *cols = w->dev.cols;
    if (device_bytes) *device_bytes = w->bytes + (w->dense ? (size_t)w->dev.rows * w->dev.cols * 2 : 0);
    return HYMT_OK;
}

int hymt_gemv(hymt_ctx *c, const hymt_weight *w, const float *x, float *y, int flags, const float *norm_w,
              float eps) {
    if (int r = check_ctx(c, false, true)) return r;
    if (!w || !x || !y) return fail(HYMT_E_ARG, "null weight or vector");
    TimedCall timed(call_timer(c), "gemv", w->dev.rows);
    if (flags & ~(HYMT_GEMV_ACCUMULATE | HYMT_GEMV_IN_RMSNORM | HYMT_GEMV_IN_SWIGLU | HYMT_GEMV_OUT_SWIGLU))
        return fail(HYMT_E_ARG, "unknown gemv flags");
    if ((flags & HYMT_GEMV_OUT_SWIGLU) && (flags & HYMT_GEMV_ACCUMULATE))
        return fail(HYMT_E_ARG, "HYMT_GEMV_OUT_SWIGLU and HYMT_GEMV_ACCUMULATE exclude each other");
    if ((flags & HYMT_GEMV_OUT_SWIGLU) && (w->dev.rows & 1))
        return fail(HYMT_E_ARG, "HYMT_GEMV_OUT_SWIGLU needs [gate; up] rows (an even count)");
    if ((flags & HYMT_GEMV_IN_RMSNORM) && (flags & HYMT_GEMV_IN_SWIGLU))
        return fail(HYMT_E_ARG, "HYMT_GEMV_IN_RMSNORM and HYMT_GEMV_IN_SWIGLU exclude each other");
    if ((flags & HYMT_GEMV_IN_RMSNORM) && !norm_w) return fail(HYMT_E_ARG, "HYMT_GEMV_IN_RMSNORM needs norm_w");
    if (misaligned16(x) || ((flags & HYMT_GEMV_IN_RMSNORM) && misaligned16(norm_w)))
        return fail(HYMT_E_ARG, "x and norm_w must be 16-byte aligned");
    try {
        HIP_TRY(hipSetDevice(c->device));
        HIP_TRY(hymt::launch_gemv(w->dev, x, y, flags, norm_w, eps, c->stream));
    } catch (const HipError &e) {
        return map_hip(e);
    }
    return HYMT_OK;
}

int hymt_embed(hymt_ctx *c, const hymt_weight *w, int row, float *out) {
    if (int r = check_ctx(c, false, true)) return r;
    if (!w || !out) return fail(HYMT_E_ARG, "null weight or output");
    TimedCall timed(call_timer(c), "embed", row);
    if (row < 0 || row >= w->dev.rows)
        return fail(HYMT_E_ARG, "row " + std::to_string(row) + " outside [0, " + std::to_string(w->dev.rows) + ")");
    try {
        HIP_TRY(hipSetDevice(c->device));
        HIP_TRY(hymt::launch_embed(w->dev, row, out, c->stream));
    } catch (const HipError &e) {
        return map_hip(e);
    }
    return HYMT_OK;
}

// ---- prefill: dense weights, GEMMs and row kernels ----------------------------

int hymt_weight_dense(hymt_ctx *c, hymt_weight *w) {
    if (int r = check_ctx(c, false, true)) return r;
    if (!w) return fail(HYMT_E_ARG, "null weight");
    if (int r = refuse_in_capture(c, "hymt_weight_dense")) return r;
    if (w->dense) return HYMT_OK;
    const int rows = w->dev.rows, cols = w->dev.cols;
    const int chunk = std::max(1, std::min(rows, (int)((64u << 20) / ((size_t)cols * 4))));
    void *tmp = nullptr;
    try {
        HIP_TRY(hipSetDevice(c->device));
        HIP_TRY(hipMalloc((void **)&w->dense, (size_t)rows * cols * 2));
        HIP_TRY(hipMalloc(&tmp, (size_t)chunk * cols * 4));
        for (int r0 = 0; r0 < rows; r0 += chunk) {
            const int n = std::min(chunk, rows - r0);
            HIP_TRY(hymt::launch_rows(w->dev, nullptr, r0, n, (float *)tmp, c->stream));
            HIP_TRY(hymt::launch_to_bf16((const float *)tmp, (size_t)n * cols, w->dense + (size_t)r0 * cols,
                                         c->stream));
        }
        HIP_TRY(hipStreamSynchronize(c->stream));
        HIP_TRY(hipFree(tmp));
    } catch (const HipError &e) {
        if (tmp) (void)hipFree(tmp);
        if (w->dense) (void)hipFree(w->dense);
        w->dense = nullptr;
        return map_hip(e);
    }
    return HYMT_OK;
}

int hymt_gemm(hymt_ctx *c, const hymt_weight *w, int row0, int nrows, const void *x, int m, void *y, int flags) {
    if (int r = check_ctx(c, false, true)) return r;
    if (!w || !x || !y) return fail(HYMT_E_ARG, "null weight or matrix");
    TimedCall timed(call_timer(c), "gemm", m);
    if (!w->dense) return fail(HYMT_E_STATE, "weight has no dense copy (hymt_weight_dense)");
    if (flags & ~(HYMT_GEMM_ACCUMULATE | HYMT_GEMM_OUT_BF16)) return fail(HYMT_E_ARG, "unknown gemm flags");
    if ((flags & HYMT_GEMM_ACCUMULATE) && (flags & HYMT_GEMM_OUT_BF16))
        return fail(HYMT_E_ARG, "HYMT_GEMM_ACCUMULATE needs an fp32 output");
    if (row0 < 0 || nrows < 1 || row0 + nrows > w->dev.rows)
        return fail(HYMT_E_ARG, "rows [" + std::to_string(row0) + ", " + std::to_string(row0 + nrows) +
                                    ") outside the weight's " + std::to_string(w->dev.rows));
    if (m < 0) return fail(HYMT_E_ARG, "negative row count");
    if (int r = refuse_in_capture(c, "hymt_gemm")) return r;
    try {
        HIP_TRY(hipSetDevice(c->device));
        if (!c->gemm && !(c->gemm = gemm_state_create())) return fail(HYMT_E_OOM, "host allocation failed");
        HIP_TRY(hymt::gemm_bf16(c->gemm, c->stream, w->dense + (size_t)row0 * w->dev.cols, nrows, w->dev.cols,
                                (const uint16_t *)x, m, y, nrows, flags & HYMT_GEMM_OUT_BF16,
                                flags & HYMT_GEMM_ACCUMULATE));
    } catch (const HipError &e) {
        return map_hip(e);
    }
    return HYMT_OK;
}

int hymt_gemm_swiglu(hymt_ctx *c, const hymt_weight *gate, const hymt_weight *up, const void *x, int m, void *act) {
    if (int r = check_ctx(c, false, true)) return r;
    if (!gate || !x || !act) return fail(HYMT_E_ARG, "null weight or matrix");
    TimedCall timed(call_timer(c), "gemm_swiglu", m);
    if (!gate->dense || (up && !up->dense)) return fail(HYMT_E_STATE, "weight has no dense copy (hymt_weight_dense)");
    const int k = gate->dev.cols;
    const int f = up ? gate->dev.rows : gate->dev.rows / 2;
    if (up ? up->dev.rows != f || up->dev.cols != k : gate->dev.rows % 2 != 0)
        return fail(HYMT_E_ARG, "gate and up must have the same shape (or one weight an even number of rows)");
    if (m < 0) return fail(HYMT_E_ARG, "negative row count");
    if (int r = refuse_in_capture(c, "hymt_gemm_swiglu")) return r;
    if (m == 0) return HYMT_OK;
    try {
        HIP_TRY(hipSetDevice(c->device));
        if (!c->gemm && !(c->gemm = gemm_state_create())) return fail(HYMT_E_OOM, "host allocation failed");
        const uint16_t *wu = up ? up->dense : gate->dense + (size_t)f * k;
        hipError_t e = hipSuccess;
        // gu: a 16-byte aligned [m][2 f] buffer of the unfused calls (only its
        // alignment enters the choice)
        if (!gemm_swiglu(c->gemm, c->stream, gate->dense, wu, up != nullptr, f, k, (const uint16_t *)x, m, nullptr,
                         (uint16_t *)act, e))
            return fail(HYMT_E_UNSUPPORTED,
                        "no fused gate/up + SwiGLU with the unfused calls' bits here (the GEMM mode, a k split for "
                        "this prompt length, the shape or a misaligned x / act)");
        HIP_TRY(e);
    } catch (const HipError &e) {
        return map_hip(e);
    }
    return HYMT_OK;
}

int hymt_embed_rows(hymt_ctx *c, const hymt_weight *w, const int32_t *rows, int n, float *out) {
    if (int r = check_ctx(c, false, true)) return r;
    if (!w || !rows || !out) return fail(HYMT_E_ARG, "null weight, rows or output");
    TimedCall timed(call_timer(c), "embed_rows", n);
    if (n < 0) return fail(HYMT_E_ARG, "negative row count");
    for (int i = 0; i < n; i++)
        if (rows[i] < 0 || rows[i] >= w->dev.rows)
            return fail(HYMT_E_ARG, "row " + std::to_string(rows[i]) + " outside [0, " +
                                        std::to_string(w->dev.rows) + ")");
    if (int r = refuse_in_capture(c, "hymt_embed_rows")) return r;
    if (n == 0) return HYMT_OK;
    try {
        HIP_TRY(hipSetDevice(c->device));
        c->rows_idx.reserve((size_t)n * 4);
        HIP_TRY(hipMemcpyAsync(c->rows_idx.p, rows, (size_t)n * 4, hipMemcpyHostToDevice, c->stream));
        HIP_TRY(hymt::launch_rows(w->dev, (const int *)c->rows_idx.p, 0, n, out, c->stream));
        HIP_TRY(hipStreamSynchronize(c->stream));  // the host array may go once this returns
    } catch (const HipError &e) {
        return map_hip(e);
    }
    return HYMT_OK;
}

int hymt_rows_rmsnorm(hymt_ctx *c, const float *x, int m, int n, const float *norm_w, float eps, void *out) {
    if (int r = check_ctx(c, false, true)) return r;
    if (!x || !norm_w || !out) return fail(HYMT_E_ARG, "null input, weight or output");
    TimedCall timed(call_timer(c), "rows_rmsnorm", m);
    if (m < 0 || n < 4 || n > 8192 || n % 4 != 0) return fail(HYMT_E_UNSUPPORTED, "row length must be a multiple of 4 up to 8192");
    if (misaligned16(x) || misaligned16(norm_w) || ((uintptr_t)out & 7u))
        return fail(HYMT_E_ARG, "x and norm_w must be 16-byte aligned, out 8-byte aligned");
    try {
        HIP_TRY(hipSetDevice(c->device));
        HIP_TRY(hymt::launch_rows_rmsnorm(x, m, n, norm_w, eps, (uint16_t *)out, c->stream));
    } catch (const HipError &e) {
        return map_hip(e);
    }
    return HYMT_OK;
}

int hymt_rows_swiglu(hymt_ctx *c, const float *gate_up, int m, int n, void *out) {
    if (int r = check_ctx(c, false, true)) return r;
    if (!gate_up || !out) return fail(HYMT_E_ARG, "null input or output");
    TimedCall timed(call_timer(c), "rows_swiglu", m);
    if (m < 0 || n < 4 || n % 4 != 0) return fail(HYMT_E_UNSUPPORTED, "row length must be a multiple of 4");
    if (misaligned16(gate_up) || ((uintptr_t)out & 7u))
        return fail(HYMT_E_ARG, "gate_up must be 16-byte aligned, out 8-byte aligned");
    try {
        HIP_TRY(hipSetDevice(c->device));
        HIP_TRY(hymt::launch_rows_swiglu(gate_up, m, n, (uint16_t *)out, c->stream));
    } catch (const HipError &e) {
        return map_hip(e);
    }
    return HYMT_OK;
}

int hymt_rows_swiglu_bf16(hymt_ctx *c, const void *gate_up, int m, int n, void *out) {
    if (int r = check_ctx(c, false, true)) return r;
    if (!gate_up || !out) return fail(HYMT_E_ARG, "null input or output");
    TimedCall timed(call_timer(c), "rows_swiglu_bf16", m);
    if (m < 0 || n < 4 || n % 4 != 0) return fail(HYMT_E_UNSUPPORTED, "row length must be a multiple of 4");
    if (((uintptr_t)gate_up & 7u) || ((uintptr_t)out & 7u))
        return fail(HYMT_E_ARG, "gate_up and out must be 8-byte aligned");
    try {
        HIP_TRY(hipSetDevice(c->device));
        HIP_TRY(hymt::launch_rows_swiglu_bf16((const uint16_t *)gate_up, m, n, (uint16_t *)out, c->stream));
    } catch (const HipError &e) {
        return map_hip(e);
    }
    return HYMT_OK;
}

int hymt_to_bf16(hymt_ctx *c, const float *x, size_t count, void *out) {
    if (int r = check_ctx(c, false, true)) return r;
    if (!x || !out) return fail(HYMT_E_ARG, "null input or output");
    TimedCall timed(call_timer(c), "to_bf16", (int)count);
    if (count % 4 != 0) return fail(HYMT_E_UNSUPPORTED, "count must be a multiple of 4");
    if (misaligned16(x) || ((uintptr_t)out & 7u)) return fail(HYMT_E_ARG, "x must be 16-byte aligned, out 8-byte aligned");
    try {
        HIP_TRY(hipSetDevice(c->device));
        HIP_TRY(hymt::launch_to_bf16(x, count, (uint16_t *)out, c->stream));
    } catch (const HipError &e) {
        return map_hip(e);
    }
    return HYMT_OK;
}

// ---- the decode step of the model, enqueued natively -------------------------

struct hymt_model {
    hymt_ctx *ctx = nullptr;
    int layers = 0, hidden = 0, ffn = 0, vocab = 0;
    float eps = 1e-5f;
    struct Layer {
        const hymt_weight *w[6] = {};  // q|k|v (or q), k, v, o, gate|up (or gate), up; down below
        const hymt_weight *down = nullptr;
        const float *attn_norm = nullptr, *ffn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
        bool set = false;
    };
    std::vector<Layer> L;
    const hymt_weight *embd = nullptr, *out = nullptr;
    const float *out_norm = nullptr;
    DevBuf h, qkv, ao, gu;
    // prefill activations (hymt_model_prefill), allocated on its first call
    // for kPrefillRows rows: x fp32 [C][H], xn bf16 [C][H], qkv bf16
    // [C][q|k|v], ao16 bf16 [C][qd] (the attention writes it as bf16), gu [C][2F] (bf16, or fp32
    // with HYMT_PREFILL_GATE_UP_F32), act bf16 [C][F]; token ids through a
    // pinned buffer whose last copy is marked by tok_ev
    DevBuf px, pxn, pqkv, pao16, pgu, pact, ptok;
    HostBuf htok;
    hipEvent_t tok_ev = nullptr;
};

namespace {
constexpr int kPrefillRows = 2048;

// The prefill GEMM path needs a bf16 dense copy of every layer weight and a
// 16-bit cache (the prefill kernels read 16-bit pages).
bool prefill_ready(const hymt_model *m) {
    if (m->ctx->kv_dtype == HYMT_F32) return false;
    for (const auto &Ly : m->L) {
        for (const hymt_weight *w : Ly.w)
            if (w && !w->dense) return false;
        if (!Ly.down->dense) return false;
    }
    return true;
}

// y (+)= x . W^T over the weight's dense copy, rows ldy elements apart
void model_gemm(hymt_ctx *c, const hymt_weight *w, const void *x, int m, void *y, int ldy, bool y_bf16, bool acc) {
    if (!c->gemm && !(c->gemm = gemm_state_create())) throw HipError{hipErrorOutOfMemory, "gemm_state_create"};
    HIP_TRY(gemm_bf16(c->gemm, c->stream, w->dense, w->dev.rows, w->dev.cols, (const uint16_t *)x, m, y, ldy, y_bf16,
                      acc));
}
}  // namespace

int hymt_model_create(hymt_ctx *c, int layers, int hidden, int ffn, int vocab, float eps, hymt_model **out) {
    if (int r = check_ctx(c, true, true)) return r;
    if (!out) return fail(HYMT_E_ARG, "null output pointer");
    *out = nullptr;
    if (layers != c->layers || hidden < 2048 || hidden % 2048 || ffn < 2048 || ffn % 2048 || vocab < 1)
        return fail(HYMT_E_ARG, "model shape does not match the cache or the GEMV limits");
    if (int r = refuse_in_capture(c, "hymt_model_create")) return r;
    hymt_model *m = new (std::nothrow) hymt_model();
    if (!m) return fail(HYMT_E_OOM, "host allocation failed");
    m->ctx = c;
    m->layers = layers;
    m->hidden = hidden;
    m->ffn = ffn;
    m->vocab = vocab;
    m->eps = eps;
    m->L.resize(layers);
    try {
        HIP_TRY(hipSetDevice(c->device));
        const size_t qd = (size_t)c->heads * c->head_dim, kd = (size_t)c->kv_heads * c->head_dim;
        m->h.reserve((size_t)hidden * 4);
        m->qkv.reserve((qd + 2 * kd) * 4);
        m->ao.reserve(qd * 4);
        m->gu.reserve((size_t)2 * ffn * 4);
    } catch (const HipError &e) {
        for (DevBuf *b : {&m->h, &m->qkv, &m->ao, &m->gu}) b->release();
        delete m;
        return map_hip(e);
    }
    *out = m;
    return HYMT_OK;
}

int hymt_model_set_layer(hymt_model *m, int layer, const hymt_weight *q_or_qkv, const hymt_weight *k,
                         const hymt_weight *v, const hymt_weight *o, const hymt_weight *gate_or_gate_up,
                         const hymt_weight *up, const hymt_weight *down, const float *attn_norm,
                         const float *ffn_norm, const float *q_norm, const float *k_norm) {
    if (!m) return fail(HYMT_E_ARG, "null model");
    if (layer < 0 || layer >= m->layers) return fail(HYMT_E_ARG, "layer out of range");
    hymt_ctx *c = m->ctx;
    const int qd = c->heads * c->head_dim, kd = c->kv_heads * c->head_dim;
    auto shape = [](const hymt_weight *w, int rows, int cols) {
        return w && w->dev.rows == rows && w->dev.cols == cols;
    };
    const bool fused_qkv = !k && !v;
    const bool fused_gu = !up;
    bool ok = fused_qkv ? shape(q_or_qkv, qd + 2 * kd, m->hidden)
                        : shape(q_or_qkv, qd, m->hidden) && shape(k, kd, m->hidden) && shape(v, kd, m->hidden);
    ok = ok && shape(o, m->hidden, qd) && shape(down, m->hidden, m->ffn);
    ok = ok && (fused_gu ? shape(gate_or_gate_up, 2 * m->ffn, m->hidden)
                         : shape(gate_or_gate_up, m->ffn, m->hidden) && shape(up, m->ffn, m->hidden));
    if (!ok) return fail(HYMT_E_ARG, "layer weights do not have the model's shapes");
    if (!attn_norm || !ffn_norm || misaligned16(attn_norm) || misaligned16(ffn_norm) || misaligned16(q_norm) ||
        misaligned16(k_norm))
        return fail(HYMT_E_ARG, "norm vectors must be 16-byte aligned device pointers");
    hymt_model::Layer &Ly = m->L[layer];
    Ly.w[0] = q_or_qkv;
    Ly.w[1] = k;
    Ly.w[2] = v;
    Ly.w[3] = o;
    Ly.w[4] = gate_or_gate_up;
    Ly.w[5] = up;
    Ly.down = down;
    Ly.attn_norm = attn_norm;
    Ly.ffn_norm = ffn_norm;
    Ly.q_norm = q_norm;
    Ly.k_norm = k_norm;
    Ly.set = true;
    return HYMT_OK;
}

int hymt_model_set_io(hymt_model *m, const hymt_weight *embd, const hymt_weight *out, const float *out_norm) {
    if (!m) return fail(HYMT_E_ARG, "null model");
    if (!embd || embd->dev.cols != m->hidden || embd->dev.rows != m->vocab)
        return fail(HYMT_E_ARG, "token_embd must be vocab x hidden");
    if (out && (out->dev.cols != m->hidden || out->dev.rows != m->vocab))
        return fail(HYMT_E_ARG, "output must be vocab x hidden");
    if (!out_norm || misaligned16(out_norm)) return fail(HYMT_E_ARG, "out_norm must be a 16-byte aligned device vector");
    m->embd = embd;
    m->out = out ? out : embd;  // the tied embedding (HunyuanDenseModel.cs:419)
    m->out_norm = out_norm;
    return HYMT_OK;
}

int hymt_model_decode(hymt_model *m, int token, int pos, float *logits) {
    if (!m) return fail(HYMT_E_ARG, "null model");
    hymt_ctx *c = m->ctx;
    if (int r = check_ctx(c, true, true)) return r;
    TimedCall timed(call_timer(c), "model_decode", pos);
    if (!m->embd || !logits) return fail(HYMT_E_STATE, "hymt_model_set_io first (and a logits buffer)");
    for (const auto &Ly : m->L)
        if (!Ly.set) return fail(HYMT_E_STATE, "every layer needs hymt_model_set_layer");
    if (token < 0 || token >= m->vocab) return fail(HYMT_E_ARG, "token out of range");
    // checked here as well as by each attention call, so that a bad position
    // enqueues nothing
    if (pos < 0) return fail(HYMT_E_ARG, "negative position");
    if ((long)pos + 1 > c->pages.max_tokens())
        return fail(HYMT_E_CAPACITY, "KV capacity " + std::to_string(c->pages.max_tokens()) + " exceeded at " +
                                         std::to_string((long)pos + 1));
    if (!c->pages.resident(pos)) return fail(HYMT_E_STATE, "device KV must hold [0, pos) before decode");
    const int qd = c->heads * c->head_dim, kd = c->kv_heads * c->head_dim;
    float *h = (float *)m->h.p, *qkv = (float *)m->qkv.p, *ao = (float *)m->ao.p, *gu = (float *)m->gu.p;
    const int norm_in = HYMT_GEMV_IN_RMSNORM;
    try {
        HIP_TRY(hipSetDevice(c->device));
        HIP_TRY(hymt::launch_embed(m->embd->dev, token, h, c->stream));
        for (int l = 0; l < m->layers; l++) {
            const hymt_model::Layer &Ly = m->L[l];
            if (!Ly.w[1]) {
                HIP_TRY(hymt::launch_gemv(Ly.w[0]->dev, h, qkv, norm_in, Ly.attn_norm, m->eps, c->stream));
            } else {
                HIP_TRY(hymt::launch_gemv(Ly.w[0]->dev, h, qkv, norm_in, Ly.attn_norm, m->eps, c->stream));
                HIP_TRY(hymt::launch_gemv(Ly.w[1]->dev, h, qkv + qd, norm_in, Ly.attn_norm, m->eps, c->stream));
                HIP_TRY(hymt::launch_gemv(Ly.w[2]->dev, h, qkv + qd + kd, norm_in, Ly.attn_norm, m->eps, c->stream));
            }
            if (int r = hymt_attn_decode(c, l, pos, qkv, qkv + qd, qkv + qd + kd, Ly.q_norm, Ly.k_norm, ao,
                                         HYMT_FLAG_DEVICE_PTRS))
                return r;
            HIP_TRY(hymt::launch_gemv(Ly.w[3]->dev, ao, h, HYMT_GEMV_ACCUMULATE, nullptr, m->eps, c->stream));
            if (!Ly.w[5]) {
                // one [gate; up] matrix: silu(gate) * up straight out of its GEMV
                HIP_TRY(hymt::launch_gemv(Ly.w[4]->dev, h, gu, norm_in | HYMT_GEMV_OUT_SWIGLU, Ly.ffn_norm, m->eps,
                                          c->stream));
                HIP_TRY(hymt::launch_gemv(Ly.down->dev, gu, h, HYMT_GEMV_ACCUMULATE, nullptr, m->eps, c->stream));
            } else {
                HIP_TRY(hymt::launch_gemv(Ly.w[4]->dev, h, gu, norm_in, Ly.ffn_norm, m->eps, c->stream));
                HIP_TRY(hymt::launch_gemv(Ly.w[5]->dev, h, gu + m->ffn, norm_in, Ly.ffn_norm, m->eps, c->stream));
                HIP_TRY(hymt::launch_gemv(Ly.down->dev, gu, h, HYMT_GEMV_ACCUMULATE | HYMT_GEMV_IN_SWIGLU, nullptr,
                                          m->eps, c->stream));
            }
        }
        HIP_TRY(hymt::launch_gemv(m->out->dev, h, logits, norm_in, m->out_norm, m->eps, c->stream));
    } catch (const HipError &e) {
        return map_hip(e);
    }
    return HYMT_OK;
}

int hymt_model_prefill(hymt_model *m, const int32_t *tokens, int n, int pos, float *logits, unsigned flags) {
    if (!m) return fail(HYMT_E_ARG, "null model");
    hymt_ctx *c = m->ctx;
    if (int r = check_ctx(c, true, true)) return r;
    TimedCall timed(call_timer(c), "model_prefill", n);
    if (!m->embd || !logits) return fail(HYMT_E_STATE, "hymt_model_set_io first (and a logits buffer)");
    for (const auto &Ly : m->L)
        if (!Ly.set) return fail(HYMT_E_STATE, "every layer needs hymt_model_set_layer");
    if (flags & ~HYMT_PREFILL_GATE_UP_F32) return fail(HYMT_E_ARG, "unknown prefill flags");
    if (n < 1 || !tokens) return fail(HYMT_E_ARG, "empty token list");
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= m->vocab) return fail(HYMT_E_ARG, "token out of range");
    if (pos < 0) return fail(HYMT_E_ARG, "negative position");
    if ((long)pos + n > c->pages.max_tokens())
        return fail(HYMT_E_CAPACITY, "KV capacity " + std::to_string(c->pages.max_tokens()) + " exceeded at " +
                                         std::to_string((long)pos + n));
    if (!c->pages.resident(pos)) return fail(HYMT_E_STATE, "device KV must hold [0, pos) before prefill");
    if (int r = refuse_in_capture(c, "hymt_model_prefill")) return r;
    if (n == 1 || !prefill_ready(m)) {
        // one token, an fp32 cache or no dense copies: the tokens run as
        // decode steps, as ForwardStep does without a prefill path
        for (int i = 0; i < n; i++)
            if (int r = hymt_model_decode(m, tokens[i], pos + i, logits)) return r;
        return HYMT_OK;
    }
    const int H = m->hidden, F = m->ffn, qd = c->heads * c->head_dim, kd = c->kv_heads * c->head_dim;
    const int ld = qd + 2 * kd;
    const bool gu32 = flags & HYMT_PREFILL_GATE_UP_F32;
    const size_t C = kPrefillRows;
    try {
        HIP_TRY(hipSetDevice(c->device));
        m->px.reserve(C * H * 4);
        m->pxn.reserve(C * H * 2);
        m->pqkv.reserve(C * ld * 2);
        m->pao16.reserve(C * qd * 2);
        m->pgu.reserve(C * 2 * F * 4);
        m->pact.reserve(C * F * 2);
        m->ptok.reserve(C * 4);
        if (!m->htok.p) {
            m->htok.reserve(C * 4);
            HIP_TRY(hipEventCreateWithFlags(&m->tok_ev, hipEventDisableTiming));
        }
        float *x = (float *)m->px.p;
        uint16_t *xn = (uint16_t *)m->pxn.p, *qkv = (uint16_t *)m->pqkv.p, *ao16 = (uint16_t *)m->pao16.p;
        uint16_t *act = (uint16_t *)m->pact.p;
        void *gu = m->pgu.p;
        for (int r0 = 0; r0 < n; r0 += kPrefillRows) {
            const int rows = std::min(kPrefillRows, n - r0), p0 = pos + r0;
            // token ids: host -> pinned -> device, the pinned buffer reused
            // once the previous chunk's copy has read it
            HIP_TRY(hipEventSynchronize(m->tok_ev));
            std::memcpy(m->htok.p, tokens + r0, (size_t)rows * 4);
            HIP_TRY(hipMemcpyAsync(m->ptok.p, m->htok.p, (size_t)rows * 4, hipMemcpyHostToDevice, c->stream));
            HIP_TRY(hipEventRecord(m->tok_ev, c->stream));
            HIP_TRY(launch_rows(m->embd->dev, (const int *)m->ptok.p, 0, rows, x, c->stream));
            for (int l = 0; l < m->layers; l++) {
                const hymt_model::Layer &Ly = m->L[l];
                HIP_TRY(launch_rows_rmsnorm(x, rows, H, Ly.attn_norm, m->eps, xn, c->stream));
                if (!Ly.w[1]) {
                    model_gemm(c, Ly.w[0], xn, rows, qkv, ld, true, false);
                } else {  // q, k, v as three matrices into the column ranges of one buffer
                    model_gemm(c, Ly.w[0], xn, rows, qkv, ld, true, false);
                    model_gemm(c, Ly.w[1], xn, rows, qkv + qd, ld, true, false);
                    model_gemm(c, Ly.w[2], xn, rows, qkv + qd + kd, ld, true, false);
                }
                if (int r = prefill_impl(c, l, p0, rows, qkv, ld, qkv + qd, qkv + qd + kd, ld, HYMT_BF16, Ly.q_norm,
                                         Ly.k_norm, (float *)ao16, HYMT_FLAG_DEVICE_PTRS, true))
                    return r;
                model_gemm(c, Ly.w[3], ao16, rows, x, H, false, true);
                HIP_TRY(launch_rows_rmsnorm(x, rows, H, Ly.ffn_norm, m->eps, xn, c->stream));
                // gate/up GEMM + SwiGLU in one launch where that gives the
                // bits of the two calls below (gemm_swiglu)
                const uint16_t *wg = Ly.w[4]->dense, *wu = Ly.w[5] ? Ly.w[5]->dense : wg + (size_t)F * H;
                hipError_t fe = hipSuccess;
                if (!gu32 && gemm_swiglu(c->gemm, c->stream, wg, wu, Ly.w[5] != nullptr, F, H, xn, rows,
                                         (const uint16_t *)gu, act, fe)) {
                    HIP_TRY(fe);
                } else {
                    if (!Ly.w[5]) {
                        model_gemm(c, Ly.w[4], xn, rows, gu, 2 * F, !gu32, false);
                    } else {  // gate and up as two matrices into the halves of one row
                        const size_t es = gu32 ? 4 : 2;
                        model_gemm(c, Ly.w[4], xn, rows, gu, 2 * F, !gu32, false);
                        model_gemm(c, Ly.w[5], xn, rows, (char *)gu + F * es, 2 * F, !gu32, false);
                    }
                    if (gu32)
                        HIP_TRY(launch_rows_swiglu((const float *)gu, rows, F, act, c->stream));
                    else
                        HIP_TRY(launch_rows_swiglu_bf16((const uint16_t *)gu, rows, F, act, c->stream));
                }
                model_gemm(c, Ly.down, act, rows, x, H, false, true);
            }
            if (r0 + rows == n)
                HIP_TRY(launch_gemv(m->out->dev, x + (size_t)(rows - 1) * H, logits, HYMT_GEMV_IN_RMSNORM,
                                    m->out_norm, m->eps, c->stream));
        }
    } catch (const HipError &e) {
        return map_hip(e);
    }
    return HYMT_OK;
}

int hymt_model_destroy(hymt_model *m) {
    if (!m) return HYMT_OK;
    hymt_ctx *c = m->ctx;
    if (c && c->has_device()) {
        (void)hipSetDevice(c->device);
        (void)hipStreamSynchronize(c->stream);
    }
    for (DevBuf *b : {&m->h, &m->qkv, &m->ao, &m->gu, &m->px, &m->pxn, &m->pqkv, &m->pao16, &m->pgu,
                      &m->pact, &m->ptok})
        b->release();
    m->htok.release();
    if (m->tok_ev) (void)hipEventDestroy(m->tok_ev);
    delete m;
    return HYMT_OK;
}
