// tsm_api.hip - the C ABI (include/tachyon_sampler.h): context, argument
// checks on the host, and the one launch of a step on the caller's stream.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "tsm_sample.h"
#include "tsm_split.h"

struct tsm_ctx {
    int device;
    uint32_t max_rows, max_vocab;
    uint32_t* status;  // TSM_STATUS_* bits of the calls since the last tsm_status()
    void* split_mem;   // the split kernel's scratch (tsm::split::SplitScratch)
    tsm::split::SplitScratch split;
    // tsm_status() waits for the last call through an event on that call's
    // stream and reads the status on a stream of the context's own (created
    // non-blocking, default priority), so it stalls no other stream
    hipEvent_t last;
    bool called;
    hipStream_t own;
    uint32_t* host_word;  // pinned: the status word read back
};

namespace {

void set_err(char* err, size_t errlen, const char* fmt, ...) {
    if (!err || errlen == 0) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, errlen, fmt, ap);
    va_end(ap);
}

struct DeviceGuard {
    int prev = -1;
    bool ok = false;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        ok = hipSetDevice(dev) == hipSuccess;
    }
    ~DeviceGuard() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_batch(uint32_t max_rows, uint32_t max_vocab, const tsm_batch* b, char* err, size_t errlen) {
    if (!b) return set_err(err, errlen, "batch is NULL"), 1;
    if (!b->logits) return set_err(err, errlen, "batch->logits is NULL"), 1;
    if (!b->params) return set_err(err, errlen, "batch->params is NULL"), 1;
    if (b->rows == 0) return set_err(err, errlen, "batch->rows is 0"), 1;
    if (b->rows > max_rows)
        return set_err(err, errlen, "batch->rows %u exceeds the maximum of %u", b->rows, max_rows), 1;
    if (b->usable == 0) return set_err(err, errlen, "batch->usable is 0"), 1;
    if (b->usable > max_vocab)
        return set_err(err, errlen, "batch->usable %u exceeds the maximum of %u", b->usable, max_vocab), 1;
    if (b->usable > b->row_stride)
        return set_err(err, errlen, "batch->usable %u exceeds row_stride %u", b->usable, b->row_stride), 1;
    if ((b->hist_ids == nullptr) != (b->hist_offsets == nullptr))
        return set_err(err, errlen, "hist_ids and hist_offsets must both be set or both be NULL"), 1;
    if (b->row_kinds & ~(TSM_ROWKIND_SPLIT | TSM_ROWKIND_WHOLE | TSM_ROWKIND_LEAN))
        return set_err(err, errlen, "batch->row_kinds 0x%x has unknown bits", b->row_kinds), 1;
    if (b->reserved != 0) return set_err(err, errlen, "batch->reserved must be 0"), 1;
    if (b->mask && b->mask_stride < (b->usable + 31) / 32)
        return set_err(err, errlen, "mask_stride %u is below ceil(usable/32) = %u", b->mask_stride,
                       (b->usable + 31) / 32), 1;
    return 0;
}

// ---- the allocation-free entry point's scratch ------------------------------------
// tsm_sample_static allocates nothing: the split kernel's records for batches
// of up to kStaticRows rows of up to kStaticVocab ids, and a status word, live
// in this file-scope array (each GPU the library runs on holds its own copy
// until the process ends).  Host code never passes `scratch` itself to a
// kernel: its device address comes from hipGetSymbolAddress, once per device.
constexpr uint32_t kStaticRows = tsm::split::kSplitRowsMax;
constexpr uint32_t kStaticVocab = 1u << 18;
constexpr uint64_t kStaticSplitBytes = tsm::split::scratch_bytes(kStaticRows, kStaticVocab);
constexpr uint64_t kStaticBytes = kStaticSplitBytes + 256;  // + the status word
static __device__ __align__(256) unsigned char scratch[kStaticBytes];

constexpr uint32_t kStaticMaxRows = 65535;  // the whole-row kernel needs no scratch but the status word
constexpr int kMaxDevices = 64;
struct StaticDev {
    void* ptr = nullptr;  // device address of `scratch` on this device
    bool ready = false;
};
StaticDev g_static[kMaxDevices];
std::mutex g_static_mu;

// Clears n words (a fill kernel rather than a memset, so that a caller may
// capture the call in a graph).
__global__ void clear_words(uint32_t* p, uint32_t n) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// The current device's scratch address and kernel attributes, set up on its
// first call.
int static_setup(int* dev_out, void** ptr_out, char* err, size_t errlen) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return set_err(err, errlen, "no current HIP device"), 1;
    std::lock_guard<std::mutex> lk(g_static_mu);
    StaticDev& d = g_static[dev];
    if (!d.ready) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, dev) != hipSuccess)
            return set_err(err, errlen, "hipGetDeviceProperties failed"), 1;
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
            return set_err(err, errlen, "device %d is %s; this library is built for gfx950", dev, prop.gcnArchName), 1;
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return set_err(err, errlen, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e)), 1;
        const hipError_t e2 = tsm::sample_set_smem_attr();
        if (e2 != hipSuccess) return set_err(err, errlen, "kernel attribute setup failed: %s", hipGetErrorString(e2)), 1;
        d.ptr = p;
        d.ready = true;
    }
    *dev_out = dev;
    *ptr_out = d.ptr;
    return 0;
}

}  // namespace

extern "C" {

const char* tsm_version(void) { return "tachyon-sampler 0.2 gfx950"; }

uint32_t tsm_row_kind(const tsm_row_params* p, uint32_t usable, uint32_t hist_len, int has_mask) {
    if (!p || usable == 0) return TSM_ROWKIND_WHOLE;
    const tsm::RowMode m = tsm::row_mode(*p, usable, hist_len, has_mask != 0);
    const uint32_t whole = tsm::lean_takes(m, *p, hist_len, usable, false) ? TSM_ROWKIND_LEAN : TSM_ROWKIND_WHOLE;
    return (tsm::split::takes_row(m, hist_len) ? TSM_ROWKIND_SPLIT : 0u) | whole;
}

tsm_ctx* tsm_create(int device, uint32_t max_rows, uint32_t max_vocab, char* err, size_t errlen) {
    if (max_rows == 0 || max_rows > 65535) {
        set_err(err, errlen, "max_rows must be in [1, 65535], got %u", max_rows);
        return nullptr;
    }
    if (max_vocab == 0 || max_vocab > TSM_MAX_VOCAB) {
        set_err(err, errlen, "max_vocab must be in [1, %u], got %u", TSM_MAX_VOCAB, max_vocab);
        return nullptr;
    }
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev) {
        set_err(err, errlen, "HIP device %d not available (%d devices)", device, ndev);
        return nullptr;
    }
    DeviceGuard g(device);
    if (!g.ok) {
        set_err(err, errlen, "hipSetDevice(%d) failed", device);
        return nullptr;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
        set_err(err, errlen, "hipGetDeviceProperties failed");
        return nullptr;
    }
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_err(err, errlen, "device %d is %s; this library is built for gfx950", device, prop.gcnArchName);
        return nullptr;
    }
    tsm_ctx* c = new tsm_ctx();
    c->device = device;
    c->max_rows = max_rows;
    c->max_vocab = max_vocab;
    c->status = nullptr;
    c->split_mem = nullptr;
    c->last = nullptr;
    c->called = false;
    c->own = nullptr;
    c->host_word = nullptr;
    hipError_t e = hipMalloc(&c->status, sizeof(uint32_t));
    if (e == hipSuccess) e = hipEventCreateWithFlags(&c->last, hipEventDisableTiming);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->own, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&c->host_word), sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemset(c->status, 0, sizeof(uint32_t));
    // the split kernel runs for batches of at most kSplitRowsMax rows
    const uint32_t split_rows = max_rows < tsm::split::kSplitRowsMax ? max_rows : tsm::split::kSplitRowsMax;
    const size_t sb = tsm::split::scratch_bytes(split_rows, max_vocab);
    if (e == hipSuccess) e = hipMalloc(&c->split_mem, sb);
    // the row counters must start at 0; the kernel returns them to 0
    if (e == hipSuccess) e = hipMemset(c->split_mem, 0, sb);
    if (e == hipSuccess) c->split = tsm::split::scratch_carve(c->split_mem, split_rows, max_vocab);
    if (e == hipSuccess) e = tsm::sample_set_smem_attr();
    if (e != hipSuccess) {
        set_err(err, errlen, "device setup failed: %s", hipGetErrorString(e));
        tsm_destroy(c);
        return nullptr;
    }
    return c;
}

void tsm_destroy(tsm_ctx* ctx) {
    if (!ctx) return;
    DeviceGuard g(ctx->device);
    (void)hipDeviceSynchronize();
    if (ctx->status) (void)hipFree(ctx->status);
    if (ctx->split_mem) (void)hipFree(ctx->split_mem);
    if (ctx->last) (void)hipEventDestroy(ctx->last);
    if (ctx->own) (void)hipStreamDestroy(ctx->own);
    if (ctx->host_word) (void)hipHostFree(ctx->host_word);
    delete ctx;
}

// Queues one step: the split kernel for the batch's split-kind rows (small
// batches, when `split` is given), the whole-row kernel for the others.
static int queue(hipStream_t s, const tsm_batch* b, const tsm_outputs* out, uint32_t* dist_ids, float* dist_probs,
                 uint32_t dist_stride, uint32_t* keep, bool distribution, uint32_t* status,
                 const tsm::split::SplitScratch* split, char* err, size_t errlen) {
    const bool vec = (b->row_stride % 4 == 0) && aligned16(b->logits);

    tsm::SampleArgs a;
    std::memset(&a, 0, sizeof(a));
    a.logits = b->logits;
    a.params = b->params;
    a.hist_ids = b->hist_ids;
    a.hist_off = b->hist_offsets;
    a.mask = distribution ? nullptr : b->mask;
    a.uniforms = b->uniforms;
    a.status = status;
    a.row_stride = b->row_stride;
    a.usable = b->usable;
    a.mask_stride = b->mask_stride;
    a.distribution = distribution ? 1u : 0u;
    if (distribution) {
        a.dist_ids = dist_ids;
        a.dist_probs = dist_probs;
        a.dist_stride = dist_stride;
        a.out_keep = keep;
    } else {
        a.out_token = out->token;
        a.out_logprob = out->logprob;
        a.out_top_ids = out->top_ids;
        a.out_top_lp = out->top_logprobs;
        a.top_stride = out->top_stride;
        a.out_prob = out->prob;
        a.out_keep = out->keep;
    }
    // one kernel per row kind the batch holds (every kernel when it does not
    // say).  The split-row kernel pays off for small batches, where one
    // workgroup per row would leave most of the chip idle; from
    // kSplitRowsMax rows on, the whole-row kernels sample every row.  The
    // lean kernel takes the common top-k rows, the general kernel every
    // other; distribution() always takes the general kernel.
    uint32_t kinds = b->row_kinds ? b->row_kinds : (TSM_ROWKIND_SPLIT | TSM_ROWKIND_WHOLE | TSM_ROWKIND_LEAN);
    if (b->rows > tsm::split::kSplitRowsMax || !split) {
        // a split-kind row takes a whole-row kernel: the one its kind names
        // beside SPLIT (kinds from tsm_row_kind always name one); a bare
        // SPLIT says nothing more, so the general kernel takes it
        if ((kinds & TSM_ROWKIND_SPLIT) && !(kinds & (TSM_ROWKIND_WHOLE | TSM_ROWKIND_LEAN))) kinds |= TSM_ROWKIND_WHOLE;
        kinds &= ~TSM_ROWKIND_SPLIT;
    }
    if (distribution && (kinds & TSM_ROWKIND_LEAN)) kinds = (kinds & ~TSM_ROWKIND_LEAN) | TSM_ROWKIND_WHOLE;
    if (kinds & TSM_ROWKIND_SPLIT) {
        tsm::split::SplitArgs sa;
        sa.s = a;
        sa.w = *split;
        sa.seg_len = tsm::split::pick_seg_len(b->rows, b->usable);
        sa.nseg = (b->usable + sa.seg_len - 1) / sa.seg_len;
        sa.general = (kinds & (TSM_ROWKIND_WHOLE | TSM_ROWKIND_LEAN)) ? 1u : 0u;
        tsm::split::launch(sa, b->rows, vec, s);
    }
    if (kinds & (TSM_ROWKIND_WHOLE | TSM_ROWKIND_LEAN)) {
        a.skip_split = (kinds & TSM_ROWKIND_SPLIT) ? 1u : 0u;
        tsm::launch_sample(a, b->rows, vec, (kinds & TSM_ROWKIND_LEAN) != 0u, (kinds & TSM_ROWKIND_WHOLE) != 0u, s);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_err(err, errlen, "kernel launch failed: %s", hipGetErrorString(e)), 1;
    return 0;
}

static int run(tsm_ctx* ctx, void* stream, const tsm_batch* b, const tsm_outputs* out, uint32_t* dist_ids,
               float* dist_probs, uint32_t dist_stride, uint32_t* keep, bool distribution, char* err,
               size_t errlen) {
    if (!ctx) return set_err(err, errlen, "context is NULL"), 1;
    if (check_batch(ctx->max_rows, ctx->max_vocab, b, err, errlen)) return 1;
    DeviceGuard g(ctx->device);
    if (!g.ok) return set_err(err, errlen, "hipSetDevice(%d) failed", ctx->device), 1;
    if (queue(static_cast<hipStream_t>(stream), b, out, dist_ids, dist_probs, dist_stride, keep, distribution,
              ctx->status, &ctx->split, err, errlen))
        return 1;
    const hipError_t e = hipEventRecord(ctx->last, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return set_err(err, errlen, "hipEventRecord failed: %s", hipGetErrorString(e)), 1;
    ctx->called = true;
    return 0;
}

int tsm_sample(tsm_ctx* ctx, void* stream, const tsm_batch* batch, const tsm_outputs* out, char* err,
               size_t errlen) {
    if (!out || !out->token) return set_err(err, errlen, "outputs->token is NULL"), 1;
    if (batch && !batch->uniforms) return set_err(err, errlen, "batch->uniforms is NULL"), 1;
    if ((out->top_ids || out->top_logprobs) && out->top_stride == 0)
        return set_err(err, errlen, "top_stride is 0 while top_ids/top_logprobs are given"), 1;
    if (out->top_logprobs && !out->top_ids)
        return set_err(err, errlen, "top_logprobs needs top_ids"), 1;
    if (out->top_stride > TSM_MAX_LOGPROBS && (out->top_ids || out->top_logprobs))
        return set_err(err, errlen, "top_stride %u exceeds TSM_MAX_LOGPROBS", out->top_stride), 1;
    return run(ctx, stream, batch, out, nullptr, nullptr, 0, nullptr, false, err, errlen);
}

int tsm_distribution(tsm_ctx* ctx, void* stream, const tsm_batch* batch, uint32_t* dist_ids, float* dist_probs,
                     uint32_t dist_stride, uint32_t* keep, char* err, size_t errlen) {
    if (!dist_ids || !dist_probs || !keep) return set_err(err, errlen, "dist_ids, dist_probs and keep are required"), 1;
    if (dist_stride == 0) return set_err(err, errlen, "dist_stride is 0"), 1;
    return run(ctx, stream, batch, nullptr, dist_ids, dist_probs, dist_stride, keep, true, err, errlen);
}

int tsm_status(tsm_ctx* ctx, uint32_t* status, char* err, size_t errlen) {
    if (!ctx || !status) return set_err(err, errlen, "context or status is NULL"), 1;
    DeviceGuard g(ctx->device);
    hipError_t e = ctx->called ? hipEventSynchronize(ctx->last) : hipSuccess;
    if (e == hipSuccess)
        e = hipMemcpyAsync(ctx->host_word, ctx->status, sizeof(uint32_t), hipMemcpyDeviceToHost, ctx->own);
    if (e == hipSuccess) e = hipMemsetAsync(ctx->status, 0, sizeof(uint32_t), ctx->own);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->own);
    if (e != hipSuccess) return set_err(err, errlen, "status read failed: %s", hipGetErrorString(e)), 1;
    *status = *ctx->host_word;
    return 0;
}

int tsm_sample_static(void* stream, const tsm_batch* batch, const tsm_outputs* out, uint32_t* status, char* err,
                      size_t errlen) {
    if (!out || !out->token) return set_err(err, errlen, "outputs->token is NULL"), 1;
    if (batch && !batch->uniforms) return set_err(err, errlen, "batch->uniforms is NULL"), 1;
    if ((out->top_ids || out->top_logprobs) && out->top_stride == 0)
        return set_err(err, errlen, "top_stride is 0 while top_ids/top_logprobs are given"), 1;
    if (out->top_logprobs && !out->top_ids) return set_err(err, errlen, "top_logprobs needs top_ids"), 1;
    if (out->top_stride > TSM_MAX_LOGPROBS && (out->top_ids || out->top_logprobs))
        return set_err(err, errlen, "top_stride %u exceeds TSM_MAX_LOGPROBS", out->top_stride), 1;
    if (check_batch(kStaticMaxRows, TSM_MAX_VOCAB, batch, err, errlen)) return 1;
    int dev = -1;
    void* base = nullptr;
    if (static_setup(&dev, &base, err, errlen)) return 1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    unsigned char* p = static_cast<unsigned char*>(base);
    uint32_t* st = status ? status : reinterpret_cast<uint32_t*>(p + kStaticSplitBytes);
    // the split kernel takes batches the scratch holds; others go whole
    const bool fits = batch->rows <= kStaticRows && batch->usable <= kStaticVocab;
    tsm::split::SplitScratch w = tsm::split::scratch_carve(p, kStaticRows, kStaticVocab);
    // what must start at 0: the row counters (a previous call returned them
    // to 0 unless it was cut short) and the status word
    hipLaunchKernelGGL(clear_words, dim3(1), dim3(256), 0, s, reinterpret_cast<uint32_t*>(w.row_ctr), 2u * kStaticRows);
    hipLaunchKernelGGL(clear_words, dim3(1), dim3(64), 0, s, st, 1u);
    return queue(s, batch, out, nullptr, nullptr, 0, nullptr, false, st, fits ? &w : nullptr, err, errlen);
}

}  // extern "C"
