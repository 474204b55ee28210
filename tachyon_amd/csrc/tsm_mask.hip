// tsm_mask.hip - the mask producer: JsonObject's allows() for every token of
// the vocabulary, on the GPU, written as the packed allow-bits that
// sample_kernel and split_kernel consume (tsm_batch.mask).
//
// One thread per token and a group of rows: the workgroup stages its 256
// tokens' bytes in LDS, then per row each thread copies the row's 12-byte
// automaton state into registers and steps it through its token's bytes until
// the first rejected byte (tsm_json.h).  A wave's 64 answers become two mask
// words by one ballot, so every word of a row's mask is written exactly once,
// coalesced, with no atomics.  Most tokens are rejected at their first byte
// outside strings (only a few bytes can follow a value, a key or a colon), so
// the work is about one load of the token's offsets and a few bytes per
// token; inside a string most tokens are walked to their end.
//
// A mask set (tsm_json_masks_*) evaluates each distinct state of a call once
// and keeps recent states' masks in device memory: the evaluation writes a
// state's mask into its slot (and its first row), and a copy kernel fills the
// other rows from there.  The host keeps the index (state -> slot, least
// recently used out first), so no lookup waits for the GPU.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <list>
#include <unordered_map>
#include <vector>

#include "tsm_device.h"
#include "tsm_json.h"

namespace tsm {
namespace mask {

constexpr int kMB = 256;             // threads per workgroup: 256 consecutive tokens
constexpr uint32_t kRowsPer = 32;    // rows per workgroup at most: the staged bytes serve each
constexpr uint32_t kFillGroups = 2048;  // workgroups a launch aims for (few rows: fewer rows per workgroup)
constexpr uint32_t kStage = 16384;   // LDS bytes for the workgroup's tokens

struct JsonMaskArgs {
    const uint8_t* bytes;
    const uint32_t* offsets;
    const uint32_t* special;
    const tsm_json_state* states;
    uint32_t* mask;
    // per-row destinations (mask sets): row r's words go to dst0[r] and, when
    // it is not 0, to dst1[r] as well; without dst0, row r is mask + r*stride
    const uint64_t* dst0;
    const uint64_t* dst1;
    uint32_t n_tokens, usable, mask_stride, nwords, rows;
    uint32_t rows_per;  // rows per workgroup, <= kRowsPer
};

// Rows per workgroup for `rows` rows over `blocks` token blocks: as many as
// keep about kFillGroups workgroups busy, at most kRowsPer.
inline uint32_t rows_per_group(uint32_t rows, uint32_t blocks) {
    const uint32_t want_y = (kFillGroups + blocks - 1) / blocks;
    const uint32_t gy = want_y < rows ? want_y : rows;
    const uint32_t rp = (rows + gy - 1) / gy;
    return rp < kRowsPer ? rp : kRowsPer;
}

// Workgroup (token block, row group): the block's token bytes are one
// contiguous range of the vocabulary's bytes, staged into LDS with coalesced
// loads once and then stepped through for each of the group's rows (a block
// whose bytes exceed the stage reads them from global memory instead).
__global__ __launch_bounds__(kMB) void json_mask_kernel(JsonMaskArgs a) {
    __shared__ uint8_t stage[kStage];
    const uint32_t tid = threadIdx.x;
    const uint32_t t0 = blockIdx.x * kMB;
    const uint32_t id = t0 + tid;
    const uint32_t lim = a.usable < a.n_tokens ? a.usable : a.n_tokens;  // ids with bytes that count
    const uint32_t tend = t0 + kMB < lim ? t0 + kMB : lim;
    bool has = false;
    uint32_t b0 = 0, b1 = 0;
    if (id < lim) {
        b0 = a.offsets[id];
        b1 = a.offsets[id + 1u];
        const bool special = a.special != nullptr && ((a.special[id >> 5] >> (id & 31u)) & 1u);
        has = !special && b1 > b0;
    }
    uint32_t lo = 0, hi = 0;
    if (t0 < tend) {
        lo = a.offsets[t0];
        hi = a.offsets[tend];
    }
    const bool staged = hi >= lo && hi - lo <= kStage;
    if (staged) {
        for (uint32_t k = tid; k < hi - lo; k += kMB) stage[k] = a.bytes[lo + k];
        __syncthreads();
    }
    // a token's bytes lie inside [lo, hi) when the offsets are ordered; a
    // token outside it is read from global memory
    const bool mine_staged = staged && b0 >= lo && b1 <= hi;
    const uint8_t* src = mine_staged ? stage + (b0 - lo) : a.bytes + b0;
    const uint32_t len = b1 - b0;
    // a token of string text only (no '"', no '\\', no control byte) is
    // accepted whole inside a string with no escape pending: found once here
    // for all the group's rows
    bool plain = has;
    for (uint32_t k = 0; plain && k < len; k++) {
        const uint8_t c = src[k];
        plain = c >= 0x20 && c != '"' && c != '\\';
    }
    const uint32_t lane = lane_id();
    const uint32_t w = (t0 + (tid & ~(kWave - 1u))) / 32u + lane;  // lanes 0, 1: the wave's words
    const uint32_t r0 = blockIdx.y * a.rows_per;
    // a mask set's states and destinations sit in mapped host memory: the
    // group's are read once, in parallel, into LDS
    __shared__ tsm_json_state g_st[kRowsPer];
    __shared__ uint64_t g_d0[kRowsPer], g_d1[kRowsPer];
    if (a.dst0 != nullptr) {
        if (tid < a.rows_per && r0 + tid < a.rows) {
            g_st[tid] = a.states[r0 + tid];
            g_d0[tid] = a.dst0[r0 + tid];
            g_d1[tid] = a.dst1[r0 + tid];
        }
        __syncthreads();
    }
    for (uint32_t r = r0; r < r0 + a.rows_per && r < a.rows; r++) {
        const tsm_json_state st = a.dst0 ? g_st[r - r0] : a.states[r];
        const bool in_text = st.state == json::JS_STR && st.aux <= 1u;
        const bool ok = has && ((in_text && plain) || json::accepts(st, src, len));
        const uint64_t b = wave_ballot(ok);
        if (lane < 2u && w < a.nwords) {
            const uint32_t word = static_cast<uint32_t>(lane ? (b >> 32) : b);
            if (a.dst0 == nullptr) {
                a.mask[static_cast<size_t>(r) * a.mask_stride + w] = word;
            } else {
                reinterpret_cast<uint32_t*>(g_d0[r - r0])[w] = word;
                if (g_d1[r - r0] != 0u) reinterpret_cast<uint32_t*>(g_d1[r - r0])[w] = word;
            }
        }
    }
}

// Copies of whole mask rows (nwords words each): copy c reads src[c] and
// writes dst[c] (the pointers in mapped host memory, read once per
// workgroup); 256 threads of a workgroup take 1024 consecutive words.
constexpr uint32_t kCopyWords = 1024;
__global__ __launch_bounds__(kMB) void mask_copy_kernel(const uint64_t* src, const uint64_t* dst, uint32_t nwords) {
    __shared__ uint64_t ptr[2];
    if (threadIdx.x < 2u) ptr[threadIdx.x] = threadIdx.x ? dst[blockIdx.y] : src[blockIdx.y];
    __syncthreads();
    const uint32_t* s = reinterpret_cast<const uint32_t*>(ptr[0]);
    uint32_t* d = reinterpret_cast<uint32_t*>(ptr[1]);
    const uint32_t w0 = blockIdx.x * kCopyWords + threadIdx.x;
    uint32_t v[kCopyWords / kMB];
#pragma unroll
    for (uint32_t k = 0; k < kCopyWords / kMB; k++) {
        const uint32_t w = w0 + k * kMB;
        v[k] = w < nwords ? s[w] : 0u;
    }
#pragma unroll
    for (uint32_t k = 0; k < kCopyWords / kMB; k++) {
        const uint32_t w = w0 + k * kMB;
        if (w < nwords) d[w] = v[k];
    }
}

void set_err(char* err, size_t errlen, const char* fmt, ...) {
    if (!err || errlen == 0) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, errlen, fmt, ap);
    va_end(ap);
}

const char* vocab_error(const tsm_vocab* vocab) {
    if (!vocab) return "vocab is NULL";
    if (vocab->reserved != 0) return "vocab->reserved must be 0";
    if (vocab->n_tokens > 0 && (!vocab->bytes || !vocab->offsets))
        return "vocab->bytes and vocab->offsets must be set when n_tokens > 0";
    return nullptr;
}

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        (void)hipSetDevice(dev);
    }
    ~DeviceGuard() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

// A state's identity: its meaningful fields (the padding is left out).
struct Key {
    uint32_t w[3];
    bool operator==(const Key& o) const { return w[0] == o.w[0] && w[1] == o.w[1] && w[2] == o.w[2]; }
};
struct KeyHash {
    size_t operator()(const Key& k) const {
        uint64_t h = 0x9E3779B97F4A7C15ull;
        for (uint32_t x : k.w) h = (h ^ x) * 0xBF58476D1CE4E5B9ull;
        return static_cast<size_t>(h ^ (h >> 31));
    }
};
inline Key key_of(const tsm_json_state& s) {
    Key k;
    k.w[0] = s.stack;
    k.w[1] = uint32_t(s.depth) | uint32_t(s.state) << 8 | uint32_t(s.aux) << 16 | uint32_t(s.len) << 24;
    k.w[2] = s.whitespace;
    return k;
}

// Staging of one call in pinned, mapped host memory, read by the kernels
// over the bus (no upload step): the states to evaluate, their destinations,
// and the row copies.  Two halves take the calls in turn, so a call only
// waits for the kernels of the call before the last.
struct Stage {
    tsm_json_state* states;
    uint64_t *dst0, *dst1, *csrc, *cdst;
};
inline size_t stage_bytes(uint32_t rows) {
    const size_t st = (static_cast<size_t>(rows) * sizeof(tsm_json_state) + 255u) & ~size_t(255);
    return st + 4u * ((static_cast<size_t>(rows) * 8u + 255u) & ~size_t(255));
}
inline Stage stage_at(uint8_t* base, uint32_t rows) {
    const size_t st = (static_cast<size_t>(rows) * sizeof(tsm_json_state) + 255u) & ~size_t(255);
    const size_t pw = (static_cast<size_t>(rows) * 8u + 255u) & ~size_t(255);
    Stage s;
    s.states = reinterpret_cast<tsm_json_state*>(base);
    s.dst0 = reinterpret_cast<uint64_t*>(base + st);
    s.dst1 = reinterpret_cast<uint64_t*>(base + st + pw);
    s.csrc = reinterpret_cast<uint64_t*>(base + st + 2 * pw);
    s.cdst = reinterpret_cast<uint64_t*>(base + st + 3 * pw);
    return s;
}

}  // namespace mask
}  // namespace tsm

// The mask set behind tsm_json_masks_*: device memory for `capacity` masks
// (one slot per state, least recently used first out), the staging, and the
// host-side index of which state each slot holds.
struct tsm_json_masks {
    int device = 0;
    uint32_t max_rows = 0, capacity = 0, usable = 0, nwords = 0, slot_words = 0;
    uint32_t* cache = nullptr;   // capacity * slot_words words
    uint8_t* hstage = nullptr;   // pinned host memory: 2 halves of stage_bytes(max_rows)
    uint8_t* dstage = nullptr;   // the same memory's device address
    size_t half_bytes = 0;
    int half = 0;
    hipEvent_t used[2] = {nullptr, nullptr};  // recorded after the kernels that read each half
    bool pending[2] = {false, false};
    hipEvent_t done = nullptr;
    bool called = false;
    // the vocabulary the slots were evaluated over
    const void* v_bytes = nullptr;
    const void* v_offsets = nullptr;
    const void* v_special = nullptr;
    uint32_t v_n = 0;
    uint64_t call = 0;
    std::unordered_map<tsm::mask::Key, uint32_t, tsm::mask::KeyHash> where;
    std::vector<tsm::mask::Key> slot_key;
    std::vector<uint64_t> slot_call;  // the last call that used the slot; 0 = free
    std::list<uint32_t> lru;          // front: most recently used
    std::vector<std::list<uint32_t>::iterator> lru_at;

    uint64_t slot_addr(uint32_t s) const {
        return reinterpret_cast<uint64_t>(cache + static_cast<size_t>(s) * slot_words);
    }
    void flush() {
        where.clear();
        for (auto& c : slot_call) c = 0;
    }
    void touch(uint32_t s) {
        lru.splice(lru.begin(), lru, lru_at[s]);
        slot_call[s] = call;
    }
    // A slot for a new state: a free one, else the least recently used one
    // that this call has not used; -1 when every slot serves this call.
    int take() {
        const uint32_t s = lru.back();
        if (slot_call[s] == call) return -1;
        if (slot_call[s] != 0) where.erase(slot_key[s]);
        touch(s);
        return static_cast<int>(s);
    }
};

extern "C" {

void tsm_json_init(tsm_json_state* s) {
    if (s) tsm::json::init(s);
}

void tsm_json_advance(tsm_json_state* s, const uint8_t* bytes, size_t n) {
    if (!s || (!bytes && n)) return;
    for (size_t i = 0; i < n; i++) (void)tsm::json::step(*s, bytes[i]);  // advance ignores rejections
}

int tsm_json_accepts(const tsm_json_state* s, const uint8_t* bytes, size_t n) {
    if (!s || (!bytes && n)) return 0;
    tsm_json_state c = *s;
    for (size_t i = 0; i < n; i++)
        if (!tsm::json::step(c, bytes[i])) return 0;
    return 1;
}

int tsm_json_is_complete(const tsm_json_state* s) { return s && s->state == tsm::json::JS_DONE ? 1 : 0; }

int tsm_json_mask(void* stream, const tsm_vocab* vocab, const tsm_json_state* states, uint32_t rows,
                  uint32_t usable, uint32_t* mask, uint32_t mask_stride, char* err, size_t errlen) {
    using tsm::mask::set_err;
    if (const char* ve = tsm::mask::vocab_error(vocab)) return set_err(err, errlen, "%s", ve), 1;
    if (!states) return set_err(err, errlen, "states is NULL"), 1;
    if (!mask) return set_err(err, errlen, "mask is NULL"), 1;
    if (rows == 0 || rows > 65535u) return set_err(err, errlen, "rows %u is outside [1, 65535]", rows), 1;
    if (usable == 0 || usable > TSM_MAX_VOCAB)
        return set_err(err, errlen, "usable %u is outside [1, %u]", usable, TSM_MAX_VOCAB), 1;
    const uint32_t nwords = (usable + 31u) / 32u;
    if (mask_stride < nwords)
        return set_err(err, errlen, "mask_stride %u is below ceil(usable / 32) = %u", mask_stride, nwords), 1;
    tsm::mask::JsonMaskArgs a;
    a.bytes = vocab->bytes;
    a.offsets = vocab->offsets;
    a.special = vocab->special;
    a.states = states;
    a.mask = mask;
    a.dst0 = nullptr;
    a.dst1 = nullptr;
    a.n_tokens = vocab->n_tokens;
    a.usable = usable;
    a.mask_stride = mask_stride;
    a.nwords = nwords;
    a.rows = rows;
    const uint32_t blocks = (usable + tsm::mask::kMB - 1) / tsm::mask::kMB;
    a.rows_per = tsm::mask::rows_per_group(rows, blocks);
    const dim3 grid(blocks, (rows + a.rows_per - 1) / a.rows_per);
    hipLaunchKernelGGL(tsm::mask::json_mask_kernel, grid, dim3(tsm::mask::kMB), 0,
                       static_cast<hipStream_t>(stream), a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_err(err, errlen, "launch failed: %s", hipGetErrorString(e)), 1;
    return 0;
}

void tsm_json_masks_destroy(tsm_json_masks* m) {
    if (!m) return;
    tsm::mask::DeviceGuard g(m->device);
    if (m->done && m->called) (void)hipEventSynchronize(m->done);
    for (int h = 0; h < 2; h++)
        if (m->used[h]) (void)hipEventDestroy(m->used[h]);
    if (m->done) (void)hipEventDestroy(m->done);
    if (m->cache) (void)hipFree(m->cache);
    if (m->hstage) (void)hipHostFree(m->hstage);
    delete m;
}

tsm_json_masks* tsm_json_masks_create(int device, uint32_t max_rows, uint32_t capacity, uint32_t usable, char* err,
                                      size_t errlen) {
    using tsm::mask::set_err;
    if (max_rows == 0 || max_rows > 65535u) return set_err(err, errlen, "max_rows %u is outside [1, 65535]", max_rows), nullptr;
    if (capacity > 65536u) return set_err(err, errlen, "capacity %u is above 65536", capacity), nullptr;
    if (usable == 0 || usable > TSM_MAX_VOCAB)
        return set_err(err, errlen, "usable %u is outside [1, %u]", usable, TSM_MAX_VOCAB), nullptr;
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev)
        return set_err(err, errlen, "device %d is not a visible GPU", device), nullptr;
    tsm::mask::DeviceGuard g(device);
    tsm_json_masks* m = new tsm_json_masks();
    m->device = device;
    m->max_rows = max_rows;
    m->capacity = capacity;
    m->usable = usable;
    m->nwords = (usable + 31u) / 32u;
    m->slot_words = (m->nwords + 63u) & ~63u;  // slots start on 256-byte boundaries
    m->half_bytes = tsm::mask::stage_bytes(max_rows);
    hipError_t e = hipSuccess;
    if (capacity > 0) e = hipMalloc(&m->cache, static_cast<size_t>(capacity) * m->slot_words * 4u);
    if (e == hipSuccess)
        e = hipHostMalloc(reinterpret_cast<void**>(&m->hstage), 2 * m->half_bytes, hipHostMallocMapped);
    if (e == hipSuccess) e = hipHostGetDevicePointer(reinterpret_cast<void**>(&m->dstage), m->hstage, 0);
    for (int h = 0; h < 2 && e == hipSuccess; h++) e = hipEventCreateWithFlags(&m->used[h], hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&m->done, hipEventDisableTiming);
    if (e != hipSuccess) {
        set_err(err, errlen, "device setup failed: %s", hipGetErrorString(e));
        tsm_json_masks_destroy(m);
        return nullptr;
    }
    m->slot_key.resize(capacity);
    m->slot_call.assign(capacity, 0);
    m->lru_at.resize(capacity);
    for (uint32_t s = 0; s < capacity; s++) m->lru_at[s] = m->lru.insert(m->lru.end(), s);
    return m;
}

void tsm_json_masks_reset(tsm_json_masks* m) {
    if (m) m->flush();
}

int tsm_json_masks_fill(tsm_json_masks* m, void* stream, const tsm_vocab* vocab, const tsm_json_state* states,
                        uint32_t rows, uint32_t* mask, uint32_t mask_stride, tsm_json_fill_stats* stats, char* err,
                        size_t errlen) {
    using tsm::mask::set_err;
    if (!m) return set_err(err, errlen, "mask set is NULL"), 1;
    if (const char* ve = tsm::mask::vocab_error(vocab)) return set_err(err, errlen, "%s", ve), 1;
    if (!states) return set_err(err, errlen, "states is NULL"), 1;
    if (!mask) return set_err(err, errlen, "mask is NULL"), 1;
    if (rows == 0 || rows > m->max_rows)
        return set_err(err, errlen, "rows %u is outside [1, %u] (the set's max_rows)", rows, m->max_rows), 1;
    if (mask_stride < m->nwords)
        return set_err(err, errlen, "mask_stride %u is below ceil(usable / 32) = %u", mask_stride, m->nwords), 1;
    tsm::mask::DeviceGuard g(m->device);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    m->call++;
    if (vocab->bytes != m->v_bytes || vocab->offsets != m->v_offsets || vocab->special != m->v_special ||
        vocab->n_tokens != m->v_n) {
        m->flush();  // the slots hold another vocabulary's masks
        m->v_bytes = vocab->bytes;
        m->v_offsets = vocab->offsets;
        m->v_special = vocab->special;
        m->v_n = vocab->n_tokens;
    }
    const int h = m->half;
    m->half ^= 1;
    if (m->pending[h]) {  // the kernels that last read this half are done
        const hipError_t e = hipEventSynchronize(m->used[h]);
        if (e != hipSuccess) return set_err(err, errlen, "waiting for the staging failed: %s", hipGetErrorString(e)), 1;
        m->pending[h] = false;
    }
    uint8_t* hbase = m->hstage + h * m->half_bytes;
    uint8_t* dbase = m->dstage + h * m->half_bytes;
    const tsm::mask::Stage hs = tsm::mask::stage_at(hbase, m->max_rows);
    const tsm::mask::Stage ds = tsm::mask::stage_at(dbase, m->max_rows);
    // this call's states: where each one's mask will be (a slot, or the
    // first row that holds it)
    std::unordered_map<tsm::mask::Key, uint64_t, tsm::mask::KeyHash> src;
    src.reserve(rows * 2u);
    uint32_t jobs = 0, copies = 0, hits = 0, distinct = 0;
    for (uint32_t r = 0; r < rows; r++) {
        const tsm::mask::Key k = tsm::mask::key_of(states[r]);
        const uint64_t out = reinterpret_cast<uint64_t>(mask + static_cast<size_t>(r) * mask_stride);
        const auto seen = src.find(k);
        if (seen != src.end()) {
            hs.csrc[copies] = seen->second;
            hs.cdst[copies++] = out;
            continue;
        }
        distinct++;
        const auto cached = m->where.find(k);
        if (cached != m->where.end()) {
            m->touch(cached->second);
            hits++;
            const uint64_t a = m->slot_addr(cached->second);
            src.emplace(k, a);
            hs.csrc[copies] = a;
            hs.cdst[copies++] = out;
            continue;
        }
        tsm_json_state st = states[r];
        std::memset(st.pad, 0, sizeof(st.pad));
        hs.states[jobs] = st;
        const int slot = m->capacity ? m->take() : -1;
        if (slot >= 0) {
            m->slot_key[slot] = k;
            m->where.emplace(k, static_cast<uint32_t>(slot));
            const uint64_t a = m->slot_addr(static_cast<uint32_t>(slot));
            hs.dst0[jobs] = a;
            hs.dst1[jobs++] = out;
            src.emplace(k, a);
        } else {
            hs.dst0[jobs] = out;
            hs.dst1[jobs++] = 0u;
            src.emplace(k, out);
        }
    }
    if (jobs > 0) {
        tsm::mask::JsonMaskArgs a;
        a.bytes = vocab->bytes;
        a.offsets = vocab->offsets;
        a.special = vocab->special;
        a.states = ds.states;
        a.mask = nullptr;
        a.dst0 = ds.dst0;
        a.dst1 = ds.dst1;
        a.n_tokens = vocab->n_tokens;
        a.usable = m->usable;
        a.mask_stride = 0;
        a.nwords = m->nwords;
        a.rows = jobs;
        const uint32_t blocks = (m->usable + tsm::mask::kMB - 1) / tsm::mask::kMB;
        a.rows_per = tsm::mask::rows_per_group(jobs, blocks);
        const dim3 grid(blocks, (jobs + a.rows_per - 1) / a.rows_per);
        hipLaunchKernelGGL(tsm::mask::json_mask_kernel, grid, dim3(tsm::mask::kMB), 0, s, a);
    }
    if (copies > 0) {
        const dim3 grid((m->nwords + tsm::mask::kCopyWords - 1) / tsm::mask::kCopyWords, copies);
        hipLaunchKernelGGL(tsm::mask::mask_copy_kernel, grid, dim3(tsm::mask::kMB), 0, s,
                           static_cast<const uint64_t*>(ds.csrc), static_cast<const uint64_t*>(ds.cdst), m->nwords);
    }
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipEventRecord(m->used[h], s);
    if (e == hipSuccess) e = hipEventRecord(m->done, s);
    if (e != hipSuccess) return set_err(err, errlen, "launch failed: %s", hipGetErrorString(e)), 1;
    m->pending[h] = true;
    m->called = true;
    if (stats) {
        stats->rows = rows;
        stats->distinct = distinct;
        stats->hits = hits;
        stats->evaluated = jobs;
    }
    return 0;
}

}  // extern "C"
