// emu_runtime.cpp - launch engine and runtime calls of the CPU HIP emulation
// (tests/emu/include/hip/hip_runtime.h).  TEST INFRASTRUCTURE ONLY.
#include <hip/hip_runtime.h>
#include <pthread.h>
#include <ucontext.h>

#include <algorithm>
#if defined(__SANITIZE_ADDRESS__)
#include <sanitizer/common_interface_defs.h>
#endif

#include <condition_variable>
#include <memory>
#include <mutex>
#include <vector>

static size_t g_max_dyn = 64 * 1024;  // hipFuncSetAttribute raises it

#ifdef EMU_THREADS
namespace emu {

thread_local dim3 t_threadIdx, t_blockIdx;
dim3 g_blockDim, g_gridDim;

namespace {

[[noreturn]] void die(const char* msg) {
    std::fprintf(stderr, "EMU FATAL: %s\n", msg);
    std::fflush(stderr);
    std::abort();
}

// Counting barrier whose membership can shrink (threads that left the kernel).
struct Barrier {
    std::mutex m;
    std::condition_variable cv;
    int live = 0, arrived = 0;
    uint64_t gen = 0;
    const char* file = nullptr;
    int line = 0;
    bool check_site = false;

    void reset(int n) {
        std::lock_guard<std::mutex> lk(m);
        live = n;
        arrived = 0;
        file = nullptr;
    }
    void release_locked() {
        arrived = 0;
        file = nullptr;
        gen++;
        cv.notify_all();
    }
    void wait(const char* f, int l) {
        std::unique_lock<std::mutex> lk(m);
        if (check_site) {
            if (arrived == 0) {
                file = f;
                line = l;
            } else if (l != line || std::strcmp(f, file) != 0) {
                std::fprintf(stderr, "EMU: divergent __syncthreads: %s:%d vs %s:%d (block %u,%u thread %u)\n", f, l,
                             file, line, t_blockIdx.x, t_blockIdx.y, t_threadIdx.x);
                die("divergent barrier");
            }
        }
        const uint64_t g = gen;
        if (++arrived == live) {
            release_locked();
        } else {
            cv.wait(lk, [&] { return gen != g; });
        }
    }
    void drop() {
        std::lock_guard<std::mutex> lk(m);
        live--;
        if (arrived > 0 && arrived == live) release_locked();
    }
};

struct Launch {
    dim3 grid, block;
    size_t smem = 0;
    const Body* body = nullptr;
    unsigned char* dyn = nullptr;
    Barrier block_bar;               // __syncthreads
    std::vector<std::unique_ptr<Barrier>> wave_bar;
    std::vector<std::vector<uint64_t>> slots;
    Barrier pool_bar;                // between blocks
};

Launch* g_launch = nullptr;
thread_local int t_flat = 0;
thread_local int t_bank = 0;

void* worker(void* arg) {
    Launch& L = *g_launch;
    const int flat = static_cast<int>(reinterpret_cast<intptr_t>(arg));
    t_flat = flat;
    const uint32_t bx = L.block.x, by = L.block.y;
    t_threadIdx = dim3(flat % bx, (flat / bx) % by, flat / (bx * by));
    const int wave = flat / 64;
    for (uint32_t gz = 0; gz < L.grid.z; gz++)
        for (uint32_t gy = 0; gy < L.grid.y; gy++)
            for (uint32_t gx = 0; gx < L.grid.x; gx++) {
                t_blockIdx = dim3(gx, gy, gz);
                t_bank = 0;
                (*L.body)();
                L.block_bar.drop();
                L.wave_bar[wave]->drop();
                L.pool_bar.wait("pool", 0);
                if (flat == 0) {
                    const int nt = static_cast<int>(L.block.x * L.block.y * L.block.z);
                    L.block_bar.reset(nt);
                    for (size_t w = 0; w < L.wave_bar.size(); w++) {
                        const int left = nt - static_cast<int>(w) * 64;
                        L.wave_bar[w]->reset(left < 64 ? left : 64);
                    }
                    if (L.dyn) std::memset(L.dyn, 0xCD, L.smem);
                }
                L.pool_bar.wait("pool", 1);
            }
    return nullptr;
}

}  // namespace

unsigned char* dyn_smem() { return g_launch->dyn; }
void syncthreads(const char* file, int line) { g_launch->block_bar.wait(file, line); }
void wave_sync() { g_launch->wave_bar[t_flat / 64]->wait("wave", 0); }
uint64_t* wave_slots() { return g_launch->slots[t_flat / 64].data(); }
int next_bank() {
    const int b = t_bank;
    t_bank ^= 1;
    return b;
}
int lane_id() { return t_flat & 63; }

void run_launch(dim3 grid, dim3 block, size_t smem, const Body& body) {
    const int nt = static_cast<int>(block.x * block.y * block.z);
    if (nt <= 0 || nt > 1024) die("block size out of range");
    if (smem > 160 * 1024) die("dynamic shared memory above 160 KiB");
    if (smem > g_max_dyn) die("dynamic shared memory above the kernel's attribute (hipFuncSetAttribute)");
    if (grid.x == 0 || grid.y == 0 || grid.z == 0) die("empty grid");
    Launch L;
    L.grid = grid;
    L.block = block;
    L.smem = smem;
    L.body = &body;
    if (smem) {
        L.dyn = static_cast<unsigned char*>(std::malloc(smem));
        std::memset(L.dyn, 0xCD, smem);
    }
    L.block_bar.check_site = true;
    L.block_bar.reset(nt);
    L.pool_bar.reset(nt);
    const int nw = (nt + 63) / 64;
    for (int w = 0; w < nw; w++) {
        L.wave_bar.emplace_back(new Barrier());
        const int left = nt - w * 64;
        L.wave_bar.back()->reset(left < 64 ? left : 64);
        L.slots.emplace_back(128, 0);
    }
    g_blockDim = block;
    g_gridDim = grid;
    g_launch = &L;
    std::vector<pthread_t> th(nt);
    pthread_attr_t attr;
    pthread_attr_init(&attr);
    pthread_attr_setstacksize(&attr, 1 << 20);
    for (int i = 0; i < nt; i++)
        if (pthread_create(&th[i], &attr, worker, reinterpret_cast<void*>(static_cast<intptr_t>(i))) != 0)
            die("pthread_create failed");
    for (int i = 0; i < nt; i++) pthread_join(th[i], nullptr);
    pthread_attr_destroy(&attr);
    g_launch = nullptr;
    std::free(L.dyn);
}

}  // namespace emu

#else
namespace emu {

EMU_TLS dim3 t_threadIdx, t_blockIdx;
dim3 g_blockDim, g_gridDim;

namespace {

[[noreturn]] void die(const char* msg) {
    std::fprintf(stderr, "EMU FATAL: %s\n", msg);
    std::fflush(stderr);
    std::abort();
}

// Fiber engine: every thread of a block is a ucontext fiber on this one OS
// thread.  A fiber runs until it reaches a barrier (block or wave) or returns;
// the scheduler releases a wave barrier once every live lane of the wave is
// at it, and the block barrier once every live thread is (checking they all
// reached the same source line).  Anything else is a deadlock and aborts.
enum State : uint8_t { RUN, AT_BLOCK, AT_WAVE, DONE };

struct Fiber {
    ucontext_t ctx;
    void* stack = nullptr;
    State st = RUN;
    int bank = 0;
    const char* file = nullptr;
    int line = 0;
};

constexpr size_t kStack = 256 * 1024;

struct Launch {
    dim3 grid, block;
    size_t smem = 0;
    const Body* body = nullptr;
    unsigned char* dyn = nullptr;
    std::vector<Fiber> fib;
    std::vector<std::vector<uint64_t>> slots;
    ucontext_t sched;
    int cur = -1;
};

Launch* g_launch = nullptr;
void* g_fake_stack = nullptr;

void switch_to_sched(Fiber& f) {
#if defined(__SANITIZE_ADDRESS__)
    __sanitizer_start_switch_fiber(&g_fake_stack, nullptr, 0);
#endif
    swapcontext(&f.ctx, &g_launch->sched);
#if defined(__SANITIZE_ADDRESS__)
    __sanitizer_finish_switch_fiber(g_fake_stack, nullptr, nullptr);
#endif
}

void fiber_entry() {
#if defined(__SANITIZE_ADDRESS__)
    __sanitizer_finish_switch_fiber(nullptr, nullptr, nullptr);
#endif
    Launch& L = *g_launch;
    (*L.body)();
    L.fib[L.cur].st = DONE;
#if defined(__SANITIZE_ADDRESS__)
    __sanitizer_start_switch_fiber(nullptr, nullptr, 0);  // this fiber ends
#endif
    setcontext(&L.sched);
}

void run_block(Launch& L) {
    const int nt = static_cast<int>(L.fib.size());
    for (int i = 0; i < nt; i++) {
        Fiber& f = L.fib[i];
        f.st = RUN;
        f.bank = 0;
        getcontext(&f.ctx);
        f.ctx.uc_stack.ss_sp = f.stack;
        f.ctx.uc_stack.ss_size = kStack;
        f.ctx.uc_link = nullptr;
        makecontext(&f.ctx, fiber_entry, 0);
    }
    const int nw = (nt + 63) / 64;
    for (;;) {
        bool any_run = false;
        for (int i = 0; i < nt; i++) {
            Fiber& f = L.fib[i];
            if (f.st != RUN) continue;
            any_run = true;
            L.cur = i;
            t_threadIdx = dim3(i % L.block.x, (i / L.block.x) % L.block.y, i / (L.block.x * L.block.y));
#if defined(__SANITIZE_ADDRESS__)
            void* fake = nullptr;
            __sanitizer_start_switch_fiber(&fake, f.stack, kStack);
#endif
            swapcontext(&L.sched, &f.ctx);
#if defined(__SANITIZE_ADDRESS__)
            __sanitizer_finish_switch_fiber(fake, nullptr, nullptr);
#endif
        }
        (void)any_run;
        // every fiber is now waiting or done
        bool released = false;
        for (int w = 0; w < nw; w++) {
            const int a = w * 64, b = std::min(nt, a + 64);
            bool all = true, some = false;
            for (int i = a; i < b; i++) {
                if (L.fib[i].st == DONE) continue;
                if (L.fib[i].st == AT_WAVE) some = true; else all = false;
            }
            if (some && all) {
                for (int i = a; i < b; i++)
                    if (L.fib[i].st == AT_WAVE) L.fib[i].st = RUN;
                released = true;
            }
        }
        if (released) continue;
        int live = 0, at_block = 0;
        const char* file = nullptr;
        int line = 0;
        for (int i = 0; i < nt; i++) {
            const Fiber& f = L.fib[i];
            if (f.st == DONE) continue;
            live++;
            if (f.st == AT_BLOCK) {
                at_block++;
                if (!file) {
                    file = f.file;
                    line = f.line;
                } else if (f.line != line || std::strcmp(f.file, file) != 0) {
                    std::fprintf(stderr, "EMU: divergent __syncthreads: %s:%d vs %s:%d (block %u,%u thread %d)\n",
                                 f.file, f.line, file, line, t_blockIdx.x, t_blockIdx.y, i);
                    die("divergent barrier");
                }
            }
        }
        if (live == 0) return;
        if (at_block == live) {
            for (int i = 0; i < nt; i++)
                if (L.fib[i].st == AT_BLOCK) L.fib[i].st = RUN;
            continue;
        }
        std::fprintf(stderr, "EMU: deadlock in block %u,%u: %d live, %d at the block barrier\n", t_blockIdx.x,
                     t_blockIdx.y, live, at_block);
        die("barrier deadlock (a wave waits on a shuffle while others wait at __syncthreads)");
    }
}

}  // namespace

unsigned char* dyn_smem() { return g_launch->dyn; }
void syncthreads(const char* file, int line) {
    Fiber& f = g_launch->fib[g_launch->cur];
    f.st = AT_BLOCK;
    f.file = file;
    f.line = line;
    switch_to_sched(f);
}
void wave_sync() {
    Fiber& f = g_launch->fib[g_launch->cur];
    f.st = AT_WAVE;
    switch_to_sched(f);
}
uint64_t* wave_slots() { return g_launch->slots[g_launch->cur / 64].data(); }
int next_bank() {
    Fiber& f = g_launch->fib[g_launch->cur];
    const int b = f.bank;
    f.bank ^= 1;
    return b;
}
int lane_id() { return g_launch->cur & 63; }

void run_launch(dim3 grid, dim3 block, size_t smem, const Body& body) {
    const int nt = static_cast<int>(block.x * block.y * block.z);
    if (nt <= 0 || nt > 1024) die("block size out of range");
    if (smem > 160 * 1024) die("dynamic shared memory above 160 KiB");
    if (smem > g_max_dyn) die("dynamic shared memory above the kernel's attribute (hipFuncSetAttribute)");
    if (grid.x == 0 || grid.y == 0 || grid.z == 0) die("empty grid");
    Launch L;
    L.grid = grid;
    L.block = block;
    L.smem = smem;
    L.body = &body;
    if (smem) L.dyn = static_cast<unsigned char*>(std::malloc(smem));
    L.fib.resize(nt);
    for (auto& f : L.fib) f.stack = std::malloc(kStack);
    L.slots.assign((nt + 63) / 64, std::vector<uint64_t>(128, 0));
    g_blockDim = block;
    g_gridDim = grid;
    g_launch = &L;
    for (uint32_t gz = 0; gz < grid.z; gz++)
        for (uint32_t gy = 0; gy < grid.y; gy++)
            for (uint32_t gx = 0; gx < grid.x; gx++) {
                t_blockIdx = dim3(gx, gy, gz);
                if (L.dyn) std::memset(L.dyn, 0xCD, smem);
                run_block(L);
            }
    g_launch = nullptr;
    for (auto& f : L.fib) std::free(f.stack);
    std::free(L.dyn);
}

}  // namespace emu

#endif

// ---- runtime calls ----

hipError_t hipMalloc(void** p, size_t n) {
    *p = std::aligned_alloc(256, ((n + 255) / 256) * 256 ? ((n + 255) / 256) * 256 : 256);
    if (!*p) return hipErrorOutOfMemory;
    std::memset(*p, 0xAB, n);
    return hipSuccess;
}
hipError_t hipFree(void* p) {
    std::free(p);
    return hipSuccess;
}
hipError_t hipMemset(void* p, int v, size_t n) {
    std::memset(p, v, n);
    return hipSuccess;
}
hipError_t hipMemsetAsync(void* p, int v, size_t n, hipStream_t) { return hipMemset(p, v, n); }
hipError_t hipMemcpy(void* d, const void* s, size_t n, hipMemcpyKind) {
    std::memcpy(d, s, n);
    return hipSuccess;
}
hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind k, hipStream_t) {
    return hipMemcpy(d, s, n, k);
}
hipError_t hipGetDeviceCount(int* n) {
    *n = 1;
    return hipSuccess;
}
hipError_t hipSetDevice(int d) { return d == 0 ? hipSuccess : hipErrorInvalidDevice; }
hipError_t hipGetDevice(int* d) {
    *d = 0;
    return hipSuccess;
}
hipError_t hipGetDeviceProperties(hipDeviceProp_t* p, int d) {
    if (d != 0) return hipErrorInvalidDevice;
    std::memset(p, 0, sizeof(*p));
    std::strcpy(p->name, "CPU emulation");
    std::strcpy(p->gcnArchName, "gfx950:sramecc+:xnack-");
    p->multiProcessorCount = 256;
    p->sharedMemPerBlock = 160 * 1024;
    return hipSuccess;
}
hipError_t hipDeviceSynchronize() { return hipSuccess; }
hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned) {
    *s = reinterpret_cast<hipStream_t>(std::malloc(16));
    return *s ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t hipStreamDestroy(hipStream_t s) {
    std::free(s);
    return hipSuccess;
}
hipError_t hipEventCreateWithFlags(hipEvent_t* e, unsigned) {
    *e = reinterpret_cast<hipEvent_t>(std::malloc(16));
    return *e ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t hipEventDestroy(hipEvent_t e) {
    std::free(e);
    return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t e, hipStream_t) { return e ? hipSuccess : hipErrorInvalidValue; }
hipError_t hipEventSynchronize(hipEvent_t e) { return e ? hipSuccess : hipErrorInvalidValue; }
hipError_t hipHostMalloc(void** p, size_t n, unsigned) {
    *p = std::malloc(n);
    return *p ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t hipHostGetDevicePointer(void** d, void* h, unsigned) {
    *d = h;
    return h ? hipSuccess : hipErrorInvalidValue;
}
hipError_t hipHostFree(void* p) {
    std::free(p);
    return hipSuccess;
}
hipError_t hipGetLastError() { return hipSuccess; }
const char* hipGetErrorString(hipError_t e) { return e == hipSuccess ? "hipSuccess" : "emulated HIP error"; }
hipError_t hipFuncSetAttribute(const void*, hipFuncAttribute a, int v) {
    if (a == hipFuncAttributeMaxDynamicSharedMemorySize) {
        if (v > 160 * 1024) return hipErrorInvalidValue;
        g_max_dyn = static_cast<size_t>(v);
    }
    return hipSuccess;
}
hipError_t hipGetSymbolAddress(void** p, const void* sym) {
    *p = const_cast<void*>(sym);
    return hipSuccess;
}
