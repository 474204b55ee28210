// hip_runtime.h - CPU emulation of the subset of HIP the sampling kernels use.
// TEST INFRASTRUCTURE ONLY: tests/emu builds the product kernel sources
// (tachyon_amd/csrc/*.hip) against this header with g++ and AddressSanitizer /
// UndefinedBehaviorSanitizer (or ThreadSanitizer), so that an out-of-bounds
// access, a misaligned vector load or a missing barrier shows up on the CPU
// instead of faulting a GPU.  Nothing in the product links this.
//
// Model: a launch runs its blocks one after another; the threads of a block
// are OS threads.  __syncthreads() is a block-wide barrier that also checks
// every live thread reached the same source line; a thread that returns from
// the kernel stops counting for the rest of its block (as an ended wave does
// on the GPU).  Shuffles exchange through a per-wave (64-lane) barrier.
// __shared__ variables are static (blocks never overlap); dynamic shared
// memory is a heap buffer of exactly the launch's size, refilled with 0xCD
// before each block, so an overrun is a heap overflow and a read of LDS that
// was never written sees garbage.
#pragma once

#include <atomic>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <tuple>
#include <utility>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __noinline__ __attribute__((noinline))
#define __launch_bounds__(...)
#define __shared__ static
#define __constant__ static
#define __align__(n) alignas(n)
#define HIP_DYNAMIC_SHARED(type, var) type* var = reinterpret_cast<type*>(::emu::dyn_smem());
#define __builtin_amdgcn_exp2f(x) exp2f(x)
#define __builtin_amdgcn_readlane(v, l) emu_shfl((v), (l))
#define __builtin_amdgcn_update_dpp(old, src, ctrl, rm, bm, bc) emu_dpp((old), (src), (ctrl), (rm), (bm), (bc))
#define __builtin_amdgcn_wave_barrier() ::emu::wave_sync()
#define HIP_SYMBOL(x) (&(x))
#define TSM_GLOBAL_AS
#define TSM_CONST_AS  // the host has one address space
#define TSM_HAVE_LOAD4

struct dim3 {
    uint32_t x, y, z;
    constexpr dim3(uint32_t x_ = 1, uint32_t y_ = 1, uint32_t z_ = 1) : x(x_), y(y_), z(z_) {}
};

struct alignas(16) float4 { float x, y, z, w; };
struct alignas(8) float2 { float x, y; };
struct alignas(8) uint2 { uint32_t x, y; };
struct alignas(16) uint4 { uint32_t x, y, z, w; };
inline uint2 make_uint2(uint32_t x, uint32_t y) { return uint2{x, y}; }
inline uint4 make_uint4(uint32_t x, uint32_t y, uint32_t z, uint32_t w) { return uint4{x, y, z, w}; }
inline float4 make_float4(float x, float y, float z, float w) { return float4{x, y, z, w}; }
inline float4 load4(const float* p) { return float4{p[0], p[1], p[2], p[3]}; }

namespace emu {
#ifdef EMU_THREADS
#define EMU_TLS thread_local
#else
#define EMU_TLS  // fibers share one OS thread; the scheduler sets these per switch
#endif
extern EMU_TLS dim3 t_threadIdx, t_blockIdx;
extern dim3 g_blockDim, g_gridDim;
unsigned char* dyn_smem();
void syncthreads(const char* file, int line);
void wave_sync();
uint64_t* wave_slots();
int next_bank();  // this lane's shuffle count parity, then advances it
int lane_id();
using Body = std::function<void()>;
void run_launch(dim3 grid, dim3 block, size_t smem, const Body& body);
}  // namespace emu

#define threadIdx (::emu::t_threadIdx)
#define blockIdx (::emu::t_blockIdx)
#define blockDim (::emu::g_blockDim)
#define gridDim (::emu::g_gridDim)
#define __syncthreads() ::emu::syncthreads(__FILE__, __LINE__)
// s_barrier: a block barrier (the kernels put their LDS fences around it)
#define __builtin_amdgcn_s_barrier() ::emu::syncthreads(__FILE__, __LINE__)

#include <type_traits>
template <class T, class U>
inline std::common_type_t<T, U> min(T a, U b) { return a < b ? a : b; }
template <class T, class U>
inline std::common_type_t<T, U> max(T a, U b) { return a > b ? a : b; }

inline uint32_t __float_as_uint(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
inline float __uint_as_float(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
inline int __float_as_int(float f) { int u; std::memcpy(&u, &f, 4); return u; }
inline float __int_as_float(int u) { float f; std::memcpy(&f, &u, 4); return f; }
inline long long __double_as_longlong(double d) { long long u; std::memcpy(&u, &d, 8); return u; }
inline double __longlong_as_double(long long u) { double d; std::memcpy(&d, &u, 8); return d; }
inline int __popc(uint32_t v) { return __builtin_popcount(v); }
inline uint32_t __builtin_amdgcn_ubfe(uint32_t v, uint32_t off, uint32_t w) {
    return w >= 32 ? v >> off : (v >> off) & ((1u << w) - 1u);
}
inline int __popcll(uint64_t v) { return __builtin_popcountll(v); }
inline int __clz(uint32_t v) { return v ? __builtin_clz(v) : 32; }
inline int __ffs(uint32_t v) { return __builtin_ffs(v); }

template <class T>
inline T emu_shfl(T v, int src) {
    static_assert(sizeof(T) <= 8, "shuffle of <= 8 bytes");
    // Two slot banks used alternately: a lane writes bank b only after the
    // wave's previous shuffle (bank b^1) released, and every lane finished
    // reading bank b two shuffles ago, so one wave barrier per shuffle is enough.
    uint64_t* slots = ::emu::wave_slots();
    const int lane = ::emu::lane_id();
    uint64_t bits = 0;
    std::memcpy(&bits, &v, sizeof(T));
    const int bank = ::emu::next_bank();
    slots[bank * 64 + lane] = bits;
    ::emu::wave_sync();
    T r;
    const uint64_t got = slots[bank * 64 + src];
    std::memcpy(&r, &got, sizeof(T));
    return r;
}
// DPP moves used by the kernels: row_shr:1..15 (0x111..0x11f) and the wave64
// row broadcasts row_bcast:15 (0x142) and row_bcast:31 (0x143).
inline int emu_dpp(int old, int src, int ctrl, int row_mask, int bank_mask, bool bound_ctrl) {
    const int lane = ::emu::lane_id();
    const int row = lane / 16, inrow = lane % 16;
    int from = -1;
    if (ctrl > 0x110 && ctrl <= 0x11f) {
        const int n = ctrl - 0x110;
        if (inrow >= n) from = lane - n;
    } else if (ctrl == 0x142) {
        if (row >= 1) from = (row - 1) * 16 + 15;
    } else if (ctrl == 0x143) {
        if (row >= 2) from = 31;
    } else {
        std::fprintf(stderr, "EMU: unsupported DPP control 0x%x\n", ctrl);
        std::abort();
    }
    const int got = emu_shfl(src, from < 0 ? lane : from);  // every lane takes part
    if (!((row_mask >> row) & 1) || !((bank_mask >> (inrow / 4)) & 1)) return old;
    if (from < 0) return bound_ctrl ? 0 : old;
    return got;
}

// Ballot over the 64 lanes of the wave (every lane must take part).
inline unsigned long long __ballot(int pred) {
    uint64_t* slots = ::emu::wave_slots();
    const int lane = ::emu::lane_id();
    const int bank = ::emu::next_bank();
    slots[bank * 64 + lane] = pred != 0;
    ::emu::wave_sync();
    unsigned long long m = 0;
    for (int i = 0; i < 64; i++)
        if (slots[bank * 64 + i]) m |= 1ull << i;
    return m;
}
// Used by the kernels only where the whole wave is active: lane 0 is the first.
#define __builtin_amdgcn_readfirstlane(v) emu_shfl((v), 0)
inline uint32_t __builtin_amdgcn_mbcnt_lo(uint32_t mask, uint32_t acc) {
    const int lane = ::emu::lane_id();
    const uint32_t below = lane >= 32 ? 0xFFFFFFFFu : ((1u << lane) - 1u);
    return acc + static_cast<uint32_t>(__builtin_popcount(mask & below));
}
inline uint32_t __builtin_amdgcn_mbcnt_hi(uint32_t mask, uint32_t acc) {
    const int lane = ::emu::lane_id();
    const uint32_t below = lane < 32 ? 0u : ((1ull << (lane - 32)) - 1ull);
    return acc + static_cast<uint32_t>(__builtin_popcount(mask & below));
}
#define __HIP_MEMORY_SCOPE_WORKGROUP 3
#define __HIP_MEMORY_SCOPE_AGENT 4
#define __builtin_amdgcn_s_waitcnt(n) ((void)(n))
inline std::memory_order emu_order(int order) {
    switch (order) {
        case __ATOMIC_RELAXED: return std::memory_order_relaxed;
        case __ATOMIC_ACQUIRE: return std::memory_order_acquire;
        case __ATOMIC_RELEASE: return std::memory_order_release;
        case __ATOMIC_ACQ_REL: return std::memory_order_acq_rel;
        default: return std::memory_order_seq_cst;
    }
}
// The kernels pair relaxed LDS atomics with LDS-only fences
// (__builtin_amdgcn_fence(..., "workgroup", "local")).  ThreadSanitizer does
// not model standalone fences, so here the fences are no-ops and every
// atomic load acquires and every atomic read-modify-write releases and
// acquires: the same orderings the fence + relaxed pairs give on the GPU.
#define __builtin_amdgcn_fence(...) ((void)0)
template <class T>
inline T __hip_atomic_load(T* p, int, int) {
    return std::atomic_ref<T>(*p).load(std::memory_order_acquire);
}
template <class T>
inline void __hip_atomic_store(T* p, T v, int, int) {
    std::atomic_ref<T>(*p).store(v, std::memory_order_release);
}
template <class T>
inline T __hip_atomic_fetch_add(T* p, T v, int, int) {
    return std::atomic_ref<T>(*p).fetch_add(v, std::memory_order_acq_rel);
}
template <class T>
inline T __hip_atomic_fetch_max(T* p, T v, int, int) {
    std::atomic_ref<T> a(*p);
    T old = a.load(std::memory_order_relaxed);
    while (!a.compare_exchange_weak(old, old > v ? old : v, std::memory_order_acq_rel, std::memory_order_relaxed)) {}
    return old;
}

// Device-scope fence: blocks run one after another here, so it only has to
// order this thread's own memory operations.
inline void __threadfence() { std::atomic_thread_fence(std::memory_order_seq_cst); }

template <class T>
inline T __shfl_xor(T v, int mask, int width = 64) {
    const int lane = ::emu::lane_id();
    int src = lane ^ mask;
    if ((src & ~(width - 1)) != (lane & ~(width - 1))) src = lane;
    return emu_shfl(v, src);
}
template <class T>
inline T __shfl_up(T v, unsigned delta, int width = 64) {
    const int lane = ::emu::lane_id();
    const int seg = lane & ~(width - 1);
    int src = lane - static_cast<int>(delta);
    if (src < seg) src = lane;
    return emu_shfl(v, src);
}
template <class T>
inline T __shfl_down(T v, unsigned delta, int width = 64) {
    const int lane = ::emu::lane_id();
    const int seg = lane & ~(width - 1);
    int src = lane + static_cast<int>(delta);
    if (src >= seg + width) src = lane;
    return emu_shfl(v, src);
}
template <class T>
inline T __shfl(T v, int src, int width = 64) {
    const int lane = ::emu::lane_id();
    return emu_shfl(v, (lane & ~(width - 1)) + (src & (width - 1)));
}

template <class T>
inline T atomicAdd(T* p, T v) { return std::atomic_ref<T>(*p).fetch_add(v); }
template <class T>
inline T atomicOr(T* p, T v) { return std::atomic_ref<T>(*p).fetch_or(v); }
template <class T>
inline T atomicAnd(T* p, T v) { return std::atomic_ref<T>(*p).fetch_and(v); }
template <class T>
inline T atomicExch(T* p, T v) { return std::atomic_ref<T>(*p).exchange(v); }
template <class T>
inline T atomicMin(T* p, T v) {
    std::atomic_ref<T> a(*p);
    T old = a.load();
    while (v < old && !a.compare_exchange_weak(old, v)) {}
    return old;
}
template <class T>
inline T atomicMax(T* p, T v) {
    std::atomic_ref<T> a(*p);
    T old = a.load();
    while (v > old && !a.compare_exchange_weak(old, v)) {}
    return old;
}
template <class T>
inline T atomicCAS(T* p, T cmp, T v) {
    std::atomic_ref<T>(*p).compare_exchange_strong(cmp, v);
    return cmp;
}

// ---- runtime ----
typedef enum hipError_t {
    hipSuccess = 0,
    hipErrorInvalidValue = 1,
    hipErrorOutOfMemory = 2,
    hipErrorInvalidDevice = 101,
    hipErrorLaunchFailure = 719,
} hipError_t;
typedef struct ihipStream_t* hipStream_t;
typedef struct ihipEvent_t* hipEvent_t;
constexpr unsigned hipEventDisableTiming = 2u;
constexpr unsigned hipStreamNonBlocking = 1u;
enum hipMemcpyKind { hipMemcpyHostToHost, hipMemcpyHostToDevice, hipMemcpyDeviceToHost, hipMemcpyDeviceToDevice,
                     hipMemcpyDefault };
enum hipFuncAttribute { hipFuncAttributeMaxDynamicSharedMemorySize = 8 };
struct hipDeviceProp_t {
    char name[256];
    char gcnArchName[256];
    int multiProcessorCount;
    size_t sharedMemPerBlock;
};

hipError_t hipMalloc(void** p, size_t n);
template <class T>
inline hipError_t hipMalloc(T** p, size_t n) { return hipMalloc(reinterpret_cast<void**>(p), n); }
hipError_t hipFree(void* p);
hipError_t hipMemset(void* p, int v, size_t n);
hipError_t hipMemsetAsync(void* p, int v, size_t n, hipStream_t s = nullptr);
hipError_t hipMemcpy(void* d, const void* s, size_t n, hipMemcpyKind k);
hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind k, hipStream_t st = nullptr);
hipError_t hipGetDeviceCount(int* n);
hipError_t hipSetDevice(int d);
hipError_t hipGetDevice(int* d);
hipError_t hipGetDeviceProperties(hipDeviceProp_t* p, int d);
hipError_t hipDeviceSynchronize();
hipError_t hipStreamSynchronize(hipStream_t s);
// streams and events: the emulation runs every launch to completion at once
hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned flags);
hipError_t hipStreamDestroy(hipStream_t s);
hipError_t hipEventCreateWithFlags(hipEvent_t* e, unsigned flags);
hipError_t hipEventDestroy(hipEvent_t e);
hipError_t hipEventRecord(hipEvent_t e, hipStream_t s = nullptr);
hipError_t hipEventSynchronize(hipEvent_t e);
hipError_t hipHostMalloc(void** p, size_t n, unsigned flags = 0);
#define hipHostMallocMapped 0x2u
// pinned host memory is the device's memory here: its device address is itself
hipError_t hipHostGetDevicePointer(void** d, void* h, unsigned flags);
hipError_t hipHostFree(void* p);
hipError_t hipGetLastError();
const char* hipGetErrorString(hipError_t e);
hipError_t hipFuncSetAttribute(const void* f, hipFuncAttribute a, int v);
hipError_t hipGetSymbolAddress(void** p, const void* sym);

template <class... KA, class... A>
inline void hipLaunchKernelGGL(void (*k)(KA...), dim3 grid, dim3 block, size_t smem, hipStream_t, A&&... args) {
    std::tuple<KA...> t(std::forward<A>(args)...);
    ::emu::run_launch(grid, block, smem, [k, t]() { std::apply(k, t); });
}
