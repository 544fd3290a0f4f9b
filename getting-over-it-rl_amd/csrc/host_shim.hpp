// host_shim.hpp - the HIP surface the step's sources use, for a sequential host build (GOI_HOST_BUILD).
//
// Compiled as C++ by the host compiler (with AddressSanitizer and UBSan in the tests), the step's sources run one
// lane per block (kBlock = 1): every world on a one-lane group, every block-cooperative pass on that lane, so the
// cross-lane operations below reduce to the lane's own value. Launches run their blocks one after another, each
// with its dynamic LDS in a heap buffer of exactly the launch's size, and the "device" allocations are host heap
// blocks of exactly the requested size: an access past a workspace, a row tile or a State leaf is a heap overflow
// the sanitizer reports with its source line. The device build never includes this file.
#pragma once

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#define __device__
#define __host__
#define __global__
#define __forceinline__ inline
#define __noinline__ __attribute__((noinline))
#define __shared__
#define __launch_bounds__(...)
#define __align__(n) alignas(n)

struct float2 { float x, y; };
struct float4 { float x, y, z, w; };
struct int2 { int x, y; };
struct int4 { int x, y, z, w; };
struct double2 { double x, y; };
struct double4 { double x, y, z, w; };
struct dim3 {
    unsigned x, y, z;
    dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};
inline float4 make_float4(float x, float y, float z, float w) { return float4{x, y, z, w}; }
inline int2 make_int2(int x, int y) { return int2{x, y}; }
inline int4 make_int4(int x, int y, int z, int w) { return int4{x, y, z, w}; }
inline double2 make_double2(double x, double y) { return double2{x, y}; }

inline unsigned __float_as_uint(float f) { unsigned u; std::memcpy(&u, &f, 4); return u; }
inline float __uint_as_float(unsigned u) { float f; std::memcpy(&f, &u, 4); return f; }
inline long long __double_as_longlong(double d) { long long u; std::memcpy(&u, &d, 8); return u; }
inline int __float_as_int(float f) { int u; std::memcpy(&u, &f, 4); return u; }
inline float __int_as_float(int u) { float f; std::memcpy(&f, &u, 4); return f; }
inline int __popcll(unsigned long long x) { return __builtin_popcountll(x); }
using std::fabs;
using std::isfinite;
using std::fma;
using std::rint;
using std::sqrt;
using std::max;
using std::min;
inline void sincos(double x, double* s, double* c) { *s = std::sin(x); *c = std::cos(x); }

// the launch position of the running "thread"
struct GoiHostIdx { unsigned x, y, z; };
inline thread_local GoiHostIdx threadIdx{0, 0, 0}, blockIdx{0, 0, 0}, blockDim{1, 1, 1}, gridDim{1, 1, 1};
inline thread_local int* goi_host_lds = nullptr;  // the running block's dynamic LDS

// one lane per group and per block: every exchange returns the lane's own value
inline void __syncthreads() {}
inline bool __any(bool p) { return p; }
template <typename T> inline T __shfl_xor(T v, int, int = 64) { return v; }
template <typename T> inline T __shfl_up(T v, unsigned, int = 64) { return v; }
template <typename T> inline T __shfl(T v, int, int = 64) { return v; }
#define __builtin_amdgcn_update_dpp(old, v, ctrl, rm, bm, bc) (v)
#define __builtin_amdgcn_fence(order, scope) ((void)0)
#define __builtin_nontemporal_load(p) (*(p))
#define __builtin_nontemporal_store(v, p) (*(p) = (v))

// the runtime API the library calls, on host memory
enum hipError_t { hipSuccess = 0, hipErrorMemoryAllocation = 2 };
typedef void* hipStream_t;
enum hipMemcpyKind { hipMemcpyHostToDevice = 1 };
enum hipDeviceAttribute_t { hipDeviceAttributeMultiprocessorCount = 0 };
inline const char* hipGetErrorString(hipError_t e) { return e == hipSuccess ? "no error" : "host build error"; }
inline hipError_t hipGetLastError() { return hipSuccess; }
inline hipError_t hipMalloc(void** p, size_t n) {
    *p = std::malloc(n ? n : 1);
    return *p ? hipSuccess : hipErrorMemoryAllocation;
}
template <typename T> inline hipError_t hipMalloc(T** p, size_t n) { return hipMalloc(reinterpret_cast<void**>(p), n); }
inline hipError_t hipFree(void* p) { std::free(p); return hipSuccess; }
inline hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind, hipStream_t) {
    if (n) std::memcpy(d, s, n);
    return hipSuccess;
}
inline hipError_t hipMemsetAsync(void* d, int v, size_t n, hipStream_t) {
    if (n) std::memset(d, v, n);
    return hipSuccess;
}
inline hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
inline hipError_t hipDeviceSynchronize() { return hipSuccess; }
inline hipError_t hipGetDevice(int* d) { *d = 0; return hipSuccess; }
inline hipError_t hipSetDevice(int) { return hipSuccess; }
inline hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t, int) { *v = 1; return hipSuccess; }
#define HIP_SYMBOL(x) (x)
template <typename T> inline hipError_t hipGetSymbolAddress(void** p, T& sym) { *p = (void*)&sym; return hipSuccess; }

// The word the host build fills scratch memory with before each launch (every block's dynamic LDS, and the constraint
// and task rows through goi_host_poison), so that a read of a word the launch has not written yields it instead of a
// leftover of an earlier launch: GOI_HOST_POISON = "nan" (a quiet NaN with payload 0xdead), an integer (say 8), or
// unset (zeros). A result that depends on such a read then differs from the oracle's.
inline bool goi_host_poison_word(int* word) {
    const char* e = std::getenv("GOI_HOST_POISON");
    if (!e || !*e) return false;
    *word = std::strcmp(e, "nan") == 0 ? 0x7fc0dead : std::atoi(e);
    return true;
}
inline void goi_host_poison(void* p, size_t bytes) {
    int word = 0;
    if (!p || !goi_host_poison_word(&word)) return;
    int* q = static_cast<int*>(p);
    for (size_t i = 0; i < bytes / sizeof(int); ++i) q[i] = word;
}

// a launch: the blocks one after another, the threads of a block one after another, each block with its own
// exactly-sized dynamic LDS (poisoned, see above); with GOI_HOST_LAUNCH_LOG set, each launch prints the kernel's name
// to stderr
template <typename K, typename... A>
inline void goi_host_launch(const char* name, K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t, A... args) {
    if (std::getenv("GOI_HOST_LAUNCH_LOG")) std::fprintf(stderr, "launch %s grid %u\n", name, grid.x);
    gridDim = GoiHostIdx{grid.x, grid.y, grid.z};
    blockDim = GoiHostIdx{block.x, block.y, block.z};
    for (unsigned by = 0; by < grid.y; ++by)
        for (unsigned bx = 0; bx < grid.x; ++bx) {
            int fill = 0;
            goi_host_poison_word(&fill);
            std::vector<int> mem((lds + sizeof(int) - 1) / sizeof(int), fill);
            goi_host_lds = mem.empty() ? nullptr : mem.data();
            blockIdx = GoiHostIdx{bx, by, 0};
            for (unsigned t = 0; t < block.x; ++t) {
                threadIdx = GoiHostIdx{t, 0, 0};
                kernel(args...);
            }
            goi_host_lds = nullptr;
        }
}
#define hipLaunchKernelGGL(kernel, grid, block, lds, stream, ...) \
    goi_host_launch(#kernel, kernel, dim3(grid), dim3(block), (size_t)(lds), stream, __VA_ARGS__)
