// Host-side stand-in for the HIP device environment (TEST INFRASTRUCTURE ONLY).
//
// Compiles the product's .hip sources as ordinary C++ for the CPU so that their kernels can be
// executed on the host for logic and bounds checks (under AddressSanitizer): every GPU thread
// is a fiber, a workgroup's fibers are scheduled cooperatively, and every cross-lane operation
// (shuffles, ballots, DPP, readlane, MFMA) and barrier is a rendezvous of the participating
// fibers. The matrix-core instruction is evaluated from its documented operand layout in double
// precision; transcendental approximations use libm. Results are therefore those of the
// kernels' logic, not the GPU's bits, except where the arithmetic is exactly specified.
// The product never includes this header: tests/emu/build_emu.py compiles the sources with it
// (through tests/emu/include/hip/*.h) into a separate library that only tests load.
#pragma once
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __shared__ static

struct dim3 {
    unsigned x, y, z;
    constexpr dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};

typedef int hipError_t;
typedef void* hipStream_t;
enum { hipSuccess = 0, hipErrorInvalidValue = 1, hipErrorLaunchFailure = 719 };
enum { hipFuncAttributeMaxDynamicSharedMemorySize = 8 };
enum { hipDeviceAttributeMultiprocessorCount = 63 };

namespace emu {
struct Index { unsigned x, y, z; };
const Index& thread_idx();
const Index& block_idx();
const Index& block_dim();
const Index& grid_dim();
int lane();
void launch(dim3 grid, dim3 block, size_t dyn_lds, std::function<void()> body);
char* dynamic_lds();
void* static_lds(int key, size_t bytes, size_t align);
void syncthreads();
void s_barrier();
void s_waitcnt(int imm);
void wave_barrier();
uint32_t shfl_u32(uint32_t v, int src_lane_xor, int mode, int width);
uint64_t ballot(bool p);
uint32_t readlane_u32(uint32_t v, int l);
uint32_t readfirstlane_u32(uint32_t v);
uint32_t update_dpp_u32(uint32_t old, uint32_t src, int ctrl, int row_mask, int bank_mask,
                        bool bound_ctrl);
void mfma_16x16x32_bf16(const void* a, const void* b, const float* c, float* d);
void global_load_lds(const void* g, uintptr_t lds, int size, int offset);
hipError_t last_error();

template <typename T>
inline T shfl_any(T v, int arg, int mode, int width) {
    static_assert(sizeof(T) == 4, "32-bit shuffles");
    return __builtin_bit_cast(T, shfl_u32(__builtin_bit_cast(uint32_t, v), arg, mode, width));
}
template <typename T>
inline T readlane_any(T v, int l) {
    static_assert(sizeof(T) == 4, "32-bit readlane");
    return __builtin_bit_cast(T, readlane_u32(__builtin_bit_cast(uint32_t, v), l));
}
template <typename T>
inline T readfirstlane_any(T v) {
    return __builtin_bit_cast(T, readfirstlane_u32(__builtin_bit_cast(uint32_t, v)));
}
}  // namespace emu

// the MFMA builtin on whatever operand vector types the kernel uses (8 x bf16 in, 4 x fp32)
template <typename A, typename C>
inline C emu_mfma_16x16x32(A a, A b, C c) {
    static_assert(sizeof(A) == 16 && sizeof(C) == 16, "16x16x32 bf16 operands");
    C d;
    ::emu::mfma_16x16x32_bf16(&a, &b, reinterpret_cast<const float*>(&c),
                              reinterpret_cast<float*>(&d));
    return d;
}

struct alignas(16) float4 { float x, y, z, w; };
struct alignas(8) uint2 { uint32_t x, y; };
inline float4 make_float4(float a, float b, float c, float d) { return float4{a, b, c, d}; }
inline uint2 make_uint2(uint32_t a, uint32_t b) { return uint2{a, b}; }

#define threadIdx (::emu::thread_idx())
#define blockIdx (::emu::block_idx())
#define blockDim (::emu::block_dim())
#define gridDim (::emu::grid_dim())

#define hipLaunchKernelGGL(K, G, B, S, ST, ...) \
    ::emu::launch(dim3(G), dim3(B), (size_t)(S), [=]() { K(__VA_ARGS__); })

inline hipError_t hipGetLastError() { return ::emu::last_error(); }
inline const char* hipGetErrorString(hipError_t e) { return e ? "emulated launch failure" : "no error"; }
inline hipError_t hipGetDevice(int* d) { *d = 0; return hipSuccess; }
inline hipError_t hipDeviceGetAttribute(int* v, int, int) { *v = 256; return hipSuccess; }
inline hipError_t hipFuncSetAttribute(const void*, int, int) { return hipSuccess; }

// device-side helpers
inline void __syncthreads() { ::emu::syncthreads(); }
inline void __threadfence() {}
template <typename T> inline T __shfl_xor(T v, int m, int w = 64) { return ::emu::shfl_any(v, m, 0, w); }
template <typename T> inline T __shfl(T v, int l, int w = 64) { return ::emu::shfl_any(v, l, 1, w); }
template <typename T> inline T __shfl_up(T v, unsigned d, int w = 64) { return ::emu::shfl_any(v, (int)d, 2, w); }
template <typename T> inline T __shfl_down(T v, unsigned d, int w = 64) { return ::emu::shfl_any(v, (int)d, 3, w); }
inline uint64_t __ballot(int p) { return ::emu::ballot(p != 0); }
inline int __popcll(unsigned long long v) { return __builtin_popcountll(v); }
inline int __popc(unsigned v) { return __builtin_popcount(v); }
inline int __ffsll(unsigned long long v) { return __builtin_ffsll((long long)v); }
inline int __clzll(unsigned long long v) { return v ? __builtin_clzll(v) : 64; }
template <typename T> inline T atomicAdd(T* p, T v) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32/64-bit atomics");
    return __atomic_fetch_add(p, v, __ATOMIC_RELAXED);   // relaxed, as the device's atomics
}
inline float __expf(float x) { return expf(x); }
inline float __uint_as_float(uint32_t v) { return __builtin_bit_cast(float, v); }
inline uint32_t __float_as_uint(float v) { return __builtin_bit_cast(uint32_t, v); }
inline float __int_as_float(int v) { return __builtin_bit_cast(float, v); }
inline int __float_as_int(float v) { return __builtin_bit_cast(int, v); }
inline int min(int a, int b) { return a < b ? a : b; }
inline int max(int a, int b) { return a > b ? a : b; }
inline unsigned min(unsigned a, unsigned b) { return a < b ? a : b; }
inline unsigned max(unsigned a, unsigned b) { return a > b ? a : b; }
inline int64_t min(int64_t a, int64_t b) { return a < b ? a : b; }
inline int64_t max(int64_t a, int64_t b) { return a > b ? a : b; }
inline int64_t min(int64_t a, int b) { return a < b ? a : b; }
inline int64_t min(int a, int64_t b) { return a < b ? a : b; }
inline uint64_t min(uint64_t a, uint64_t b) { return a < b ? a : b; }

// AMDGPU builtins
#define __builtin_amdgcn_s_waitcnt(x) ::emu::s_waitcnt(x)
#define __builtin_amdgcn_sched_barrier(x) ((void)0)
#define __builtin_amdgcn_sched_group_barrier(a, b, c) ((void)0)
#define __builtin_amdgcn_fence(order, scope) ((void)0)
#define __builtin_amdgcn_wave_barrier() ::emu::wave_barrier()
#define __builtin_amdgcn_exp2f(x) exp2f(x)
#define __builtin_amdgcn_rcpf(x) (1.0f / (x))
#define __builtin_amdgcn_readfirstlane(x) ::emu::readfirstlane_any(x)
#define __builtin_amdgcn_readlane(x, l) ::emu::readlane_any((x), (l))
#define __builtin_amdgcn_update_dpp(old, src, ctrl, rm, bm, bc)                                  \
    ((int)::emu::update_dpp_u32((uint32_t)(old), (uint32_t)(src), (ctrl), (rm), (bm), (bc)))
#define __builtin_amdgcn_global_load_lds(g, l, size, off, aux) \
    ::emu::global_load_lds((const void*)(g), (uintptr_t)(l), (size), (off))
#define __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, cbsz, abid, blgp) \
    ::emu_mfma_16x16x32((a), (b), (c))
