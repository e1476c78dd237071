// Shared device helpers for the gfx950 MoE kernels: bf16 storage, MFMA operand vectors,
// wavefront reductions, the fp32 exponential the router uses, and error plumbing for the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>
#include <initializer_list>

namespace tsm {

typedef uint16_t bf16_t;                                            // bf16 storage (raw bits)
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));          // MFMA A/B operand (8 x bf16)
typedef float f32x4 __attribute__((ext_vector_type(4)));            // 16x16 MFMA accumulator
typedef float f32x16 __attribute__((ext_vector_type(16)));          // 32x32 MFMA accumulator
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));         // 16-byte memory chunk

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(bf16_t v) {
    return __uint_as_float(((uint32_t)v) << 16);
}

// Round to nearest even (the hardware conversion, v_cvt_pk_bf16_f32; same rule as torch's
// float -> bfloat16 cast).
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
    return __builtin_bit_cast(bf16_t, (__bf16)f);
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Low / high bf16 of a packed 32-bit word as fp32 (exact).
__device__ __forceinline__ float lo_bf16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

// SwiGLU with the reference's rounding points (tinykernels.py:293-297; the reference stores gate
// and up as bf16 and F.silu returns bf16): silu(g) = g * sigmoid(g) is rounded to bf16 before the
// multiply by u. sigmoid uses the hardware exp2 and reciprocal (about 1 fp32 ulp each), so the
// rounded silu equals that of an exactly rounded sigmoid except within a few fp32 ulps of a bf16
// rounding boundary. Every kernel that applies SwiGLU calls this one definition, so all weight
// layouts and tile shapes give identical bits.
__device__ __forceinline__ float swiglu_bf16(float g, float u) {
    g = round_bf16(g);
    u = round_bf16(u);
    const float s = round_bf16(g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)));
    return s * u;
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// XOR-butterfly sum over the 64 lanes of a wavefront. Every lane ends with the same value; the
// addition tree is fixed (partners at distance 32, 16, 8, 4, 2, 1), so the result is deterministic
// and the host oracle reproduces it bit for bit.
__device__ __forceinline__ float wave_sum_butterfly(float v) {
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) v += __shfl_xor(v, s);
    return v;
}

// Cross-lane reductions whose result does not depend on the combination order (max, and argmax
// under a total order) use DPP row operations instead of LDS-routed shuffles: xor 1 and xor 2
// within quads, mirrors within 8 and 16 lanes, then the row-15 / row-31 broadcasts carry the
// row results up to lane 63, which is read back into every lane.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(v, v, CTRL, ROW_MASK, 0xF, false);
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ void max_step(float& v) {
    v = fmaxf(v, __int_as_float(dpp_i<CTRL, ROW_MASK>(__float_as_int(v))));
}

__device__ __forceinline__ float wave_max(float v) {
    max_step<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
    max_step<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
    max_step<0x141, 0xF>(v);  // row_half_mirror
    max_step<0x140, 0xF>(v);  // row_mirror
    max_step<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    max_step<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// (largest value, lowest index among equal values) over the wavefront, for values that are
// +0 or more, or -inf. In that domain the IEEE bit patterns order like signed integers, so the
// pair is one order-preserving 64-bit key, (bits ^ sign) << 32 | ~index, and every step is a
// 64-bit compare and two selects with no branches.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ void key_max_step(uint32_t& hi, uint32_t& lo) {
    const uint32_t ohi = (uint32_t)dpp_i<CTRL, ROW_MASK>((int)hi);
    const uint32_t olo = (uint32_t)dpp_i<CTRL, ROW_MASK>((int)lo);
    const uint64_t k = ((uint64_t)hi << 32) | lo, o = ((uint64_t)ohi << 32) | olo;
    const bool take = o > k;
    hi = take ? ohi : hi;
    lo = take ? olo : lo;
}

__device__ __forceinline__ void wave_argmax(float& bv, int& bi) {
    uint32_t hi = __float_as_uint(bv) ^ 0x80000000u, lo = ~(uint32_t)bi;
    key_max_step<0xB1, 0xF>(hi, lo);   // quad_perm [1,0,3,2]
    key_max_step<0x4E, 0xF>(hi, lo);   // quad_perm [2,3,0,1]
    key_max_step<0x141, 0xF>(hi, lo);  // row_half_mirror
    key_max_step<0x140, 0xF>(hi, lo);  // row_mirror
    key_max_step<0x142, 0xA>(hi, lo);  // row_bcast:15 into rows 1 and 3
    key_max_step<0x143, 0xC>(hi, lo);  // row_bcast:31 into rows 2 and 3
    bv = __uint_as_float(__builtin_amdgcn_readlane(hi, 63) ^ 0x80000000u);
    bi = (int)~__builtin_amdgcn_readlane(lo, 63);
}

// exp(x) in fp32 for the router softmax, written out with explicit fmaf so the host oracle
// (oracle/moe_oracle.c, same algorithm) produces identical bits:
//   n = rint(x*log2(e)); r = x - n*ln2 (two-constant Cody-Waite reduction, |r| <= ln2/2);
//   exp(r) by the degree-7 Taylor polynomial in Horner form; result = 2^n * exp(r).
// Inputs below -86 (including -inf and NaN) return 0, so results are never subnormal.
__device__ __forceinline__ float router_expf(float x) {
#pragma clang fp contract(off)
    // branch-free: the polynomial runs on the input clamped to [-86, 88] (unchanged inside that
    // range), and the out-of-range results are selected afterwards
    const float xc = __builtin_fminf(__builtin_fmaxf(x, -86.0f), 88.0f);
    float n = __builtin_rintf(xc * 1.44269504088896341f);
    float r = __builtin_fmaf(-n, 0.693145751953125f, xc);
    r = __builtin_fmaf(-n, 1.42860682030941723e-06f, r);
    float p = 1.98412698412698413e-04f;  // 1/7!
    p = __builtin_fmaf(p, r, 1.38888888888888889e-03f);  // 1/6!
    p = __builtin_fmaf(p, r, 8.33333333333333333e-03f);  // 1/5!
    p = __builtin_fmaf(p, r, 4.16666666666666667e-02f);  // 1/4!
    p = __builtin_fmaf(p, r, 1.66666666666666667e-01f);  // 1/3!
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const float e = __builtin_ldexpf(p, (int)n);
    return (x >= -86.0f) ? (x > 88.0f ? __builtin_huge_valf() : e) : 0.0f;
}

}  // namespace tsm

// ---- host-side error plumbing shared by the C-ABI translation units ----
namespace tsm {
void set_error(const char* fmt, ...);
void clear_error();
int check_launch(const char* what);
// Status of a launch helper that already collected hipGetLastError(): the stage's name goes into
// the error message (a later check_launch would no longer see the error, which the first
// hipGetLastError call cleared).
int launch_status(hipError_t e, const char* what);
}  // namespace tsm

// True when every non-null pointer is a multiple of `a` bytes (the kernels' vector accesses).
inline bool tsm_aligned(size_t a, std::initializer_list<const void*> ptrs) {
    for (const void* p : ptrs)
        if (p && (reinterpret_cast<uintptr_t>(p) % a) != 0) return false;
    return true;
}

#define TSM_REQUIRE(cond, code, ...)          \
    do {                                       \
        if (!(cond)) {                         \
            ::tsm::set_error(__VA_ARGS__);     \
            return (code);                     \
        }                                      \
    } while (0)
