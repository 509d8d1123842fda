// Device-side building blocks shared by the gfx950 kernels.
//
// Wavefronts are 64 lanes. A DPP "row" is 16 consecutive lanes; the reductions
// below use DPP moves inside a row and readlane across rows, so no reduction
// touches LDS and none needs a barrier.
//
// Every reduction combines its operands in an order fixed by lane position,
// and a + b == b + a holds exactly in IEEE arithmetic, so every lane receives
// the bit-identical total. Combined with a fixed column -> lane assignment,
// that makes a row's result independent of where the row sits in a launch,
// which is what keeps a batched forward pass bitwise equal to single images.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace cuvit::device {

constexpr int kWave = 64;

// DPP control words (GFX9 encoding).
constexpr int kDppQuadSwap1 = 0xB1;     // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppQuadSwap2 = 0x4E;     // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kDppRowHalfMirror = 0x141; // lane j of 8 <- 7 - j
constexpr int kDppRowMirror = 0x140;     // lane j of 16 <- 15 - j

template <int Control> __device__ __forceinline__ float dpp_move(float value) {
    return __int_as_float(
        __builtin_amdgcn_mov_dpp(__float_as_int(value), Control, 0xF, 0xF, false));
}

struct Sum {
    __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
};
struct Max {
    __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

/// All-reduce over each group of 16 lanes. Lane i of a group first combines
/// with i^1, then i^2, then the mirrored half and the mirrored row, so every
/// lane of the group ends with op over all 16 inputs.
template <typename Op> __device__ __forceinline__ float row16_allreduce(float value, Op op) {
    value = op(value, dpp_move<kDppQuadSwap1>(value));
    value = op(value, dpp_move<kDppQuadSwap2>(value));
    value = op(value, dpp_move<kDppRowHalfMirror>(value));
    value = op(value, dpp_move<kDppRowMirror>(value));
    return value;
}

/// All-reduce over the whole wavefront: 16-lane reduction, then the four row
/// totals combined as (r0 op r1) op (r2 op r3) in scalar registers.
template <typename Op> __device__ __forceinline__ float wave_allreduce(float value, Op op) {
    value = row16_allreduce(value, op);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(value), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(value), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(value), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(value), 48));
    return op(op(r0, r1), op(r2, r3));
}

/// Lane index inside the wavefront.
__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x) & (kWave - 1); }

// -- bfloat16 -----------------------------------------------------------------

/// Widens bf16 bits to float: the bits are the upper half of the float.
__device__ __forceinline__ float bf16_to_float(std::uint16_t bits) {
    return __uint_as_float(static_cast<std::uint32_t>(bits) << 16);
}

/// Rounds a float to bf16 bits, to nearest with ties to even, on gfx950's
/// conversion unit (v_cvt_pk_bf16_f32); NaN stays a quiet NaN.
__device__ __forceinline__ std::uint16_t float_to_bf16(float value) {
    return __builtin_bit_cast(std::uint16_t, static_cast<__bf16>(value));
}

/// Two floats rounded to bf16 and packed (@p low in bits 0-15), by one
/// v_cvt_pk_bf16_f32: the same rounding as float_to_bf16 on each, in one
/// instruction instead of two conversions, a shift and an or.
__device__ __forceinline__ std::uint32_t pack_bf16x2(float low, float high) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float floatx2 __attribute__((ext_vector_type(2)));
    const floatx2 pair = {low, high};
    return __builtin_bit_cast(std::uint32_t, __builtin_convertvector(pair, bf16x2));
}

// -- erf GELU -------------------------------------------------------------------

/// GELU in its erf form, x * Phi(x) = 0.5 x (1 + erf(x / sqrt 2)), branch-free.
/// With z = |x| / sqrt 2 and t = 1 / (1 + z / 2),
///   erfc(z) = t exp(-z^2 + P(t)),
/// the functional form of the Chebyshev erfc of Press et al., Numerical
/// Recipes 6.2; P is this library's own degree-7 fit (gelu_fit.py in this
/// folder: Chebyshev interpolation in float64 over z in [0, 10], largest error
/// of P 7.4e-7, which is erfc's relative error). The evaluation runs in base 2
/// with every constant folded in: w = z sqrt(log2 e), so -z^2 log2 e = -w^2
/// and 1 + z / 2 = 1 + w / (2 sqrt(log2 e)), and Q = P log2 e - 1 also
/// carries the factor 1/2, so that
///   erfc(z) / 2 = t exp2(-w^2 + Q(t))
/// takes one fused multiply-add and one exp2. Then Phi(x) = erfc(z) / 2 for
/// x < 0 and 1 - erfc(z) / 2 (one fused multiply-add) otherwise, so the
/// negative tail keeps its relative accuracy instead of cancelling in 1 + erf. Emulated in float32
/// over [-12, 12] against float64: at most 3.8e-7 absolute error, 5.4e-6
/// relative over the tail [-9, -3], inside the reference's GELU tolerance
/// (rtol 1e-5, atol 1e-6; elementwise_test.cu:48-49); rounded to bf16, about
/// 5e-5 of normally distributed inputs land one ulp from the correctly
/// rounded GELU. 17 instructions, two of them transcendental (rcp, exp2):
/// the GELU of a GEMM epilogue costs about as much issue time as the MFMAs
/// of a K = 768 product, so every instruction counts here.
__device__ __forceinline__ float gelu(float x) {
    const float w = fabsf(x) * 0.84932180028801907F;                              // sqrt(log2(e) / 2)
    const float t = __builtin_amdgcn_rcpf(fmaf(w, 0.41627730557884884F, 1.0F));  // 1 / (2 sqrt(log2 e))
    float q = -2.718776930e-01F;
    q = fmaf(q, t, 1.087971315e+00F);
    q = fmaf(q, t, -1.449840281e+00F);
    q = fmaf(q, t, 5.090884594e-01F);
    q = fmaf(q, t, -5.895698485e-02F);
    q = fmaf(q, t, 5.686708691e-01F);
    q = fmaf(q, t, 1.440642000e+00F);
    q = fmaf(q, t, -2.825698747e+00F);
    const float e = __builtin_amdgcn_exp2f(fmaf(-w, w, q));  // erfc(z) / 2 = t e
    return x * (x < 0.0F ? t * e : fmaf(-t, e, 1.0F));
}

// -- 16-byte vectors ----------------------------------------------------------

/// Sixteen bytes moved by one global_load_dwordx4 / global_store_dwordx4.
struct alignas(16) Vec16 {
    std::uint32_t w[4];
};

__device__ __forceinline__ Vec16 load16(const void* pointer) {
    const uint4 v = *reinterpret_cast<const uint4*>(pointer);
    return Vec16{{v.x, v.y, v.z, v.w}};
}

__device__ __forceinline__ void store16(void* pointer, const Vec16& value) {
    *reinterpret_cast<uint4*>(pointer) = make_uint4(value.w[0], value.w[1], value.w[2], value.w[3]);
}

/// A 16-byte store marked non-temporal (streaming): for outputs written once
/// and not read again by the same kernel. On MI355X it skips the L2
/// write-allocate and the end-of-kernel write-back of those lines, which
/// measured 0.7 us faster for a 9.7 MB LayerNorm and 0.7 us for the 38.5 MB
/// patch gather. Kernels that rewrite lines they have just read (in-place
/// softmax, the positional add) gain from it only with non-temporal loads of
/// those lines too.
__device__ __forceinline__ void store16_streaming(void* pointer, const Vec16& value) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = {value.w[0], value.w[1], value.w[2], value.w[3]};
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(pointer));
}

/// A 16-byte load marked non-temporal (streaming): for inputs read once. With
/// streaming stores beside it, a cold 38.5 MB device copy measured 7.7 us on
/// MI355X against 8.3 us with plain loads and 10.3 us with neither.
__device__ __forceinline__ Vec16 load16_streaming(const void* pointer) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(pointer));
    return Vec16{{v[0], v[1], v[2], v[3]}};
}

/// Element access for the two storage types the kernels handle. A Vec16 holds
/// 4 fp32 or 8 bf16 values.
template <typename T> struct Elem;

template <> struct Elem<float> {
    static constexpr int kPerVec = 4;
    __device__ __forceinline__ static float get(const Vec16& v, int i) {
        return __uint_as_float(v.w[i]);
    }
    __device__ __forceinline__ static void set(Vec16& v, int i, float x) { v.w[i] = __float_as_uint(x); }
    __device__ __forceinline__ static float load(const float* p) { return *p; }
    __device__ __forceinline__ static void store(float* p, float x) { *p = x; }
    /// Non-temporal (streaming) forms of load and store.
    __device__ __forceinline__ static float load_streaming(const float* p) {
        return __builtin_nontemporal_load(p);
    }
    __device__ __forceinline__ static void store_streaming(float* p, float x) {
        __builtin_nontemporal_store(x, p);
    }
    /// Copies element @p p into slot @p i of @p v without conversion.
    __device__ __forceinline__ static void put_bits(Vec16& v, int i, const float* p) {
        v.w[i] = __float_as_uint(*p);
    }
    /// Writes slot @p i of @p v to @p p without conversion.
    __device__ __forceinline__ static void store_bits(float* p, const Vec16& v, int i) {
        *p = __uint_as_float(v.w[i]);
    }
};

template <> struct Elem<std::uint16_t> {
    static constexpr int kPerVec = 8;
    __device__ __forceinline__ static float get(const Vec16& v, int i) {
        const std::uint32_t word = v.w[i >> 1];
        return bf16_to_float(static_cast<std::uint16_t>((i & 1) ? (word >> 16) : (word & 0xFFFFU)));
    }
    __device__ __forceinline__ static void set(Vec16& v, int i, float x) {
        const std::uint32_t bits = float_to_bf16(x);
        std::uint32_t& word = v.w[i >> 1];
        word = (i & 1) ? ((word & 0x0000FFFFU) | (bits << 16)) : ((word & 0xFFFF0000U) | bits);
    }
    __device__ __forceinline__ static float load(const std::uint16_t* p) { return bf16_to_float(*p); }
    __device__ __forceinline__ static void store(std::uint16_t* p, float x) { *p = float_to_bf16(x); }
    __device__ __forceinline__ static float load_streaming(const std::uint16_t* p) {
        return bf16_to_float(__builtin_nontemporal_load(p));
    }
    __device__ __forceinline__ static void store_streaming(std::uint16_t* p, float x) {
        __builtin_nontemporal_store(static_cast<std::uint16_t>(float_to_bf16(x)), p);
    }
    __device__ __forceinline__ static void put_bits(Vec16& v, int i, const std::uint16_t* p) {
        const std::uint32_t bits = *p;
        std::uint32_t& word = v.w[i >> 1];
        word = (i & 1) ? ((word & 0x0000FFFFU) | (bits << 16)) : ((word & 0xFFFF0000U) | bits);
    }
    __device__ __forceinline__ static void store_bits(std::uint16_t* p, const Vec16& v, int i) {
        const std::uint32_t word = v.w[i >> 1];
        *p = static_cast<std::uint16_t>((i & 1) ? (word >> 16) : (word & 0xFFFFU));
    }
};

/// True when @p pointer is 16-byte aligned.
inline bool aligned16(const void* pointer) {
    return (reinterpret_cast<std::uintptr_t>(pointer) & 15U) == 0;
}

} // namespace cuvit::device
