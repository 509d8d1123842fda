// The per-row softmax arithmetic shared by the softmax kernels and the fused
// bf16 attention, so that both produce the same bits for a row.
//
// A row is reduced by a team of L lanes (16: one DPP row; 64: the wavefront):
// column c is lane c % L's (c / L)-th term, the lane folds its terms in order
// from +0, then a fixed DPP tree combines the team. Exponentials are
// exp2((x - max) * log2 e) on the hardware exp2 for fp32 rows, and
// exp2(fma(x, log2 e, -(max * log2 e))) for bf16 rows (one instruction a term
// fewer: the row's shift is formed once; its rounding moves the exponent by at
// most an ulp of max * log2 e, far below the bf16 rounding of the result).
#pragma once

#include "device_common.hpp"

namespace cuvit::device {

constexpr float kLog2e = 1.4426950408889634F;

/// exp(x - max).
__device__ __forceinline__ float shifted_exp(float x, float max) {
    return __builtin_amdgcn_exp2f((x - max) * kLog2e);
}

/// All-reduce over a team of L lanes (16: one DPP row; 64: the wavefront).
template <int L, typename Op> __device__ __forceinline__ float team_allreduce(float value, Op op) {
    static_assert(L == 16 || L == 64, "teams are 16 or 64 lanes");
    if constexpr (L == 16) {
        return row16_allreduce(value, op);
    } else {
        return wave_allreduce(value, op);
    }
}

/// exp(x - max) as exp2(x * log2 e + shift), shift = -(max * log2 e) rounded
/// once, the product kept exact by the fused multiply-add (the bf16 rows' form).
__device__ __forceinline__ float shifted_exp_fused(float x, float shift) {
    return __builtin_amdgcn_exp2f(fmaf(x, kLog2e, shift));
}

/// Softmax of one row whose J terms per lane are in @p x (-inf past the row):
/// on return x holds the outputs. Team lane @p t holds columns t + L * j.
/// J may exceed the row's need: a term past the row is -inf before and 0
/// after the exponential, which changes no bit of the max or the sum.
/// @tparam kFused the bf16 rows' exponential (shifted_exp_fused).
template <int L, int J, bool kFused = false>
__device__ __forceinline__ void softmax_terms(float (&x)[J], int t, int columns) {
    float maximum = x[0];
#pragma unroll
    for (int j = 1; j < J; ++j) {
        maximum = fmaxf(maximum, x[j]);
    }
    const float row_maximum = team_allreduce<L>(maximum, Max{});
    const float shift = -(row_maximum * kLog2e);
    float sum = 0.F;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const float e = kFused ? shifted_exp_fused(x[j], shift) : shifted_exp(x[j], row_maximum);
        x[j] = t + L * j < columns ? e : 0.F;
        sum += x[j];
    }
    const float inverse = 1.0F / team_allreduce<L>(sum, Sum{});
#pragma unroll
    for (int j = 0; j < J; ++j) {
        x[j] *= inverse;
    }
}

} // namespace cuvit::device
