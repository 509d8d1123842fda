// The per-row softmax arithmetic shared by the softmax kernels and the fused
// bf16 attention, so that both produce the same bits for a row.
//
// A row is reduced by a team of L lanes (16: one DPP row; 64: the wavefront):
// column c is lane c % L's (c / L)-th term, the lane folds its terms in order
// from +0, then a fixed DPP tree combines the team. Exponentials are
// exp2((x - max) * log2 e) on the hardware exp2.
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

/// Softmax of one row whose J terms per lane are in @p x (-inf past the row):
/// on return x holds the outputs. Team lane @p t holds columns t + L * j.
/// J may exceed the row's need: a term past the row is -inf before and 0
/// after the exponential, which changes no bit of the max or the sum.
template <int L, int J>
__device__ __forceinline__ void softmax_terms(float (&x)[J], int t, int columns) {
    float maximum = x[0];
#pragma unroll
    for (int j = 1; j < J; ++j) {
        maximum = fmaxf(maximum, x[j]);
    }
    const float row_maximum = team_allreduce<L>(maximum, Max{});
    float sum = 0.F;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        x[j] = t + L * j < columns ? shifted_exp(x[j], row_maximum) : 0.F;
        sum += x[j];
    }
    const float inverse = 1.0F / team_allreduce<L>(sum, Sum{});
#pragma unroll
    for (int j = 0; j < J; ++j) {
        x[j] *= inverse;
    }
}

} // namespace cuvit::device
