// One AdamW update of the language-model shell's training step: gradient
// clipping's scale, the FP32 master update and the BF16 weight write-back in
// one pass over HBM.
//
// The reference's step (reproduction/experiments/optim.py:30-50, the "wiki"
// recipe) runs four passes over every parameter: clip_grad_norm_ scales the
// BF16 gradients in place, master.grad = grad.float() copies them to FP32,
// torch's fused AdamW updates the FP32 masters and both moments, and
// p.copy_(master) rounds the masters back into the BF16 weights.  Here one
// thread reads 4 consecutive elements of the BF16 gradient, the master and
// both moments, and writes the master, the moments and the BF16 weight:
// 28 bytes per parameter instead of ~44.
//
// The arithmetic is torch's fused AdamW (ATen's adam_math, ADAMW mode, no
// amsgrad, no maximize) with its types: the decay, both moment updates and
// the denominator's "+ eps" in double, rounded to float where torch stores a
// float; the bias corrections rounded to float; step_size * m / denom in
// float.  The gradient is round_bf16(g * scale), the value clip_grad_norm_'s
// in-place multiply leaves in a BF16 gradient.
#include "bdm_common.h"

namespace bdm {
namespace {

constexpr int kAdamwThreads = 256;
constexpr int kAdamwIlp = 4;

struct AdamwScalars {
    double lr, beta1, beta2, eps;
    float bias_correction1, bias_correction2_sqrt, step_size;
};

// The double multiply-adds are written as the fused operations torch's
// build makes of its expressions (param - lr*wd*param, beta1*m + (1-beta1)*g,
// beta2*v + (1-beta2)*g*g: the first product fused with the add), so the
// compiler cannot fuse the other product instead.
__device__ __forceinline__ void adamw_element(float &param, float grad, float &exp_avg, float &exp_avg_sq,
                                              double weight_decay, const AdamwScalars &s) {
    if (weight_decay != 0.0) param = float(fma(-(s.lr * weight_decay), double(param), double(param)));
    exp_avg = float(fma(s.beta1, double(exp_avg), (1 - s.beta1) * double(grad)));
    exp_avg_sq = float(fma(s.beta2, double(exp_avg_sq), (1 - s.beta2) * double(grad) * double(grad)));
    const float denom = float(double(sqrtf(exp_avg_sq) / s.bias_correction2_sqrt) + s.eps);
    param -= s.step_size * exp_avg / denom;
}

// One workgroup per (tensor, chunk) of the block table; a thread takes 4
// consecutive elements per iteration (16-byte FP32 and 8-byte BF16 accesses
// when the tensor's pointers allow, element by element otherwise).
__global__ __launch_bounds__(kAdamwThreads) void adamw_kernel(const bdm_adamw_tensor *__restrict__ tensors,
                                                              const int32_t *__restrict__ block_tensor,
                                                              const int64_t *__restrict__ block_start,
                                                              int64_t chunk, float *__restrict__ master,
                                                              float *__restrict__ exp_avg,
                                                              float *__restrict__ exp_avg_sq,
                                                              const float *__restrict__ grad_scale, AdamwScalars s) {
    const bdm_adamw_tensor t = tensors[block_tensor[blockIdx.x]];
    const int64_t begin = block_start[blockIdx.x];
    const int64_t end = min(t.numel, begin + chunk);
    const float scale = grad_scale ? *grad_scale : 1.f;
    bf16_t *param = static_cast<bf16_t *>(t.param);
    const bf16_t *grad = static_cast<const bf16_t *>(t.grad);
    float *pm = master + t.offset, *pa = exp_avg + t.offset, *pv = exp_avg_sq + t.offset;
    const bool vec = (reinterpret_cast<uintptr_t>(param) % 8 == 0) && (reinterpret_cast<uintptr_t>(grad) % 8 == 0) &&
                     t.offset % kAdamwIlp == 0 && begin % kAdamwIlp == 0;
    for (int64_t i = begin + int64_t(threadIdx.x) * kAdamwIlp; i < end; i += int64_t(kAdamwThreads) * kAdamwIlp) {
        if (vec && i + kAdamwIlp <= end) {
            const uint2 graw = *reinterpret_cast<const uint2 *>(grad + i);
            float4 m = *reinterpret_cast<const float4 *>(pm + i);
            float4 a = *reinterpret_cast<const float4 *>(pa + i);
            float4 v = *reinterpret_cast<const float4 *>(pv + i);
            const float g[4] = {__uint_as_float(graw.x << 16), __uint_as_float(graw.x & 0xffff0000u),
                                __uint_as_float(graw.y << 16), __uint_as_float(graw.y & 0xffff0000u)};
            float *mm = &m.x, *aa = &a.x, *vv = &v.x;
#pragma unroll
            for (int j = 0; j < kAdamwIlp; ++j)
                adamw_element(mm[j], round_bf16(g[j] * scale), aa[j], vv[j], t.weight_decay, s);
            *reinterpret_cast<float4 *>(pm + i) = m;
            *reinterpret_cast<float4 *>(pa + i) = a;
            *reinterpret_cast<float4 *>(pv + i) = v;
            *reinterpret_cast<uint2 *>(param + i) = make_uint2(pack_bf16x2(m.x, m.y), pack_bf16x2(m.z, m.w));
        } else {
            for (int64_t e = i; e < min(end, i + kAdamwIlp); ++e) {
                float m = pm[e], a = pa[e], v = pv[e];
                adamw_element(m, round_bf16(to_f32(grad[e]) * scale), a, v, t.weight_decay, s);
                pm[e] = m;
                pa[e] = a;
                pv[e] = v;
                param[e] = from_f32<bf16_t>(m);
            }
        }
    }
}

}  // namespace
}  // namespace bdm

extern "C" int bdm_adamw_step(const bdm_adamw_args *a, void *stream) {
    using namespace bdm;
    if (!a) return fail(BDM_ERR_INVALID, "adamw: null args");
    if (a->blocks < 0 || a->tensor_count < 0 || a->chunk <= 0 || a->chunk % kAdamwIlp != 0)
        return fail(BDM_ERR_INVALID, "adamw: bad block table");
    if (a->blocks == 0) return BDM_OK;
    if (!a->tensors || !a->block_tensor || !a->block_start || !a->master || !a->exp_avg || !a->exp_avg_sq)
        return fail(BDM_ERR_INVALID, "adamw: null pointer");
    if (!aligned(a->master, 16) || !aligned(a->exp_avg, 16) || !aligned(a->exp_avg_sq, 16))
        return fail(BDM_ERR_INVALID, "adamw: FP32 state buffers must be 16-byte aligned");
    if (a->blocks > int64_t(INT32_MAX)) return fail(BDM_ERR_UNSUPPORTED, "adamw: too many blocks");
    if (!(a->step >= 1.0)) return fail(BDM_ERR_INVALID, "adamw: step must be >= 1");
    AdamwScalars s;
    s.lr = a->lr;
    s.beta1 = a->beta1;
    s.beta2 = a->beta2;
    s.eps = a->eps;
    // torch evaluates these per launch in double and hands them to the update
    // as float (the step count is a float tensor)
    const double step = double(float(a->step));
    s.bias_correction1 = float(1 - pow(a->beta1, step));
    s.bias_correction2_sqrt = float(sqrt(1 - pow(a->beta2, step)));
    s.step_size = float(a->lr / double(s.bias_correction1));
    hipStream_t st = as_stream(stream);
    adamw_kernel<<<unsigned(a->blocks), kAdamwThreads, 0, st>>>(a->tensors, a->block_tensor, a->block_start, a->chunk,
                                                                a->master, a->exp_avg, a->exp_avg_sq, a->grad_scale, s);
    return check_launch("adamw_kernel");
}
