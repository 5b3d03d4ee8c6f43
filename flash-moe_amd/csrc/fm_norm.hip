// fm_norm.hip -- RMS norm with bf16 weights, and the elementwise SwiGLU, on
// the device.
//
// cpu_rms_norm (cpu_kernels.h:235-246) / rms_norm_sum_sq + rms_norm_apply_bf16
// (shaders.metal:792-870) as used for the next layer's input norm at the end
// of the decode step (layer_forward.h:3995-4029):
//   out[i] = x[i] * (1 / sqrtf(sum(x^2) / dim + eps)) * w[i]
// One 1024-thread workgroup per vector; the sum of squares is a tree sum
// (deterministic), so it differs from the sequential CPU sum by rounding only.
#include "fm_decode.h"

__global__ __launch_bounds__(1024) void fm_rms_norm_kernel(const float *__restrict__ x, const uint16_t *__restrict__ w,
                                                           uint32_t dim, float eps, float *__restrict__ out,
                                                           uint16_t *__restrict__ out_bf16) {
    __shared__ float part[16];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    float s = 0.f;
    for (uint32_t i = tid; i < dim; i += 1024) s = __builtin_fmaf(x[i], x[i], s);
    s = fm_lane_sum<64>(s);
    if (lane == 0) part[wv] = s;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int k = 0; k < 16; k++) tot += part[k];
    const float inv = 1.0f / sqrtf(tot / (float)dim + eps);
    for (uint32_t i = tid; i < dim; i += 1024) {
        const float v = x[i] * inv * fm_bf16_to_f32(w[i]);
        out[i] = v;
        if (out_bf16) out_bf16[i] = fm_f32_to_bf16(v);
    }
}

int fm_launch_rms_norm(const float *x, const uint16_t *w, uint32_t dim, float eps, float *out, uint16_t *out_bf16,
                       hipStream_t st) {
    hipLaunchKernelGGL(fm_rms_norm_kernel, dim3(1), dim3(1024), 0, st, x, w, dim, eps, out, out_bf16);
    return fm_check_launch("fm_rms_norm_kernel");
}

extern "C" int fm_rms_norm(const float *x, const uint16_t *w, uint32_t dim, float eps, float *out,
                           uint16_t *out_bf16, void *stream) {
    fm_clear_error();
    FM_REQUIRE(x && w && out, "fm_rms_norm: NULL argument");
    FM_REQUIRE(dim >= 1, "fm_rms_norm: dim 0");
    FM_REQUIRE(eps >= 0.f, "fm_rms_norm: eps < 0");
    return fm_launch_rms_norm(x, w, dim, eps, out, out_bf16, fm_stream(stream));
}

// act[i] = silu(gate[i]) * up[i] (cpu_swiglu, cpu_kernels.h:249-255; the
// swiglu_fused kernel of shaders.metal:714-727), for the step-by-step decode.
__global__ __launch_bounds__(256) void fm_swiglu_kernel(const float *__restrict__ g, const float *__restrict__ u,
                                                        float *__restrict__ act, uint32_t n) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) act[i] = fm_silu_mul(g[i], u[i]);
}

extern "C" int fm_swiglu(const float *gate, const float *up, float *act, uint32_t n, void *stream) {
    fm_clear_error();
    FM_REQUIRE(gate && up && act, "fm_swiglu: NULL argument");
    if (n == 0) return FM_OK;
    hipLaunchKernelGGL(fm_swiglu_kernel, dim3((n + 255) / 256), dim3(256), 0, fm_stream(stream), gate, up, act, n);
    return fm_check_launch("fm_swiglu_kernel");
}
