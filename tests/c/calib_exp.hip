// Sweeps every f32 d in [-87, 1] on the GPU and reports the largest relative
// errors of zs_exp_fast and zs_exp_hw against the glibc-identical zs_expf; the
// certified increments of zllm_amd/csrc/zs_terms.h assume them below
// ZS_EXP_EPS / 2 and ZS_EXP_HW_EPS / 2.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include "../../zllm_amd/csrc/zs_terms.h"

__global__ void sweep(uint32_t lo, uint32_t n, unsigned long long* worst) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    double w = 0.0, wh = 0.0;
    for (uint32_t k = i; k < n; k += gridDim.x * blockDim.x) {
        float d = zs_u2f(lo + k);
        if (!(d >= -87.0f && d <= 1.0f)) continue;
        double a = zs_exp_fast(d), h = zs_exp_hw(d), e = zs_expf(d);
        double r = fabs(a - e) / e, rh = fabs(h - e) / e;
        w = r > w ? r : w;
        wh = rh > wh ? rh : wh;
    }
    atomicMax(worst, (unsigned long long)zs_d2u(w));
    atomicMax(worst + 1, (unsigned long long)zs_d2u(wh));
}

int main() {
    unsigned long long* d;
    hipMalloc(&d, 16);
    hipMemset(d, 0, 16);
    // positive d in [0, 1]: bit patterns 0 .. 0x3f800000; negative d in [-87, -0]
    sweep<<<4096, 256>>>(0u, 0x3f800001u, d);
    sweep<<<4096, 256>>>(0x80000000u, 0x42ae0001u, d);
    unsigned long long h[2] = {0, 0};
    hipMemcpy(h, d, 16, hipMemcpyDeviceToHost);
    double w = zs_u2d(h[0]), wh = zs_u2d(h[1]);
    printf("max_rel_err %.6e (2^%.2f) eps 2^-21\n", w, w > 0 ? log2(w) : -1000.0);
    printf("hw max_rel_err %.6e (2^%.2f) eps 2^-16\n", wh, wh > 0 ? log2(wh) : -1000.0);
    return (w < 0x1p-22 && wh < 0x1p-17) ? 0 : 1;
}
