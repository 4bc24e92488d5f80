// Calibration of the fast Gumbel term of zs_k_bsample (zs_lane.hip): the
// largest |g_fast - g_exact| over all 2^24 uniforms u = ((r >> 8) + 0.5) / 2^24
// the hash can give (shaders.rs:812-815), where g = -ln(-ln u) with the
// f32-rounded double log and g_fast uses v_log_f32. The kernel assumes it is
// below ZS_GUMBEL_EPS = 2^-16; this checks it is below 2^-16 / 4. Exit 0 on
// success. Test program only (tests/test_gpu_calib.py builds and runs it).
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdint.h>
#include <string.h>
__device__ float gfast(float u) {
    const float w = -(__builtin_amdgcn_logf(u) * 0.693147180559945309f);
    return -(__builtin_amdgcn_logf(w) * 0.693147180559945309f);
}
__device__ float gexact(float u) {
    const float w = -(float)log((double)u);
    return -(float)log((double)w);
}
__global__ void k(unsigned int* maxbits, unsigned int* nonfinite) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (1u << 24)) return;
    float u = ((float)i + 0.5f) / 16777216.0f;   // as zs_rand01 (f32 ops)
    float a = gfast(u), b = gexact(u);
    if (!(a == a) || !(b == b) || a == INFINITY || b == INFINITY || a == -INFINITY || b == -INFINITY) {
        if (!(a == b)) atomicAdd(nonfinite, 1u);
        return;
    }
    float d = fabsf(a - b);
    atomicMax(maxbits, __float_as_uint(d));
}
int main() {
    unsigned int *m, *nf; hipMalloc(&m, 4); hipMalloc(&nf, 4); hipMemset(m, 0, 4); hipMemset(nf, 0, 4);
    hipLaunchKernelGGL(k, dim3((1u << 24) / 256), dim3(256), 0, 0, m, nf);
    unsigned int hm, hn; hipMemcpy(&hm, m, 4, hipMemcpyDeviceToHost); hipMemcpy(&hn, nf, 4, hipMemcpyDeviceToHost);
    float f; memcpy(&f, &hm, 4);
    printf("max |g_fast - g_exact| = %a (%.3e); non-finite mismatches %u; bound 2^-16\n", f, f, hn);
    return (f <= 0x1p-18f && hn == 0) ? 0 : 1;
}
