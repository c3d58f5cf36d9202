// vk_lm.hip — the elementwise pieces of the speech-LLM text-decoder step
// (crates/vokra-models/src/voxtral/text_decoder.rs:1147-1420) for gfx950:
// rotary position embedding and the SwiGLU gate.
//
// RoPE (text_decoder.rs:858-891): for a row at position m and each head, the
// pair (x_j, x_{j+hd/2}) rotates by m * theta_j, theta_j = base^(-2j/hd):
//   x_j' = x_j c - x_{j+hd/2} s,  x_{j+hd/2}' = x_j s + x_{j+hd/2} c.
// theta_j comes from a table the host fills with the reference's own f32
// expression, so the angle m * theta_j is the reference's f32 product bit for
// bit; sin / cos are the device library's (within ~1 ulp of libm). Products
// and differences are not fused (the reference has no FMA).
//
// SwiGLU (text_decoder.rs:826-847, 1405-1410): out = (g * (1 / (1 + e^-g))) * u
// with the reference's three roundings in its order.
#include <algorithm>

#include "vk_common.h"

namespace vk {

// One thread per (row, head, pair j); x is [rows][n_head * hd], rotated in place.
__global__ void vk_rope_rows(float* __restrict__ x, int rows, int n_head, int hd, const float* __restrict__ theta,
                             const int* __restrict__ positions, int pos_offset) {
    const int half = hd >> 1;
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t per_row = (size_t)n_head * half;
    if (gid >= (size_t)rows * per_row) return;
    const int r = (int)(gid / per_row);
    const int rem = (int)(gid % per_row);
    const int h = rem / half, j = rem % half;
    const int pos = positions ? positions[r] : pos_offset + r;
    const float m = (float)pos;
    const float angle = m * theta[j];
    const float s = sinf(angle), c = cosf(angle);
    float* row = x + (size_t)r * n_head * hd + (size_t)h * hd;
    const float a = row[j], b = row[j + half];
    const float ac = a * c, bs = b * s, as = a * s, bc = b * c;
    row[j] = ac - bs;
    row[j + half] = as + bc;
}

// The same rotation over two arrays in one launch: q [rows][hq * hd] and
// k [rows][hkv * hd] (heads 0 .. hq-1 of the grid are q's, the rest k's).
__global__ void vk_rope_rows_qk(float* __restrict__ q, float* __restrict__ k, int rows, int hq, int hkv, int hd,
                                const float* __restrict__ theta, const int* __restrict__ positions) {
    const int half = hd >> 1;
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t per_row = (size_t)(hq + hkv) * half;
    if (gid >= (size_t)rows * per_row) return;
    const int r = (int)(gid / per_row);
    const int rem = (int)(gid % per_row);
    const int hh = rem / half, j = rem % half;
    const bool is_q = hh < hq;
    const int h = is_q ? hh : hh - hq, nh = is_q ? hq : hkv;
    const float m = (float)positions[r];
    const float angle = m * theta[j];
    const float s = sinf(angle), c = cosf(angle);
    float* row = (is_q ? q : k) + (size_t)r * nh * hd + (size_t)h * hd;
    const float a = row[j], b = row[j + half];
    const float ac = a * c, bs = b * s, as = a * s, bc = b * c;
    row[j] = ac - bs;
    row[j + half] = as + bc;
}

// The rotation's (cos, sin) of every (row, j) of one step: the angles of
// vk_rope_rows_qk, computed once per step for every layer and head that a
// fused consumer rotates (the K/V cache write and the GQA kernel's q load
// apply vk_rope_pair with them: the same products and sums, bit for bit).
__global__ void vk_rope_table(const int* __restrict__ positions, const float* __restrict__ theta, int rows, int half,
                              float2* __restrict__ cs) {
    const int gid = blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= rows * half) return;
    const int r = gid / half, j = gid % half;
    const float angle = (float)positions[r] * theta[j];
    cs[gid] = make_float2(cosf(angle), sinf(angle));
}

// out[i] = silu(g[i]) * u[i]; out may alias g.
__global__ void vk_swiglu_f32(const float* g, const float* __restrict__ u, float* out, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const float x = g[i];
        const float sg = 1.0f / (1.0f + expf(-x));
        const float t = x * sg;
        out[i] = t * u[i];
    }
}

}  // namespace vk

#include "vk_launch.h"

namespace vk {

hipError_t launch_rope_rows(hipStream_t s, float* x, int rows, int n_head, int hd, const float* theta,
                            const int* positions, int pos_offset) {
    const size_t threads = (size_t)rows * n_head * (hd / 2);
    if (threads == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_rope_rows, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, x, rows, n_head, hd,
                       theta, positions, pos_offset);
    return hipGetLastError();
}

hipError_t launch_rope_rows_qk(hipStream_t s, float* q, float* k, int rows, int hq, int hkv, int hd,
                               const float* theta, const int* positions) {
    const size_t threads = (size_t)rows * (hq + hkv) * (hd / 2);
    if (threads == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_rope_rows_qk, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, q, k, rows, hq, hkv,
                       hd, theta, positions);
    return hipGetLastError();
}

hipError_t launch_rope_table(hipStream_t s, const int* positions, const float* theta, int rows, int half, float2* cs) {
    const int threads = rows * half;
    if (threads == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_rope_table, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, positions, theta, rows,
                       half, cs);
    return hipGetLastError();
}

hipError_t launch_swiglu_f32(hipStream_t s, const float* g, const float* u, float* out, size_t n) {
    if (n == 0) return hipSuccess;
    const size_t blocks = std::min<size_t>((n + 255) / 256, 65536);
    hipLaunchKernelGGL(vk_swiglu_f32, dim3((unsigned)blocks), dim3(256), 0, s, g, u, out, n);
    return hipGetLastError();
}

}  // namespace vk
