// vk_frontend.hip — the Whisper front end on gfx950: log-mel spectrogram
// (crates/vokra-models/src/whisper/mel.rs:123-183, fused form
// crates/vokra-ops/src/fused_logmel.rs:80-175) and 1-D convolution
// (crates/vokra-backend-cpu/src/kernels/mod.rs:583-822) for the encoder's conv
// stem (crates/vokra-models/src/whisper/encoder.rs:58-108).
//
// The STFT is a GEMM: every 400-sample frame (reflect-padded, windowed) times a
// [402 x 400] basis of cos / sin rows gives the 201 complex bins; the power
// spectrum times the [n_mels x 201] filter bank is a second GEMM; both run on
// the f32 matrix-core GEMM (vk_gemm_f32). log10, the per-clip maximum and the
// (max(v, gmax - 8) + 4) / 4 normalisation follow in two small passes.
// Convolution is im2col + the same GEMM.
#include <cmath>
#include <vector>

#include "vk_common.h"

namespace vk {

namespace fe {
constexpr int NS = 480000, NFFT = 400, HOP = 160, NFR = 3000, NB = 201, PAD = 200;
constexpr int LOG_ROWS = 16;  // frames per workgroup of the log pass
}  // namespace fe

// numpy mode="reflect" (crates/vokra-ops/src/stft.rs:269-285) for the
// single reflection the 200-sample centre padding needs.
__device__ __forceinline__ int fe_reflect(int i, int n) { return i < 0 ? -i : (i >= n ? 2 * (n - 1) - i : i); }

// frames[b * 3000 + t][i] = clip_b[reflect(160 t + i - 200)] * window[i], the
// clip zero-padded / trimmed to 480000 samples (mel.rs:134-137, fused_logmel.rs:135-138).
__global__ void vk_stft_frames(const float* __restrict__ pcm, int n_samples, const float* __restrict__ win,
                               float* __restrict__ frames, int batch) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)batch * fe::NFR * fe::NFFT;
    if (gid >= total) return;
    const int i = (int)(gid % fe::NFFT);
    const size_t bt = gid / fe::NFFT;
    const int t = (int)(bt % fe::NFR), b = (int)(bt / fe::NFR);
    const int q = fe_reflect(t * fe::HOP + i - fe::PAD, fe::NS);
    const float x = q < n_samples ? pcm[(size_t)b * n_samples + q] : 0.0f;
    frames[gid] = x * win[i];
}

// power[r][k] = re^2 + im^2 of the spectrum rows [re 0..200 | im 0..200].
__global__ void vk_power_spec(const float* __restrict__ spec, float* __restrict__ power, size_t rows) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= rows * fe::NB) return;
    const size_t r = gid / fe::NB;
    const int k = (int)(gid % fe::NB);
    const float re = spec[r * (2 * fe::NB) + k], im = spec[r * (2 * fe::NB) + fe::NB + k];
    power[gid] = re * re + im * im;
}

// out[b][m][t] = log10(max(mel[b * 3000 + t][m], 1e-10)); one workgroup per
// (clip, 16 frames) writes its partial maximum to partial[b][wg].
__global__ __launch_bounds__(256) void vk_logmel_log(const float* __restrict__ mel, int n_mels,
                                                     float* __restrict__ out, float* __restrict__ partial) {
    __shared__ float red[4];
    const int b = blockIdx.y, t0 = blockIdx.x * fe::LOG_ROWS;
    float mx = -INFINITY;
    for (int idx = threadIdx.x; idx < fe::LOG_ROWS * n_mels; idx += 256) {
        const int m = idx / fe::LOG_ROWS, t = t0 + idx % fe::LOG_ROWS;  // consecutive threads: consecutive t
        if (t >= fe::NFR) continue;
        const float v = mel[((size_t)b * fe::NFR + t) * n_mels + m];
        const float l = log10f(v > 1e-10f ? v : 1e-10f);
        out[((size_t)b * n_mels + m) * fe::NFR + t] = l;
        mx = fmaxf(mx, l);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, VK_WAVE));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    if (threadIdx.x == 0) partial[(size_t)b * gridDim.x + blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// out = (max(out, gmax - 8) + 4) / 4 with gmax the clip's maximum (every
// workgroup reduces the clip's partials itself; mel.rs:176-181).
__global__ __launch_bounds__(256) void vk_logmel_norm(float* __restrict__ out, int n_mels,
                                                      const float* __restrict__ partial, int n_partial) {
    __shared__ float red[4];
    const int b = blockIdx.y;
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < n_partial; i += 256) mx = fmaxf(mx, partial[(size_t)b * n_partial + i]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, VK_WAVE));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    const float floor_v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])) - 8.0f;
    const size_t n = (size_t)n_mels * fe::NFR;
    float* o = out + (size_t)b * n;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        o[i] = (fmaxf(o[i], floor_v) + 4.0f) / 4.0f;
}

// im2col over x(b, c, p) = x[b * sb + c * sc + p * sp] (zero outside 0..in_len):
// TRANS: col[b * out_len + t][c * kernel + kk]; else col[c * kernel + kk][t]
// (batch 1), the reference's layout (mod.rs:794-806).
template <bool TRANS>
__global__ void vk_im2col(const float* __restrict__ x, size_t sb, size_t sc, size_t sp, int batch, int in_ch,
                          int in_len, int kernel, int stride, int padding, int out_len, float* __restrict__ col) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t kk_total = (size_t)in_ch * kernel;
    const size_t total = (size_t)batch * out_len * kk_total;
    if (gid >= total) return;
    size_t row, t, b, r;
    if (TRANS) {
        r = gid % kk_total;
        row = gid / kk_total;  // b * out_len + t
        t = row % out_len;
        b = row / out_len;
    } else {
        t = gid % out_len;
        r = gid / out_len;
        b = 0;
    }
    const int c = (int)(r / kernel), kk = (int)(r % kernel);
    const long pos = (long)t * stride + kk - padding;
    col[gid] = (pos >= 0 && pos < in_len) ? x[b * sb + c * sc + (size_t)pos * sp] : 0.0f;
}

// out[oc][t] += bias[oc] (the reference adds the bias after its GEMM, mod.rs:814-820).
__global__ void vk_add_row_bias(float* __restrict__ out, const float* __restrict__ bias, int rows, int cols) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (size_t)rows * cols) return;
    out[gid] = out[gid] + bias[gid / cols];
}

// out[r][c] = out[r][c] + pos[r % period][c] (encoder.rs:98-104: conv output
// plus positional embedding, per clip of a batch).
__global__ void vk_add_pos(float* __restrict__ out, const float* __restrict__ pos, size_t rows, int d, int period) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= rows * d) return;
    const size_t r = gid / d;
    const int c = (int)(gid % d);
    out[gid] = out[gid] + pos[(r % period) * d + c];
}

template __global__ void vk_im2col<true>(const float*, size_t, size_t, size_t, int, int, int, int, int, int, int,
                                         float*);
template __global__ void vk_im2col<false>(const float*, size_t, size_t, size_t, int, int, int, int, int, int, int,
                                          float*);

// ---------------------------------------------------------------------------
// Host-side tables (built once per context, in double, cast to f32 as the
// reference does).

// Periodic Hann (crates/vokra-ops/src/window.rs:31,42-55).
void fe_hann_periodic(std::vector<float>& w) {
    w.resize(fe::NFFT);
    for (int n = 0; n < fe::NFFT; ++n) {
        const double x = 2.0 * M_PI * (double)n / (double)fe::NFFT;
        w[n] = (float)(0.5 - 0.5 * std::cos(x));
    }
}

// DFT basis rows: k-th cos row, then k-th -sin row (k = 0..200).
void fe_dft_basis(std::vector<float>& b) {
    b.assign((size_t)2 * fe::NB * fe::NFFT, 0.0f);
    for (int k = 0; k < fe::NB; ++k)
        for (int n = 0; n < fe::NFFT; ++n) {
            const double th = 2.0 * M_PI * (double)((k * n) % fe::NFFT) / (double)fe::NFFT;
            b[(size_t)k * fe::NFFT + n] = (float)std::cos(th);
            b[(size_t)(fe::NB + k) * fe::NFFT + n] = (float)-std::sin(th);
        }
}

// Slaney mel scale and the filter bank of crates/vokra-ops/src/mel.rs:29-130
// (triangles linear in Hz, Slaney norm), the Whisper front end's choice
// (crates/vokra-ops/src/frontend.rs:62-80).
static double fe_hz_to_mel(double f) {
    const double f_sp = 200.0 / 3.0, min_log_hz = 1000.0, min_log_mel = min_log_hz / f_sp;
    const double logstep = std::log(6.4) / 27.0;
    return f >= min_log_hz ? min_log_mel + std::log(f / min_log_hz) / logstep : f / f_sp;
}
static double fe_mel_to_hz(double mel) {
    const double f_sp = 200.0 / 3.0, min_log_hz = 1000.0, min_log_mel = min_log_hz / f_sp;
    const double logstep = std::log(6.4) / 27.0;
    return mel >= min_log_mel ? min_log_hz * std::exp(logstep * (mel - min_log_mel)) : f_sp * mel;
}
void fe_mel_filterbank(int n_mels, std::vector<float>& w) {
    const double sr = 16000.0, lo = fe_hz_to_mel(0.0), hi = fe_hz_to_mel(sr / 2.0);
    std::vector<double> band(n_mels + 2);
    for (int i = 0; i < n_mels + 2; ++i) band[i] = fe_mel_to_hz(lo + (hi - lo) * (double)i / (double)(n_mels + 1));
    w.assign((size_t)n_mels * fe::NB, 0.0f);
    for (int m = 0; m < n_mels; ++m) {
        const double left = band[m], center = band[m + 1], right = band[m + 2];
        for (int k = 0; k < fe::NB; ++k) {
            const double f = (double)k * sr / (double)fe::NFFT;
            const double lower = center > left ? (f - left) / (center - left) : 0.0;
            const double upper = right > center ? (right - f) / (right - center) : 0.0;
            const float v = (float)std::max(0.0, std::min(lower, upper));
            w[(size_t)m * fe::NB + k] = (float)((double)v * (2.0 / (right - left)));
        }
    }
}

int fe_n_frames() { return fe::NFR; }
int fe_n_bins() { return fe::NB; }
int fe_n_fft() { return fe::NFFT; }

hipError_t launch_stft_frames(hipStream_t s, const float* pcm, int batch, int n_samples, const float* win,
                              float* frames) {
    const size_t total = (size_t)batch * fe::NFR * fe::NFFT;
    hipLaunchKernelGGL(vk_stft_frames, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, pcm, n_samples, win,
                       frames, batch);
    return hipGetLastError();
}

hipError_t launch_power_spec(hipStream_t s, const float* spec, float* power, size_t rows) {
    hipLaunchKernelGGL(vk_power_spec, dim3((unsigned)((rows * fe::NB + 255) / 256)), dim3(256), 0, s, spec, power,
                       rows);
    return hipGetLastError();
}

int logmel_n_partial() { return (fe::NFR + fe::LOG_ROWS - 1) / fe::LOG_ROWS; }

hipError_t launch_logmel_finish(hipStream_t s, const float* mel, int batch, int n_mels, float* out, float* partial) {
    const int np = logmel_n_partial();
    hipLaunchKernelGGL(vk_logmel_log, dim3(np, batch), dim3(256), 0, s, mel, n_mels, out, partial);
    hipLaunchKernelGGL(vk_logmel_norm, dim3(64, batch), dim3(256), 0, s, out, n_mels, partial, np);
    return hipGetLastError();
}

hipError_t launch_im2col(hipStream_t s, bool trans, const float* x, size_t sb, size_t sc, size_t sp, int batch,
                         int in_ch, int in_len, int kernel, int stride, int padding, int out_len, float* col) {
    const size_t total = (size_t)batch * out_len * in_ch * kernel;
    if (total == 0) return hipSuccess;
    const dim3 grid((unsigned)((total + 255) / 256));
    if (trans)
        hipLaunchKernelGGL(vk_im2col<true>, grid, dim3(256), 0, s, x, sb, sc, sp, batch, in_ch, in_len, kernel, stride,
                           padding, out_len, col);
    else
        hipLaunchKernelGGL(vk_im2col<false>, grid, dim3(256), 0, s, x, sb, sc, sp, batch, in_ch, in_len, kernel, stride,
                           padding, out_len, col);
    return hipGetLastError();
}

hipError_t launch_add_row_bias(hipStream_t s, float* out, const float* bias, int rows, int cols) {
    const size_t total = (size_t)rows * cols;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_add_row_bias, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, out, bias, rows, cols);
    return hipGetLastError();
}

hipError_t launch_add_pos(hipStream_t s, float* out, const float* pos, size_t rows, int d, int period) {
    const size_t total = rows * d;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_add_pos, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, out, pos, rows, d, period);
    return hipGetLastError();
}

}  // namespace vk
