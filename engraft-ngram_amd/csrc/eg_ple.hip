// The PLE block that consumes the gathered rows (engraft/replica/layers.py:
// 565-626): after the two projections key = emb @ w_key^T [T, hc*n] and
// value = emb @ w_value^T [T, n] (library GEMMs on the matrix cores),
//
//   ple_gate_kernel   one workgroup per (position, stream j): the RMS norms
//                     of key_j and hidden_j, s_j = <key_j^, hidden_j^>/sqrt(n),
//                     gate_j = sigmoid(sign(s_j) sqrt(max(|s_j|, 1e-6))),
//                     gated_j = value * gate_j and its RMS norm (norm_conv):
//                     normed [T, hc*n], s and gate [T, hc]
//   ple_conv_kernel   one workgroup per 256 channels x 32 positions: the causal
//                     depthwise
//                     convolution over [history; normed] with dilation d,
//                     SiLU, and out = (hidden + gated) + conv
//
// fp32 throughout, the reference's operation order within each element; the
// reductions are workgroup tree sums (a different association from torch's).
#include <string.h>

#include "eg_common.h"

namespace eg {

constexpr int kPleThreads = 256;

__device__ inline float block_sum(float x, float* red) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  __syncthreads();  // the previous use of red is complete
  if (lane == 0) red[wave] = x;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int w = 0; w < kPleThreads / 64; ++w) t += red[w];
  return t;
}

// n <= kPleThreads * kPleMaxPer values per stream.
constexpr int kPleMaxPer = 16;

__global__ __launch_bounds__(kPleThreads) void ple_gate_kernel(
    const float* __restrict__ key, const float* __restrict__ value, const float* __restrict__ hidden,
    const float* __restrict__ norm_key, const float* __restrict__ norm_query, const float* __restrict__ norm_conv,
    int hc, int n, float eps, float inv_sqrt_n, float* __restrict__ normed, float* __restrict__ s_out,
    float* __restrict__ gate_out) {
  __shared__ float red[kPleThreads / 64];
  const int64_t t = blockIdx.x / hc;
  const int j = (int)(blockIdx.x - t * hc);
  const int tid = threadIdx.x;
  const int per = (n + kPleThreads - 1) / kPleThreads;
  // Every load of the workgroup is issued before the first reduction (indices
  // clamped into the row; entries past n are masked to zero).
  const int64_t row = (t * hc + j) * n;
  float v[kPleMaxPer], k[kPleMaxPer], h[kPleMaxPer], wk[kPleMaxPer], wq[kPleMaxPer];
#pragma unroll
  for (int m = 0; m < kPleMaxPer; ++m) {
    if (m < per) {
      const int i = min(tid + m * kPleThreads, n - 1);
      v[m] = value[t * n + i];
      k[m] = key[row + i];
      h[m] = hidden[row + i];
      wk[m] = norm_key[j * n + i];
      wq[m] = norm_query[j * n + i];
    }
  }
  float sk = 0.0f, sh = 0.0f;
#pragma unroll
  for (int m = 0; m < kPleMaxPer; ++m) {
    const bool ok = m < per && tid + m * kPleThreads < n;
    if (!ok) v[m] = k[m] = h[m] = 0.0f;
    sk += k[m] * k[m];
    sh += h[m] * h[m];
  }
  const float rk = 1.0f / sqrtf(block_sum(sk, red) / (float)n + eps);
  const float rq = 1.0f / sqrtf(block_sum(sh, red) / (float)n + eps);
  float dot = 0.0f;
#pragma unroll
  for (int m = 0; m < kPleMaxPer; ++m) {
    if (m < per && tid + m * kPleThreads < n) {
      const float kn = (k[m] * rk) * wk[m];
      const float qn = (h[m] * rq) * wq[m];
      dot += kn * qn;
    }
  }
  const float s = block_sum(dot, red) * inv_sqrt_n;
  const float mag = sqrtf(fmaxf(fabsf(s), 1e-6f));
  const float sg = s > 0.0f ? mag : (s < 0.0f ? -mag : 0.0f);
  const float gate = 1.0f / (1.0f + expf(-sg));
  float sq = 0.0f;
#pragma unroll
  for (int m = 0; m < kPleMaxPer; ++m) {
    const float g = v[m] * gate;
    sq += g * g;
  }
  const float rg = 1.0f / sqrtf(block_sum(sq, red) / (float)n + eps);
#pragma unroll
  for (int m = 0; m < kPleMaxPer; ++m) {
    const int i = tid + m * kPleThreads;
    if (m < per && i < n) normed[row + i] = ((v[m] * gate) * rg) * norm_conv[j * n + i];
  }
  if (tid == 0) {
    s_out[t * hc + j] = s;
    gate_out[t * hc + j] = gate;
  }
}

// Workgroup = 256 channels x kConvRun consecutive positions: a tap reads a row
// the same workgroup read a few positions earlier (L1), so every normed value
// comes from HBM about once.
constexpr int kConvRun = 32;

__global__ __launch_bounds__(256) void ple_conv_kernel(const float* __restrict__ full, int64_t hist_rows, int64_t T,
                                                       int hc, int n, const float* __restrict__ conv_w, int taps,
                                                       int dil, const float* __restrict__ hidden,
                                                       const float* __restrict__ value,
                                                       const float* __restrict__ gate, float* __restrict__ out) {
  const int C = hc * n;
  const int n_cblk = (C + 255) / 256;
  const int cblk = (int)(blockIdx.x % n_cblk);
  const int64_t t0 = (int64_t)(blockIdx.x / n_cblk) * kConvRun;
  const int c = cblk * 256 + threadIdx.x;
  if (c >= C) return;
  const int j = c / n;
  const int i = c - j * n;
  constexpr int kMaxTaps = 8;
  float w[kMaxTaps];
#pragma unroll
  for (int k = 0; k < kMaxTaps; ++k)
    if (k < taps) w[k] = conv_w[(int64_t)c * taps + k];
  const int64_t t_end = min(t0 + kConvRun, T);
  for (int64_t t = t0; t < t_end; ++t) {
    // a tap before the first row reads row 0 with its weight dropped (every load is issued)
    float x[kMaxTaps];
    bool ok[kMaxTaps];
#pragma unroll
    for (int k = 0; k < kMaxTaps; ++k) {
      if (k < taps) {
        const int64_t src = hist_rows + t - (int64_t)(taps - 1 - k) * dil;
        ok[k] = src >= 0;
        x[k] = full[(ok[k] ? src : 0) * C + c];
      }
    }
    const int64_t o = t * C + c;
    const float hv = hidden[o];
    const float vv = value[t * n + i];
    const float gj = gate[t * hc + j];
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < kMaxTaps; ++k)
      if (k < taps && ok[k]) acc += x[k] * w[k];
    const float silu = acc / (1.0f + expf(-acc));
    out[o] = (hv + vv * gj) + silu;
  }
}

}  // namespace eg

using namespace eg;

extern "C" {

int eg_ple_gate(const float* key, const float* value, const float* hidden, const float* norm_key,
                const float* norm_query, const float* norm_conv, int64_t n_pos, int32_t hc, int32_t n_embd, float eps,
                float* normed, float* s_out, float* gate_out, void* stream) {
  EG_CHECK_ARG(n_pos >= 0 && n_pos * hc < (1LL << 31), "n_pos=%lld", (long long)n_pos);
  EG_CHECK_ARG(hc >= 1 && hc <= 64 && n_embd >= 1 && n_embd <= kPleThreads * kPleMaxPer,
               "hc=%d n_embd=%d (n_embd <= %d)", hc, n_embd, kPleThreads * kPleMaxPer);
  EG_CHECK_ARG(n_pos == 0 || (key && value && hidden && norm_key && norm_query && norm_conv && normed && s_out &&
                              gate_out),
               "NULL argument");
  if (n_pos == 0) return EG_OK;
  hipLaunchKernelGGL(ple_gate_kernel, dim3((unsigned)(n_pos * hc)), dim3(kPleThreads), 0, (hipStream_t)stream, key,
                     value, hidden, norm_key, norm_query, norm_conv, hc, n_embd, eps, (float)(1.0 / sqrt((double)n_embd)),
                     normed, s_out, gate_out);
  return launch_status("ple_gate_kernel");
}

int eg_ple_conv(const float* full, int64_t hist_rows, int64_t n_pos, int32_t hc, int32_t n_embd,
                const float* conv_w, int32_t taps, int32_t dilation, const float* hidden, const float* value,
                const float* gate, float* out, void* stream) {
  EG_CHECK_ARG(n_pos >= 0 && hist_rows >= 0 && hc >= 1 && n_embd >= 1 && taps >= 1 && taps <= 8 && dilation >= 1,
               "n_pos=%lld hist_rows=%lld hc=%d n_embd=%d taps=%d dilation=%d", (long long)n_pos,
               (long long)hist_rows, hc, n_embd, taps, dilation);
  EG_CHECK_ARG(n_pos < (1LL << 31) && (int64_t)hc * n_embd < (1LL << 31), "too many elements");
  EG_CHECK_ARG(n_pos == 0 || (full && conv_w && hidden && value && gate && out), "NULL argument");
  if (n_pos == 0) return EG_OK;
  const int64_t blocks = (int64_t)((hc * n_embd + 255) / 256) * ((n_pos + kConvRun - 1) / kConvRun);
  EG_CHECK_ARG(blocks < (1LL << 32), "too many elements");
  hipLaunchKernelGGL(ple_conv_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, full,
                     hist_rows, n_pos, hc, n_embd, conv_w, taps, dilation, hidden, value, gate, out);
  return launch_status("ple_conv_kernel");
}

}  // extern "C"
