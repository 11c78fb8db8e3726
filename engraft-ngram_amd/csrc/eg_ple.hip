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
//                     depthwise convolution over [history; normed] with
//                     dilation d, SiLU, and out = (hidden + gated) + conv
//                     (gated + conv without hidden, conv alone without value);
//                     with a shared history every position is a one-token
//                     continuation of the same history (the batch of
//                     engraft/lens.py ple_out_at)
//   ple_rms_kernel    one workgroup per (row, stream j): x * 1/sqrt(mean(x^2)
//                     + eps) * w_j, the per-stream RMS norm on its own
//
// fp32 throughout, the reference's operation order within each element and no
// contracted multiply-adds; the reductions are workgroup tree sums (a
// different association from torch's).
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
#pragma clang fp contract(off)
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
constexpr int kConvBatch = 4;  // positions whose loads are issued together

// MODE 0: out = (hidden + value*gate) + conv; 1: value*gate + conv; 2: conv.
template <int MODE, bool SHARED>
__global__ __launch_bounds__(256) void ple_conv_kernel(const float* __restrict__ full, int64_t hist_rows, int64_t T,
                                                       int hc, int n, const float* __restrict__ conv_w, int taps,
                                                       int dil, const float* __restrict__ hidden,
                                                       const float* __restrict__ value,
                                                       const float* __restrict__ gate, float* __restrict__ out) {
#pragma clang fp contract(off)
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
  // kConvBatch positions at a time: all their loads are issued before the first
  // is used (a position past t_end re-reads the last one and stores nothing);
  // a tap before the first row reads row 0 with its weight dropped.
  for (int64_t t = t0; t < t_end; t += kConvBatch) {
    float x[kConvBatch][kMaxTaps];
    bool ok[kConvBatch][kMaxTaps];
    float hv[kConvBatch], vv[kConvBatch], gj[kConvBatch];
#pragma unroll
    for (int b = 0; b < kConvBatch; ++b) {
      const int64_t tb = min(t + b, t_end - 1);
#pragma unroll
      for (int k = 0; k < kMaxTaps; ++k) {
        if (k < taps) {
          const int64_t back = (int64_t)(taps - 1 - k) * dil;
          const int64_t src = SHARED ? (back == 0 ? hist_rows + tb : hist_rows - back) : hist_rows + tb - back;
          ok[b][k] = src >= 0;
          x[b][k] = full[(ok[b][k] ? src : 0) * C + c];
        }
      }
      hv[b] = vv[b] = gj[b] = 0.0f;
      if constexpr (MODE == 0) hv[b] = hidden[tb * C + c];
      if constexpr (MODE <= 1) {
        vv[b] = value[tb * n + i];
        gj[b] = gate[tb * hc + j];
      }
    }
#pragma unroll
    for (int b = 0; b < kConvBatch; ++b) {
      if (t + b >= t_end) break;
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k < kMaxTaps; ++k)
        if (k < taps && ok[b][k]) acc += x[b][k] * w[k];
      const float silu = acc / (1.0f + expf(-acc));
      const int64_t o = (t + b) * C + c;
      if constexpr (MODE == 0) out[o] = (hv[b] + vv[b] * gj[b]) + silu;
      else if constexpr (MODE == 1) out[o] = vv[b] * gj[b] + silu;
      else out[o] = silu;
    }
  }
}

// The per-stream RMS norm, with the reductions of ple_gate_kernel (same thread
// layout and tree), so it reproduces that kernel's normed values bit for bit.
__global__ __launch_bounds__(kPleThreads) void ple_rms_kernel(const float* __restrict__ x, int hc, int n, float eps,
                                                            const float* __restrict__ w, float* __restrict__ out) {
#pragma clang fp contract(off)
  __shared__ float red[kPleThreads / 64];
  const int64_t t = blockIdx.x / hc;
  const int j = (int)(blockIdx.x - t * hc);
  const int tid = threadIdx.x;
  const int per = (n + kPleThreads - 1) / kPleThreads;
  const int64_t row = (t * hc + j) * n;
  float v[kPleMaxPer];
#pragma unroll
  for (int m = 0; m < kPleMaxPer; ++m)
    if (m < per) v[m] = x[row + min(tid + m * kPleThreads, n - 1)];
  float sq = 0.0f;
#pragma unroll
  for (int m = 0; m < kPleMaxPer; ++m) {
    if (!(m < per && tid + m * kPleThreads < n)) v[m] = 0.0f;
    sq += v[m] * v[m];
  }
  const float r = 1.0f / sqrtf(block_sum(sq, red) / (float)n + eps);
#pragma unroll
  for (int m = 0; m < kPleMaxPer; ++m) {
    const int i = tid + m * kPleThreads;
    if (m < per && i < n) out[row + i] = (v[m] * r) * w[j * n + i];
  }
}

template <int MODE, bool SHARED>
static void launch_conv(dim3 grid, hipStream_t st, const float* full, int64_t hist_rows, int64_t n_pos, int hc, int n,
                        const float* conv_w, int taps, int dil, const float* hidden, const float* value,
                        const float* gate, float* out) {
  hipLaunchKernelGGL((ple_conv_kernel<MODE, SHARED>), grid, dim3(256), 0, st, full, hist_rows, n_pos, hc, n, conv_w,
                     taps, dil, hidden, value, gate, out);
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
                const float* conv_w, int32_t taps, int32_t dilation, int32_t shared_history, const float* hidden,
                const float* value, const float* gate, float* out, void* stream) {
  EG_CHECK_ARG(n_pos >= 0 && hist_rows >= 0 && hc >= 1 && n_embd >= 1 && taps >= 1 && taps <= 8 && dilation >= 1,
               "n_pos=%lld hist_rows=%lld hc=%d n_embd=%d taps=%d dilation=%d", (long long)n_pos,
               (long long)hist_rows, hc, n_embd, taps, dilation);
  EG_CHECK_ARG(n_pos < (1LL << 31) && (int64_t)hc * n_embd < (1LL << 31), "too many elements");
  EG_CHECK_ARG(n_pos == 0 || (full && conv_w && out), "NULL argument");
  EG_CHECK_ARG(value != nullptr || hidden == nullptr, "hidden without value");
  EG_CHECK_ARG(value == nullptr || gate != nullptr, "value without gate");
  if (n_pos == 0) return EG_OK;
  const int64_t blocks = (int64_t)((hc * n_embd + 255) / 256) * ((n_pos + kConvRun - 1) / kConvRun);
  EG_CHECK_ARG(blocks < (1LL << 32), "too many elements");
  const dim3 grid((unsigned)blocks);
  hipStream_t st = (hipStream_t)stream;
  const int mode = hidden ? 0 : (value ? 1 : 2);
  const bool sh = shared_history != 0;
#define EG_CONV(M, S) launch_conv<M, S>(grid, st, full, hist_rows, n_pos, hc, n_embd, conv_w, taps, dilation, \
                                          hidden, value, gate, out)
  if (mode == 0) sh ? EG_CONV(0, true) : EG_CONV(0, false);
  else if (mode == 1) sh ? EG_CONV(1, true) : EG_CONV(1, false);
  else sh ? EG_CONV(2, true) : EG_CONV(2, false);
#undef EG_CONV
  return launch_status("ple_conv_kernel");
}

int eg_ple_rms(const float* x, int64_t n_rows, int32_t hc, int32_t n_embd, const float* weight, float eps, float* out,
               void* stream) {
  EG_CHECK_ARG(n_rows >= 0 && n_rows * hc < (1LL << 31), "n_rows=%lld", (long long)n_rows);
  EG_CHECK_ARG(hc >= 1 && hc <= 64 && n_embd >= 1 && n_embd <= kPleThreads * kPleMaxPer,
               "hc=%d n_embd=%d (n_embd <= %d)", hc, n_embd, kPleThreads * kPleMaxPer);
  EG_CHECK_ARG(n_rows == 0 || (x && weight && out), "NULL argument");
  if (n_rows == 0) return EG_OK;
  hipLaunchKernelGGL(ple_rms_kernel, dim3((unsigned)(n_rows * hc)), dim3(kPleThreads), 0, (hipStream_t)stream, x, hc,
                     n_embd, eps, weight, out);
  return launch_status("ple_rms_kernel");
}

}  // extern "C"
