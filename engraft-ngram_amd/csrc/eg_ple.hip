// The PLE block that consumes the gathered rows (engraft/replica/layers.py:
// 565-626): after the two projections key = emb @ w_key^T [T, hc*n] and
// value = emb @ w_value^T [T, n] (fp32 library GEMMs, or eg_gemm_bf16x3),
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
//                     engraft/lens.py ple_out_at); ple_conv_win_kernel is
//                     the same for 4 taps at dilation 3 with each channel's
//                     rows held in registers (every row read once)
//   ple_rms_kernel   one workgroup per (row, stream j): x * 1/sqrt(mean(x^2)
//                     + eps) * w_j, the per-stream RMS norm on its own
//
// fp32 throughout, the reference's operation order within each element and no
// contracted multiply-adds; the reductions are workgroup tree sums (a
// different association from torch's).
#include <string.h>

#include <type_traits>

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
    float* __restrict__ gate_out, float* __restrict__ rstd_out) {
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
    if (rstd_out != nullptr) {  // the three RMS factors, for the backward
      rstd_out[(t * hc + j) * 3 + 0] = rk;
      rstd_out[(t * hc + j) * 3 + 1] = rq;
      rstd_out[(t * hc + j) * 3 + 2] = rg;
    }
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
                                                       const float* __restrict__ gate, float* __restrict__ out,
                                                       float* __restrict__ pre) {
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
      if (pre != nullptr) pre[o] = acc;  // the backward's SiLU derivative
      if constexpr (MODE == 0) out[o] = (hv[b] + vv[b] * gj[b]) + silu;
      else if constexpr (MODE == 1) out[o] = vv[b] * gj[b] + silu;
      else out[o] = silu;
    }
  }
}

// ple_conv_kernel for a fixed tap count and dilation, one position per row:
// each thread keeps its channel's rows t0-H .. t0+kConvRun-1 in registers
// (H = (TAPS-1)*DIL), so every row of `full` is read once per workgroup
// instead of once per tap.  Same arithmetic in the same order as
// ple_conv_kernel (bit-identical results).
template <int MODE, int TAPS, int DIL>
__global__ __launch_bounds__(256) void ple_conv_win_kernel(const float* __restrict__ full, int64_t hist_rows,
                                                           int64_t T, int hc, int n, const float* __restrict__ conv_w,
                                                           const float* __restrict__ hidden,
                                                           const float* __restrict__ value,
                                                           const float* __restrict__ gate, float* __restrict__ out,
                                                           float* __restrict__ pre) {
#pragma clang fp contract(off)
  constexpr int H = (TAPS - 1) * DIL;
  constexpr int RUN = kConvRun;
  const int C = hc * n;
  const int n_cblk = (C + 255) / 256;
  const int cblk = (int)(blockIdx.x % n_cblk);
  const int64_t t0 = (int64_t)(blockIdx.x / n_cblk) * RUN;
  const int c = cblk * 256 + threadIdx.x;
  if (c >= C) return;
  const int j = c / n;
  const int i = c - j * n;
  float w[TAPS];
#pragma unroll
  for (int k = 0; k < TAPS; ++k) w[k] = conv_w[(int64_t)c * TAPS + k];
  // window slot q holds row hist_rows + t0 - H + q; a row before the first is
  // not read (its taps are dropped), a row past the last (positions >= T,
  // never stored) re-reads the last
  const int64_t last = hist_rows + T - 1;
  float win[RUN + H];
#pragma unroll
  for (int q = 0; q < RUN + H; ++q) {
    const int64_t r = hist_rows + t0 - H + q;
    win[q] = full[(r < 0 ? 0 : (r > last ? last : r)) * C + c];
  }
  float hv[RUN], vv[RUN], gj[RUN];
#pragma unroll
  for (int b = 0; b < RUN; ++b) {
    const int64_t tb = min(t0 + b, T - 1);
    hv[b] = vv[b] = gj[b] = 0.0f;
    if constexpr (MODE == 0) hv[b] = hidden[tb * C + c];
    if constexpr (MODE <= 1) {
      vv[b] = value[tb * n + i];
      gj[b] = gate[tb * hc + j];
    }
  }
#pragma unroll
  for (int b = 0; b < RUN; ++b) {
    if (t0 + b >= T) break;
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < TAPS; ++k)
      if (hist_rows + t0 - H + b + k * DIL >= 0) acc += win[b + k * DIL] * w[k];
    const float silu = acc / (1.0f + expf(-acc));
    const int64_t o = (t0 + b) * C + c;
    if (pre != nullptr) pre[o] = acc;
    if constexpr (MODE == 0) out[o] = (hv[b] + vv[b] * gj[b]) + silu;
    else if constexpr (MODE == 1) out[o] = vv[b] * gj[b] + silu;
    else out[o] = silu;
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

// The same two kernels with 16-byte accesses: 128 threads per (row, stream),
// each P = n/512 float4 spaced 512 values apart (n a multiple of 512, P <= 8).
// The gate and RMS forms share their per-thread order and their tree
// (wavefront butterfly, then the two wavefronts in order), so the RMS kernel
// still reproduces the gate kernel's normed values bit for bit.  (One float4
// per thread, n/4 threads, ran 8 % slower than the scalar form: ten
// wavefronts per reduction.)
constexpr int kVecThreads = 128, kVecMaxP = 8;

__device__ inline float block_sum_2w(float x, float* red) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  __syncthreads();  // the previous use of red is complete
  if (lane == 0) red[wave] = x;
  __syncthreads();
  return red[0] + red[1];
}

__device__ inline void f4(const float* p, float* o) {
  const float4 v = *(const float4*)p;
  o[0] = v.x;
  o[1] = v.y;
  o[2] = v.z;
  o[3] = v.w;
}

template <int P>
__global__ __launch_bounds__(kVecThreads) void ple_gate_vec_kernel(
    const float* __restrict__ key, const float* __restrict__ value, const float* __restrict__ hidden,
    const float* __restrict__ norm_key, const float* __restrict__ norm_query, const float* __restrict__ norm_conv,
    int hc, int n, float eps, float inv_sqrt_n, float* __restrict__ normed, float* __restrict__ s_out,
    float* __restrict__ gate_out, float* __restrict__ rstd_out) {
#pragma clang fp contract(off)
  __shared__ float red[2];
  const int64_t t = blockIdx.x / hc;
  const int j = (int)(blockIdx.x - t * hc);
  const int64_t row = (t * hc + j) * n;
  float v[P][4], k[P][4], h[P][4], wk[P][4], wq[P][4];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int i = 4 * threadIdx.x + p * 4 * kVecThreads;
    f4(value + t * n + i, v[p]);
    f4(key + row + i, k[p]);
    f4(hidden + row + i, h[p]);
    f4(norm_key + (int64_t)j * n + i, wk[p]);
    f4(norm_query + (int64_t)j * n + i, wq[p]);
  }
  float sk = 0.0f, sh = 0.0f;
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sk += k[p][e] * k[p][e];
        sh += h[p][e] * h[p][e];
      }
  const float rk = 1.0f / sqrtf(block_sum_2w(sk, red) / (float)n + eps);
  const float rq = 1.0f / sqrtf(block_sum_2w(sh, red) / (float)n + eps);
  float dot = 0.0f;
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float kn = (k[p][e] * rk) * wk[p][e];
        const float qn = (h[p][e] * rq) * wq[p][e];
        dot += kn * qn;
      }
  const float s = block_sum_2w(dot, red) * inv_sqrt_n;
  const float mag = sqrtf(fmaxf(fabsf(s), 1e-6f));
  const float sg = s > 0.0f ? mag : (s < 0.0f ? -mag : 0.0f);
  const float gate = 1.0f / (1.0f + expf(-sg));
  float sq = 0.0f;
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float g = v[p][e] * gate;
        sq += g * g;
      }
  const float rg = 1.0f / sqrtf(block_sum_2w(sq, red) / (float)n + eps);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int i = 4 * threadIdx.x + p * 4 * kVecThreads;
    float wc[4], o[4];
    f4(norm_conv + (int64_t)j * n + i, wc);
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = ((v[p][e] * gate) * rg) * wc[e];
    *(float4*)(normed + row + i) = make_float4(o[0], o[1], o[2], o[3]);
  }
  if (threadIdx.x == 0) {
    s_out[t * hc + j] = s;
    gate_out[t * hc + j] = gate;
    if (rstd_out != nullptr) {
      rstd_out[(t * hc + j) * 3 + 0] = rk;
      rstd_out[(t * hc + j) * 3 + 1] = rq;
      rstd_out[(t * hc + j) * 3 + 2] = rg;
    }
  }
}

template <int P>
__global__ __launch_bounds__(kVecThreads) void ple_rms_vec_kernel(const float* __restrict__ x, int hc, int n,
                                                                 float eps, const float* __restrict__ w,
                                                                 float* __restrict__ out) {
#pragma clang fp contract(off)
  __shared__ float red[2];
  const int64_t t = blockIdx.x / hc;
  const int j = (int)(blockIdx.x - t * hc);
  const int64_t row = (t * hc + j) * n;
  float v[P][4];
#pragma unroll
  for (int p = 0; p < P; ++p) f4(x + row + 4 * threadIdx.x + p * 4 * kVecThreads, v[p]);
  float sq = 0.0f;
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
      for (int e = 0; e < 4; ++e) sq += v[p][e] * v[p][e];
  const float r = 1.0f / sqrtf(block_sum_2w(sq, red) / (float)n + eps);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int i = 4 * threadIdx.x + p * 4 * kVecThreads;
    float wv[4], o[4];
    f4(w + (int64_t)j * n + i, wv);
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = (v[p][e] * r) * wv[e];
    *(float4*)(out + row + i) = make_float4(o[0], o[1], o[2], o[3]);
  }
}

// ---------------------------------------------------------------------------
// Backward (gradients to the GEMM outputs, the hidden state and the history;
// the weights' gradients are not computed here)
// ---------------------------------------------------------------------------
// ple_conv_bwd_kernel: workgroup = 256 channels x kConvRun rows of full.
//   d_acc[t] = d_out[t] * silu'(acc[t]), silu'(x) = sg (1 + x (1 - sg)), acc
//   recomputed from the taps; the d_acc of the positions the rows need are
//   staged in LDS (each thread its own channel column), then
//   d_full[r] = sum_k w_k d_acc[r - hist_rows + back_k] (+ the gradient of the
//   returned history tail).
constexpr int kConvBwdMaxBack = 32;  // (taps - 1) * dilation the LDS window holds
constexpr int kConvBwdRun = 16;      // rows of full per workgroup
constexpr int kConvBwdBatch = 4;     // positions whose loads are issued together

template <bool PRE>
__global__ __launch_bounds__(256) void ple_conv_bwd_kernel(const float* __restrict__ full, int64_t hist_rows,
                                                           int64_t T, int hc, int n,
                                                           const float* __restrict__ conv_w, int taps, int dil,
                                                           const float* __restrict__ pre,
                                                           const float* __restrict__ d_out,
                                                           const float* __restrict__ d_tail, int64_t tail_rows,
                                                           float* __restrict__ d_full) {
#pragma clang fp contract(off)
  extern __shared__ float dacc[];  // [kConvBwdRun + (taps-1)*dil][256]
  const int C = hc * n;
  const int n_cblk = (C + 255) / 256;
  const int cblk = (int)(blockIdx.x % n_cblk);
  const int64_t r0 = (int64_t)(blockIdx.x / n_cblk) * kConvBwdRun;
  const int tid = threadIdx.x;
  const int c = cblk * 256 + tid;
  if (c >= C) return;  // no barrier below: every thread reads only its own column
  constexpr int kMaxTaps = 8;
  float w[kMaxTaps];
#pragma unroll
  for (int k = 0; k < kMaxTaps; ++k)
    if (k < taps) w[k] = conv_w[(int64_t)c * taps + k];
  const int64_t R = hist_rows + T;
  const int64_t r1 = min(r0 + kConvBwdRun, R);
  const int64_t max_back = (int64_t)(taps - 1) * dil;
  const int64_t ta = max(r0 - hist_rows, (int64_t)0);
  const int64_t tb = min(r1 - hist_rows + max_back, T);
  for (int64_t t = ta; t < tb; t += kConvBwdBatch) {
    float x[kConvBwdBatch][kMaxTaps];
    bool ok[kConvBwdBatch][kMaxTaps];
    float dv[kConvBwdBatch], pa[kConvBwdBatch];
#pragma unroll
    for (int b = 0; b < kConvBwdBatch; ++b) {
      const int64_t tt = min(t + b, tb - 1);
      if constexpr (PRE) {
        pa[b] = pre[tt * C + c];  // the forward's pre-activation
      } else {
#pragma unroll
        for (int k = 0; k < kMaxTaps; ++k) {
          if (k < taps) {
            const int64_t src = hist_rows + tt - (int64_t)(taps - 1 - k) * dil;
            ok[b][k] = src >= 0;
            x[b][k] = full[(ok[b][k] ? src : 0) * C + c];
          }
        }
      }
      dv[b] = d_out[tt * C + c];
    }
#pragma unroll
    for (int b = 0; b < kConvBwdBatch; ++b) {
      if (t + b >= tb) break;
      float acc = 0.0f;
      if constexpr (PRE) {
        acc = pa[b];
      } else {
#pragma unroll
        for (int k = 0; k < kMaxTaps; ++k)
          if (k < taps && ok[b][k]) acc += x[b][k] * w[k];
      }
      const float sg = 1.0f / (1.0f + expf(-acc));
      dacc[(t + b - ta) * 256 + tid] = dv[b] * (sg * (1.0f + acc * (1.0f - sg)));
    }
  }
  const int64_t tail0 = R - tail_rows;
  for (int64_t r = r0; r < r1; ++r) {
    float g = 0.0f;
#pragma unroll
    for (int k = 0; k < kMaxTaps; ++k) {
      if (k < taps) {
        const int64_t t = r - hist_rows + (int64_t)(taps - 1 - k) * dil;
        if (t >= 0 && t < T) g += w[k] * dacc[(t - ta) * 256 + tid];
      }
    }
    if (d_tail != nullptr && r >= tail0) g += d_tail[(r - tail0) * C + c];
    d_full[r * C + c] = g;
  }
}

// ple_gate_bwd_kernel: one workgroup of 1024 threads per position, every
// stream (hc <= 4, n <= 4096).  With x = value * gate_j (gated), y = normed,
// dy = d_normed, r = the forward's RMS factors:
//   d_gated = d_out + r_g nc dy - x r_g^3 / n * sum(dy nc x)
//   d_value = sum_j d_gated_j gate_j;  d_gate_j = sum(d_gated_j value)
//   d_s = d_gate g (1 - g) / (2 sqrt|s|) for |s| > 1e-6, else 0
//   d_key_raw = r_k nk (d_s q^ / sqrt n) - k r_k^2 d_s s / n
//   d_hidden  = d_out + r_q nq (d_s k^ / sqrt n) - h r_q^2 d_s s / n
// (the key and query norms' sums close to d_s s / r: sum(k^ q^) = s sqrt n).
constexpr int kGbThreads = 1024;
constexpr int kGbMaxPer = 4;
constexpr int kGbMaxHc = 4;

__device__ inline void block_sum4(float v[kGbMaxHc], float* red) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int kWaves = kGbThreads / 64;
#pragma unroll
  for (int j = 0; j < kGbMaxHc; ++j)
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v[j] += __shfl_xor(v[j], o);
  __syncthreads();  // the previous use of red is complete
  if (lane == 0)
#pragma unroll
    for (int j = 0; j < kGbMaxHc; ++j) red[j * kWaves + wave] = v[j];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kGbMaxHc; ++j) {
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) t += red[j * kWaves + w];
    v[j] = t;
  }
}

__global__ __launch_bounds__(kGbThreads) void ple_gate_bwd_kernel(
    const float* __restrict__ key, const float* __restrict__ value, const float* __restrict__ hidden,
    const float* __restrict__ norm_key, const float* __restrict__ norm_query, const float* __restrict__ norm_conv,
    const float* __restrict__ s_in, const float* __restrict__ gate_in, const float* __restrict__ rstd,
    const float* __restrict__ d_out, const float* __restrict__ d_normed, int hc, int n, float inv_sqrt_n,
    int detach_value, int detach_gate, float* __restrict__ d_key, float* __restrict__ d_value,
    float* __restrict__ d_hidden, float* __restrict__ d_s) {
#pragma clang fp contract(off)
  __shared__ float red[kGbMaxHc * (kGbThreads / 64)];
  const int64_t t = blockIdx.x;
  const int tid = threadIdx.x;
  const int per = (n + kGbThreads - 1) / kGbThreads;
  const float inv_n = 1.0f / (float)n;
  float sj[kGbMaxHc], gj[kGbMaxHc], rk[kGbMaxHc], rq[kGbMaxHc], rg[kGbMaxHc];
#pragma unroll
  for (int j = 0; j < kGbMaxHc; ++j) {
    const int jj = min(j, hc - 1);
    sj[j] = s_in[t * hc + jj];
    gj[j] = gate_in[t * hc + jj];
    rk[j] = rstd[(t * hc + jj) * 3 + 0];
    rq[j] = rstd[(t * hc + jj) * 3 + 1];
    rg[j] = rstd[(t * hc + jj) * 3 + 2];
  }
  float val[kGbMaxPer];
#pragma unroll
  for (int m = 0; m < kGbMaxPer; ++m)
    if (m < per) val[m] = value[t * n + min(tid + m * kGbThreads, n - 1)];
  // first reduction: sum(dy nc x) per stream; d_gated without its last term
  float dg[kGbMaxHc][kGbMaxPer], acc[kGbMaxHc];
#pragma unroll
  for (int j = 0; j < kGbMaxHc; ++j) {
    acc[j] = 0.0f;
    const int jj = min(j, hc - 1);
    const int64_t row = (t * hc + jj) * n;
#pragma unroll
    for (int m = 0; m < kGbMaxPer; ++m) {
      if (m < per) {
        const int i = min(tid + m * kGbThreads, n - 1);
        const bool ok = j < hc && tid + m * kGbThreads < n;
        const float dy = d_normed[row + i];
        const float wc = norm_conv[jj * n + i];
        const float x = val[m] * gj[j];
        dg[j][m] = d_out[row + i] + rg[j] * (wc * dy);
        if (ok) acc[j] += (dy * wc) * x;
      }
    }
  }
  block_sum4(acc, red);
#pragma unroll
  for (int j = 0; j < kGbMaxHc; ++j) {
    const float coef = ((rg[j] * rg[j]) * rg[j]) * inv_n * acc[j];
#pragma unroll
    for (int m = 0; m < kGbMaxPer; ++m)
      if (m < per) dg[j][m] = dg[j][m] - (val[m] * gj[j]) * coef;
  }
  if (!detach_value && d_value != nullptr) {
#pragma unroll
    for (int m = 0; m < kGbMaxPer; ++m) {
      const int i = tid + m * kGbThreads;
      if (m < per && i < n) {
        float dv = 0.0f;
#pragma unroll
        for (int j = 0; j < kGbMaxHc; ++j)
          if (j < hc) dv += dg[j][m] * gj[j];
        d_value[t * n + i] = dv;
      }
    }
  }
  // second reduction: d_gate per stream -> d_s
  float ds[kGbMaxHc];
#pragma unroll
  for (int j = 0; j < kGbMaxHc; ++j) ds[j] = 0.0f;
  if (!detach_gate) {  // uniform
#pragma unroll
    for (int j = 0; j < kGbMaxHc; ++j) {
      acc[j] = 0.0f;
#pragma unroll
      for (int m = 0; m < kGbMaxPer; ++m)
        if (m < per && j < hc && tid + m * kGbThreads < n) acc[j] += dg[j][m] * val[m];
    }
    block_sum4(acc, red);
#pragma unroll
    for (int j = 0; j < kGbMaxHc; ++j) {
      const float du = acc[j] * (gj[j] * (1.0f - gj[j]));
      const float as = fabsf(sj[j]);
      ds[j] = as > 1e-6f ? du * (0.5f / sqrtf(as)) : 0.0f;
    }
  }
  if (d_s != nullptr && threadIdx.x == 0)  // the score gradient, for the norm weights' gradients
#pragma unroll
    for (int j = 0; j < kGbMaxHc; ++j)
      if (j < hc) d_s[t * hc + j] = ds[j];
  // the key and query norms' backward, and the hidden state's gradient
#pragma unroll
  for (int j = 0; j < kGbMaxHc; ++j) {
    if (j >= hc) break;
    const int64_t row = (t * hc + j) * n;
    float k[kGbMaxPer], h[kGbMaxPer], wk[kGbMaxPer], wq[kGbMaxPer], dd[kGbMaxPer];
#pragma unroll
    for (int m = 0; m < kGbMaxPer; ++m) {
      if (m < per) {
        const int i = min(tid + m * kGbThreads, n - 1);
        k[m] = key[row + i];
        h[m] = hidden[row + i];
        wk[m] = norm_key[j * n + i];
        wq[m] = norm_query[j * n + i];
        dd[m] = d_out[row + i];
      }
    }
    const float ck = ((rk[j] * rk[j]) * ds[j]) * sj[j] * inv_n;
    const float cq = ((rq[j] * rq[j]) * ds[j]) * sj[j] * inv_n;
    const float dsn = ds[j] * inv_sqrt_n;
#pragma unroll
    for (int m = 0; m < kGbMaxPer; ++m) {
      const int i = tid + m * kGbThreads;
      if (m < per && i < n) {
        const float kn = (k[m] * rk[j]) * wk[m];
        const float qn = (h[m] * rq[j]) * wq[m];
        if (d_key != nullptr) d_key[row + i] = (rk[j] * wk[m]) * (dsn * qn) - k[m] * ck;
        if (d_hidden != nullptr) d_hidden[row + i] = dd[m] + ((rq[j] * wq[m]) * (dsn * kn) - h[m] * cq);
      }
    }
  }
}


// Sum over the workgroup of up to kGbMaxHc values per thread, for any whole
// number of wavefronts (the vector form below runs n/4 threads).
__device__ inline void block_sum4_n(float v[kGbMaxHc], float* red) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
#pragma unroll
  for (int j = 0; j < kGbMaxHc; ++j)
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v[j] += __shfl_xor(v[j], o);
  __syncthreads();  // the previous use of red is complete
  if (lane == 0)
#pragma unroll
    for (int j = 0; j < kGbMaxHc; ++j) red[j * (kGbThreads / 64) + wave] = v[j];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kGbMaxHc; ++j) {
    float t = 0.0f;
    for (int w = 0; w < nw; ++w) t += red[j * (kGbThreads / 64) + w];
    v[j] = t;
  }
}

// ple_gate_bwd_kernel with one float4 per thread: n/4 threads per position
// (n a multiple of 256, so whole wavefronts), 16-byte loads and stores, the
// same arithmetic per element.
// hi = rne(x), lo = rne(x - hi) of 4 values, stored at hi + o, lo + o.
__device__ inline void store_planes4(const float* x, __bf16* hi, __bf16* lo, int64_t o) {
  typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
  bf16x4 h, l;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    h[e] = (__bf16)x[e];
    l[e] = (__bf16)(x[e] - (float)h[e]);
  }
  *(bf16x4*)(hi + o) = h;
  *(bf16x4*)(lo + o) = l;
}

// PLANES: d_key and d_value are written as their bf16 hi / lo planes (the
// operands of eg_gemm_bf16x3), d_key_lo / d_value_lo the lo planes.
template <bool PLANES>
__global__ __launch_bounds__(kGbThreads) void ple_gate_bwd_vec_kernel(
    const float* __restrict__ key, const float* __restrict__ value, const float* __restrict__ hidden,
    const float* __restrict__ norm_key, const float* __restrict__ norm_query, const float* __restrict__ norm_conv,
    const float* __restrict__ s_in, const float* __restrict__ gate_in, const float* __restrict__ rstd,
    const float* __restrict__ d_out, const float* __restrict__ d_normed, int hc, int n, float inv_sqrt_n,
    int detach_value, int detach_gate, float* __restrict__ d_key, float* __restrict__ d_value,
    float* __restrict__ d_hidden, __bf16* __restrict__ d_key_lo, __bf16* __restrict__ d_value_lo,
    float* __restrict__ d_s) {
#pragma clang fp contract(off)
  __shared__ float red[kGbMaxHc * (kGbThreads / 64)];
  const int64_t t = blockIdx.x;
  const int i0 = 4 * threadIdx.x;
  const float inv_n = 1.0f / (float)n;
  float sj[kGbMaxHc], gj[kGbMaxHc], rk[kGbMaxHc], rq[kGbMaxHc], rg[kGbMaxHc];
#pragma unroll
  for (int j = 0; j < kGbMaxHc; ++j) {
    const int jj = min(j, hc - 1);
    sj[j] = s_in[t * hc + jj];
    gj[j] = gate_in[t * hc + jj];
    rk[j] = rstd[(t * hc + jj) * 3 + 0];
    rq[j] = rstd[(t * hc + jj) * 3 + 1];
    rg[j] = rstd[(t * hc + jj) * 3 + 2];
  }
  const float4 v4 = *(const float4*)(value + t * n + i0);
  const float val[4] = {v4.x, v4.y, v4.z, v4.w};
  // first reduction: sum(dy nc x) per stream; d_gated without its last term
  float dg[kGbMaxHc][4], acc[kGbMaxHc];
#pragma unroll
  for (int j = 0; j < kGbMaxHc; ++j) {
    acc[j] = 0.0f;
    const int jj = min(j, hc - 1);
    const int64_t row = (t * hc + jj) * n;
    const float4 dy4 = *(const float4*)(d_normed + row + i0);
    const float4 wc4 = *(const float4*)(norm_conv + (int64_t)jj * n + i0);
    const float4 do4 = *(const float4*)(d_out + row + i0);
    const float dy[4] = {dy4.x, dy4.y, dy4.z, dy4.w}, wc[4] = {wc4.x, wc4.y, wc4.z, wc4.w};
    const float dd[4] = {do4.x, do4.y, do4.z, do4.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float x = val[e] * gj[j];
      dg[j][e] = dd[e] + rg[j] * (wc[e] * dy[e]);
      if (j < hc) acc[j] += (dy[e] * wc[e]) * x;
    }
  }
  block_sum4_n(acc, red);
#pragma unroll
  for (int j = 0; j < kGbMaxHc; ++j) {
    const float coef = ((rg[j] * rg[j]) * rg[j]) * inv_n * acc[j];
#pragma unroll
    for (int e = 0; e < 4; ++e) dg[j][e] = dg[j][e] - (val[e] * gj[j]) * coef;
  }
  if (!detach_value && d_value != nullptr) {
    float dv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      dv[e] = 0.0f;
#pragma unroll
      for (int j = 0; j < kGbMaxHc; ++j)
        if (j < hc) dv[e] += dg[j][e] * gj[j];
    }
    if constexpr (PLANES) store_planes4(dv, (__bf16*)d_value, d_value_lo, t * n + i0);
    else *(float4*)(d_value + t * n + i0) = make_float4(dv[0], dv[1], dv[2], dv[3]);
  }
  // second reduction: d_gate per stream -> d_s
  float ds[kGbMaxHc];
#pragma unroll
  for (int j = 0; j < kGbMaxHc; ++j) ds[j] = 0.0f;
  if (!detach_gate) {  // uniform
#pragma unroll
    for (int j = 0; j < kGbMaxHc; ++j) {
      acc[j] = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (j < hc) acc[j] += dg[j][e] * val[e];
    }
    block_sum4_n(acc, red);
#pragma unroll
    for (int j = 0; j < kGbMaxHc; ++j) {
      const float du = acc[j] * (gj[j] * (1.0f - gj[j]));
      const float as = fabsf(sj[j]);
      ds[j] = as > 1e-6f ? du * (0.5f / sqrtf(as)) : 0.0f;
    }
  }
  if (d_s != nullptr && threadIdx.x == 0)  // the score gradient, for the norm weights' gradients
#pragma unroll
    for (int j = 0; j < kGbMaxHc; ++j)
      if (j < hc) d_s[t * hc + j] = ds[j];
  // the key and query norms' backward, and the hidden state's gradient
#pragma unroll
  for (int j = 0; j < kGbMaxHc; ++j) {
    if (j >= hc) break;
    const int64_t row = (t * hc + j) * n;
    const float4 k4 = *(const float4*)(key + row + i0), h4 = *(const float4*)(hidden + row + i0);
    const float4 wk4 = *(const float4*)(norm_key + (int64_t)j * n + i0);
    const float4 wq4 = *(const float4*)(norm_query + (int64_t)j * n + i0);
    const float4 do4 = *(const float4*)(d_out + row + i0);
    const float k[4] = {k4.x, k4.y, k4.z, k4.w}, h[4] = {h4.x, h4.y, h4.z, h4.w};
    const float wk[4] = {wk4.x, wk4.y, wk4.z, wk4.w}, wq[4] = {wq4.x, wq4.y, wq4.z, wq4.w};
    const float dd[4] = {do4.x, do4.y, do4.z, do4.w};
    const float ck = ((rk[j] * rk[j]) * ds[j]) * sj[j] * inv_n;
    const float cq = ((rq[j] * rq[j]) * ds[j]) * sj[j] * inv_n;
    const float dsn = ds[j] * inv_sqrt_n;
    float dk[4], dh[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float kn = (k[e] * rk[j]) * wk[e];
      const float qn = (h[e] * rq[j]) * wq[e];
      dk[e] = (rk[j] * wk[e]) * (dsn * qn) - k[e] * ck;
      dh[e] = dd[e] + ((rq[j] * wq[e]) * (dsn * kn) - h[e] * cq);
    }
    if (d_key != nullptr) {
      if constexpr (PLANES) store_planes4(dk, (__bf16*)d_key, d_key_lo, row + i0);
      else *(float4*)(d_key + row + i0) = make_float4(dk[0], dk[1], dk[2], dk[3]);
    }
    if (d_hidden != nullptr) *(float4*)(d_hidden + row + i0) = make_float4(dh[0], dh[1], dh[2], dh[3]);
  }
}

// Gradients of the norm and convolution weights: sums over the positions of
// per-element products, column c = j*n + i per thread (j the stream).  With
// the forward's RMS factors r and d_s the score gradient:
//   d_norm_key[c]   = sum_t (d_s_j / sqrt n) q^[t,c] * key[t,c] r_k
//   d_norm_query[c] = sum_t (d_s_j / sqrt n) k^[t,c] * hidden[t,c] r_q
//   d_norm_conv[c]  = sum_t d_normed[t,c] * value[t,i] gate_j r_g
//   d_conv[c,k]     = sum_t d_acc[t,c] * full[hist + t - (taps-1-k) dil, c]
// with d_acc = d_out silu'(pre).  Each workgroup sums kWgChunk positions of
// 256 columns; the chunks' partial sums are then added in chunk order (fixed
// association, no float atomics).
constexpr int kWgChunk = 64;
constexpr int kWgMaxTaps = 8;

template <int TAPS>
__global__ __launch_bounds__(256) void ple_wgrad_part_kernel(
    const float* __restrict__ key, const float* __restrict__ value, const float* __restrict__ hidden,
    const float* __restrict__ gate, const float* __restrict__ rstd, const float* __restrict__ d_s,
    const float* __restrict__ norm_key, const float* __restrict__ norm_query, const float* __restrict__ d_out,
    const float* __restrict__ d_normed, const float* __restrict__ full, int64_t hist_rows,
    const float* __restrict__ pre, int64_t T, int hc, int n, int dil, float inv_sqrt_n, float* __restrict__ part) {
#pragma clang fp contract(off)
  const int C = hc * n;
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= C) return;  // no barrier: a thread touches its own column only
  const int j = c / n, i = c - j * n;
  const int64_t t0 = (int64_t)blockIdx.y * kWgChunk;
  const int64_t t1 = min(t0 + kWgChunk, T);
  const float nk = norm_key[c], nq = norm_query[c];
  float a_nk = 0.0f, a_nq = 0.0f, a_nc = 0.0f, a_w[TAPS];
#pragma unroll
  for (int k = 0; k < TAPS; ++k) a_w[k] = 0.0f;
  for (int64_t t = t0; t < t1; ++t) {
    const int64_t pj = t * hc + j;
    const float rk = rstd[pj * 3 + 0], rq = rstd[pj * 3 + 1], rg = rstd[pj * 3 + 2];
    const float g = gate[pj], dsn = d_s[pj] * inv_sqrt_n;
    const int64_t e = t * C + c;
    const float kr = key[e] * rk, hr = hidden[e] * rq;
    a_nk += (dsn * (hr * nq)) * kr;
    a_nq += (dsn * (kr * nk)) * hr;
    a_nc += d_normed[e] * ((value[t * n + i] * g) * rg);
    const float x = pre[e];
    const float sg = 1.0f / (1.0f + expf(-x));
    const float da = d_out[e] * (sg * (1.0f + x * (1.0f - sg)));
#pragma unroll
    for (int k = 0; k < TAPS; ++k) {
      const int64_t src = hist_rows + t - (int64_t)(TAPS - 1 - k) * dil;
      if (src >= 0) a_w[k] += da * full[src * C + c];
    }
  }
  constexpr int Q = 3 + TAPS;
  float* out = part + (int64_t)blockIdx.y * Q * C + c;
  out[0] = a_nk;
  out[C] = a_nq;
  out[2 * (int64_t)C] = a_nc;
#pragma unroll
  for (int k = 0; k < TAPS; ++k) out[(3 + (int64_t)k) * C] = a_w[k];
}

// Chunk partial sums added in chunk order; q < 3: the norm weights, else conv tap q-3.
__global__ __launch_bounds__(256) void ple_wgrad_sum_kernel(const float* __restrict__ part, int64_t n_chunks,
                                                           int Q, int C, int taps, float* __restrict__ d_norm_key,
                                                           float* __restrict__ d_norm_query,
                                                           float* __restrict__ d_norm_conv,
                                                           float* __restrict__ d_conv) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)Q * C) return;
  const int q = (int)(idx / C), c = (int)(idx - (int64_t)q * C);
  float acc = 0.0f;
  for (int64_t ch = 0; ch < n_chunks; ++ch) acc += part[(ch * Q + q) * C + c];
  if (q == 0) { if (d_norm_key) d_norm_key[c] = acc; }
  else if (q == 1) { if (d_norm_query) d_norm_query[c] = acc; }
  else if (q == 2) { if (d_norm_conv) d_norm_conv[c] = acc; }
  else if (d_conv) d_conv[(int64_t)c * taps + (q - 3)] = acc;
}

// Calls f with std::integral_constant<int, p> for p = 1..kVecMaxP.
template <typename F>
static void launch_vec_p(int p, F&& f) {
  switch (p) {
    case 1: f(std::integral_constant<int, 1>{}); break;
    case 2: f(std::integral_constant<int, 2>{}); break;
    case 3: f(std::integral_constant<int, 3>{}); break;
    case 4: f(std::integral_constant<int, 4>{}); break;
    case 5: f(std::integral_constant<int, 5>{}); break;
    case 6: f(std::integral_constant<int, 6>{}); break;
    case 7: f(std::integral_constant<int, 7>{}); break;
    default: f(std::integral_constant<int, 8>{}); break;
  }
}

template <int MODE, bool SHARED>
static void launch_conv(dim3 grid, hipStream_t st, const float* full, int64_t hist_rows, int64_t n_pos, int hc, int n,
                        const float* conv_w, int taps, int dil, const float* hidden, const float* value,
                        const float* gate, float* out, float* pre) {
  if (!SHARED && taps == 4 && dil == 3) {  // the model's shape
    hipLaunchKernelGGL((ple_conv_win_kernel<MODE, 4, 3>), grid, dim3(256), 0, st, full, hist_rows, n_pos, hc, n,
                       conv_w, hidden, value, gate, out, pre);
    return;
  }
  hipLaunchKernelGGL((ple_conv_kernel<MODE, SHARED>), grid, dim3(256), 0, st, full, hist_rows, n_pos, hc, n, conv_w,
                     taps, dil, hidden, value, gate, out, pre);
}

}  // namespace eg

using namespace eg;

extern "C" {

int eg_ple_gate(const float* key, const float* value, const float* hidden, const float* norm_key,
                const float* norm_query, const float* norm_conv, int64_t n_pos, int32_t hc, int32_t n_embd, float eps,
                float* normed, float* s_out, float* gate_out, float* rstd_out, void* stream) {
  EG_CHECK_ARG(n_pos >= 0 && n_pos * hc < (1LL << 31), "n_pos=%lld", (long long)n_pos);
  EG_CHECK_ARG(hc >= 1 && hc <= 64 && n_embd >= 1 && n_embd <= kPleThreads * kPleMaxPer,
               "hc=%d n_embd=%d (n_embd <= %d)", hc, n_embd, kPleThreads * kPleMaxPer);
  EG_CHECK_ARG(n_pos == 0 || (key && value && hidden && norm_key && norm_query && norm_conv && normed && s_out &&
                              gate_out),
               "NULL argument");
  if (n_pos == 0) return EG_OK;
  const bool vec = n_embd % (4 * kVecThreads) == 0 &&
                   ((uintptr_t)key | (uintptr_t)value | (uintptr_t)hidden | (uintptr_t)norm_key |
                    (uintptr_t)norm_query | (uintptr_t)norm_conv | (uintptr_t)normed) % 16 == 0;
  if (vec)
    launch_vec_p(n_embd / (4 * kVecThreads), [&](auto pc) {
      hipLaunchKernelGGL(ple_gate_vec_kernel<decltype(pc)::value>, dim3((unsigned)(n_pos * hc)), dim3(kVecThreads), 0,
                         (hipStream_t)stream, key, value, hidden, norm_key, norm_query, norm_conv, hc, n_embd, eps,
                         (float)(1.0 / sqrt((double)n_embd)), normed, s_out, gate_out, rstd_out);
    });
  else
    hipLaunchKernelGGL(ple_gate_kernel, dim3((unsigned)(n_pos * hc)), dim3(kPleThreads), 0, (hipStream_t)stream, key,
                       value, hidden, norm_key, norm_query, norm_conv, hc, n_embd, eps,
                       (float)(1.0 / sqrt((double)n_embd)), normed, s_out, gate_out, rstd_out);
  return launch_status("ple_gate_kernel");
}

int eg_ple_conv(const float* full, int64_t hist_rows, int64_t n_pos, int32_t hc, int32_t n_embd,
                const float* conv_w, int32_t taps, int32_t dilation, int32_t shared_history, const float* hidden,
                const float* value, const float* gate, float* out, float* pre, void* stream) {
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
                                          hidden, value, gate, out, pre)
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
  // the form eg_ple_gate takes for the same n_embd and alignment: normed values bit for bit
  const bool vec = n_embd % (4 * kVecThreads) == 0 && ((uintptr_t)x | (uintptr_t)weight | (uintptr_t)out) % 16 == 0;
  if (vec)
    launch_vec_p(n_embd / (4 * kVecThreads), [&](auto pc) {
      hipLaunchKernelGGL(ple_rms_vec_kernel<decltype(pc)::value>, dim3((unsigned)(n_rows * hc)), dim3(kVecThreads), 0,
                         (hipStream_t)stream, x, hc, n_embd, eps, weight, out);
    });
  else
    hipLaunchKernelGGL(ple_rms_kernel, dim3((unsigned)(n_rows * hc)), dim3(kPleThreads), 0, (hipStream_t)stream, x, hc,
                       n_embd, eps, weight, out);
  return launch_status("ple_rms_kernel");
}

int eg_ple_conv_backward(const float* full, int64_t hist_rows, int64_t n_pos, int32_t hc, int32_t n_embd,
                         const float* conv_w, int32_t taps, int32_t dilation, const float* pre, const float* d_out,
                         const float* d_tail, int64_t tail_rows, float* d_full, void* stream) {
  EG_CHECK_ARG(n_pos >= 0 && hist_rows >= 0 && hc >= 1 && n_embd >= 1 && taps >= 1 && taps <= 8 && dilation >= 1,
               "n_pos=%lld hist_rows=%lld hc=%d n_embd=%d taps=%d dilation=%d", (long long)n_pos,
               (long long)hist_rows, hc, n_embd, taps, dilation);
  if ((int64_t)(taps - 1) * dilation > kConvBwdMaxBack)
    return set_error(EG_ERR_UNSUPPORTED, "convolution backward for (taps-1)*dilation = %lld > %d",
                     (long long)(taps - 1) * dilation, kConvBwdMaxBack);
  EG_CHECK_ARG(tail_rows >= 0 && tail_rows <= hist_rows + n_pos, "tail_rows=%lld", (long long)tail_rows);
  EG_CHECK_ARG(n_pos < (1LL << 31) && (int64_t)hc * n_embd < (1LL << 31), "too many elements");
  const int64_t rows = hist_rows + n_pos;
  EG_CHECK_ARG(rows == 0 || (full && conv_w && d_full && (n_pos == 0 || d_out)), "NULL argument");
  EG_CHECK_ARG(tail_rows == 0 || d_tail != nullptr, "d_tail is NULL");
  if (rows == 0) return EG_OK;
  const int64_t blocks = (int64_t)((hc * n_embd + 255) / 256) * ((rows + kConvBwdRun - 1) / kConvBwdRun);
  EG_CHECK_ARG(blocks < (1LL << 32), "too many elements");
  const size_t lds = (size_t)(kConvBwdRun + (taps - 1) * dilation) * 256 * sizeof(float);
  if (pre != nullptr)
    hipLaunchKernelGGL(ple_conv_bwd_kernel<true>, dim3((unsigned)blocks), dim3(256), lds, (hipStream_t)stream, full,
                       hist_rows, n_pos, hc, n_embd, conv_w, taps, dilation, pre, d_out, tail_rows ? d_tail : nullptr,
                       tail_rows, d_full);
  else
    hipLaunchKernelGGL(ple_conv_bwd_kernel<false>, dim3((unsigned)blocks), dim3(256), lds, (hipStream_t)stream, full,
                       hist_rows, n_pos, hc, n_embd, conv_w, taps, dilation, pre, d_out, tail_rows ? d_tail : nullptr,
                       tail_rows, d_full);
  return launch_status("ple_conv_bwd_kernel");
}

int eg_ple_gate_backward(const float* key, const float* value, const float* hidden, const float* norm_key,
                         const float* norm_query, const float* norm_conv, const float* s, const float* gate,
                         const float* rstd, const float* d_out, const float* d_normed, int64_t n_pos, int32_t hc,
                         int32_t n_embd, int32_t detach_value, int32_t detach_gate, float* d_key, float* d_value,
                         float* d_hidden, float* d_s, void* stream) {
  EG_CHECK_ARG(n_pos >= 0 && n_pos < (1LL << 31), "n_pos=%lld", (long long)n_pos);
  if (hc < 1 || hc > kGbMaxHc || n_embd < 1 || n_embd > kGbThreads * kGbMaxPer)
    return set_error(EG_ERR_UNSUPPORTED, "gate backward for hc=%d n_embd=%d (built: hc <= %d, n_embd <= %d)", hc,
                     n_embd, kGbMaxHc, kGbThreads * kGbMaxPer);
  EG_CHECK_ARG(n_pos == 0 || (key && value && hidden && norm_key && norm_query && norm_conv && s && gate && rstd &&
                              d_out && d_normed),
               "NULL argument");
  if (n_pos == 0) return EG_OK;
  // the float4 form needs 16-byte aligned rows of whole wavefronts of float4
  const bool vec = n_embd % 256 == 0 &&
                   ((uintptr_t)key | (uintptr_t)value | (uintptr_t)hidden | (uintptr_t)norm_key |
                    (uintptr_t)norm_query | (uintptr_t)norm_conv | (uintptr_t)d_out | (uintptr_t)d_normed |
                    (uintptr_t)d_key | (uintptr_t)d_value | (uintptr_t)d_hidden) % 16 == 0;
  if (vec)
    hipLaunchKernelGGL(ple_gate_bwd_vec_kernel<false>, dim3((unsigned)n_pos), dim3(n_embd / 4), 0, (hipStream_t)stream,
                       key, value, hidden, norm_key, norm_query, norm_conv, s, gate, rstd, d_out, d_normed, hc, n_embd,
                       (float)(1.0 / sqrt((double)n_embd)), detach_value, detach_gate, detach_gate ? nullptr : d_key,
                       detach_value ? nullptr : d_value, d_hidden, nullptr, nullptr, d_s);
  else
    hipLaunchKernelGGL(ple_gate_bwd_kernel, dim3((unsigned)n_pos), dim3(kGbThreads), 0, (hipStream_t)stream, key,
                       value, hidden, norm_key, norm_query, norm_conv, s, gate, rstd, d_out, d_normed, hc, n_embd,
                       (float)(1.0 / sqrt((double)n_embd)), detach_value, detach_gate, detach_gate ? nullptr : d_key,
                       detach_value ? nullptr : d_value, d_hidden, d_s);
  return launch_status("ple_gate_bwd_kernel");
}

int eg_ple_gate_backward_planes(const float* key, const float* value, const float* hidden, const float* norm_key,
                                const float* norm_query, const float* norm_conv, const float* s, const float* gate,
                                const float* rstd, const float* d_out, const float* d_normed, int64_t n_pos,
                                int32_t hc, int32_t n_embd, int32_t detach_value, int32_t detach_gate,
                                void* d_key_hi, void* d_key_lo, void* d_value_hi, void* d_value_lo, float* d_hidden,
                                float* d_s, void* stream) {
  EG_CHECK_ARG(n_pos >= 0 && n_pos < (1LL << 31), "n_pos=%lld", (long long)n_pos);
  if (hc < 1 || hc > kGbMaxHc || n_embd < 256 || n_embd > kGbThreads * 4 || n_embd % 256 != 0)
    return set_error(EG_ERR_UNSUPPORTED, "gate backward to planes for hc=%d n_embd=%d (built: hc <= %d, n_embd a "
                     "multiple of 256 up to %d)", hc, n_embd, kGbMaxHc, kGbThreads * 4);
  EG_CHECK_ARG(n_pos == 0 || (key && value && hidden && norm_key && norm_query && norm_conv && s && gate && rstd &&
                              d_out && d_normed),
               "NULL argument");
  EG_CHECK_ARG((d_key_hi == nullptr) == (d_key_lo == nullptr) && (d_value_hi == nullptr) == (d_value_lo == nullptr),
               "hi and lo planes go together");
  const bool aligned = ((uintptr_t)key | (uintptr_t)value | (uintptr_t)hidden | (uintptr_t)norm_key |
                        (uintptr_t)norm_query | (uintptr_t)norm_conv | (uintptr_t)d_out | (uintptr_t)d_normed |
                        (uintptr_t)d_hidden) % 16 == 0 &&
                       ((uintptr_t)d_key_hi | (uintptr_t)d_key_lo | (uintptr_t)d_value_hi | (uintptr_t)d_value_lo) % 8 == 0;
  EG_CHECK_ARG(aligned, "pointers must be 16-byte aligned (planes 8-byte)");
  if (n_pos == 0) return EG_OK;
  hipLaunchKernelGGL(ple_gate_bwd_vec_kernel<true>, dim3((unsigned)n_pos), dim3(n_embd / 4), 0, (hipStream_t)stream,
                     key, value, hidden, norm_key, norm_query, norm_conv, s, gate, rstd, d_out, d_normed, hc, n_embd,
                     (float)(1.0 / sqrt((double)n_embd)), detach_value, detach_gate,
                     detach_gate ? nullptr : (float*)d_key_hi, detach_value ? nullptr : (float*)d_value_hi, d_hidden,
                     (__bf16*)d_key_lo, (__bf16*)d_value_lo, d_s);
  return launch_status("ple_gate_bwd_vec_kernel");
}

size_t eg_ple_weight_grads_workspace_size(int64_t n_pos, int32_t hc, int32_t n_embd, int32_t taps) {
  if (n_pos <= 0 || hc < 1 || n_embd < 1 || taps < 1) return 0;
  return (size_t)((n_pos + kWgChunk - 1) / kWgChunk) * (size_t)(3 + taps) * (size_t)hc * (size_t)n_embd * 4;
}

int eg_ple_weight_grads(const float* key, const float* value, const float* hidden, const float* gate,
                        const float* rstd, const float* d_s, const float* norm_key, const float* norm_query,
                        const float* d_out, const float* d_normed, const float* full, int64_t hist_rows,
                        const float* pre, int64_t n_pos, int32_t hc, int32_t n_embd, int32_t taps, int32_t dilation,
                        float* d_norm_key, float* d_norm_query, float* d_norm_conv, float* d_conv_w, void* workspace,
                        size_t workspace_bytes, void* stream) {
  EG_CHECK_ARG(n_pos >= 0 && n_pos < (1LL << 31) && hist_rows >= 0 && hc >= 1 && n_embd >= 1 && dilation >= 1,
               "n_pos=%lld hist_rows=%lld hc=%d n_embd=%d dilation=%d", (long long)n_pos, (long long)hist_rows, hc,
               n_embd, dilation);
  if (taps < 1 || taps > kWgMaxTaps)
    return set_error(EG_ERR_UNSUPPORTED, "weight gradients for %d taps (built: 1..%d)", taps, kWgMaxTaps);
  EG_CHECK_ARG((int64_t)hc * n_embd < (1LL << 31), "too many columns");
  const int C = hc * n_embd;
  const int64_t n_chunks = (n_pos + kWgChunk - 1) / kWgChunk;
  const int Q = 3 + taps;
  hipStream_t st = (hipStream_t)stream;
  EG_CHECK_ARG(n_pos >= 1, "eg_ple_weight_grads needs at least one position");
  EG_CHECK_ARG(key && value && hidden && gate && rstd && d_s && norm_key && norm_query && d_out && d_normed && full &&
                   pre,
               "NULL argument");
  const size_t need = eg_ple_weight_grads_workspace_size(n_pos, hc, n_embd, taps);
  if (workspace_bytes < need)
    return set_error(EG_ERR_WORKSPACE, "workspace of %zu bytes < %zu needed", workspace_bytes, need);
  EG_CHECK_ARG(need == 0 || workspace != nullptr, "workspace is NULL");
  float* part = (float*)workspace;
  {
    const dim3 grid((unsigned)((C + 255) / 256), (unsigned)n_chunks);
    const float isn = (float)(1.0 / sqrt((double)n_embd));
#define EG_WG(TP)                                                                                                  \
  hipLaunchKernelGGL(ple_wgrad_part_kernel<TP>, grid, dim3(256), 0, st, key, value, hidden, gate, rstd, d_s,       \
                     norm_key, norm_query, d_out, d_normed, full, hist_rows, pre, n_pos, hc, n_embd, dilation, isn, \
                     part)
    switch (taps) {
      case 1: EG_WG(1); break;
      case 2: EG_WG(2); break;
      case 3: EG_WG(3); break;
      case 4: EG_WG(4); break;
      case 5: EG_WG(5); break;
      case 6: EG_WG(6); break;
      case 7: EG_WG(7); break;
      default: EG_WG(8); break;
    }
#undef EG_WG
  }
  const int64_t total = (int64_t)Q * C;
  hipLaunchKernelGGL(ple_wgrad_sum_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, part, n_chunks, Q,
                     C, taps, d_norm_key, d_norm_query, d_norm_conv, d_conv_w);
  return launch_status("ple_wgrad kernels");
}

}  // extern "C"
