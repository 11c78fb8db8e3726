// Seeded synthetic table rows, generated in place on the device (a 43.5 GB
// table in a few tens of milliseconds) and reproducible on the CPU from the row
// id alone: value j of row r is qtable[mix64(seed*C + r*dim + j) >> 50], with
// mix64 the SplitMix64 output function (Steele, Lea, Flood, OOPSLA 2014) and
// qtable a 16,384-entry table of normal quantiles staged in LDS.  Every 32-value
// block is then quantised with the format's rule using only IEEE fp32 division,
// RNE rounding and integer bit manipulation, so the CPU restatement matches
// byte for byte.
#include "eg_common.h"

namespace eg {

constexpr int kQTable = 16384;
constexpr uint64_t kSeedMul = 0xD1B54A32D192ED03ull;

__device__ inline uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

template <int FMT>
__global__ __launch_bounds__(256) void synth_kernel(uint8_t* __restrict__ payload, uint8_t* __restrict__ scales,
                                                    int dim, uint64_t base, const float* __restrict__ qtable,
                                                    int64_t row0, int64_t n_blocks) {
  __shared__ float q[kQTable];
  for (int i = threadIdx.x; i < kQTable; i += 256) q[i] = qtable[i];
  __syncthreads();
  const int nbpr = dim >> 5;
  for (int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x; b < n_blocks; b += (int64_t)gridDim.x * 256) {
    const int64_t row = row0 + b / nbpr;
    const int blk = (int)(b - (b / nbpr) * nbpr);
    const uint64_t idx0 = base + (uint64_t)row * (uint64_t)dim + (uint64_t)(blk * 32);
    float x[32];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      x[j] = q[mix64(idx0 + j) >> 50];
      amax = fmaxf(amax, fabsf(x[j]));
    }
    const int64_t vbase = row * dim + blk * 32;  // value index of the block's first value
    if constexpr (FMT == EG_FMT_BF16) {
      u32x4* dst = (u32x4*)(payload + vbase * 2);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        u32x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = pack_bf16x2(x[w * 8 + 2 * i], x[w * 8 + 2 * i + 1]);
        dst[w] = o;
      }
    } else if constexpr (FMT == EG_FMT_Q8_0) {
      const uint16_t dh = f32_to_f16(amax / 127.0f);
      const float d = f16_to_f32(dh);
      u32x4 o[2];
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float r = (d == 0.0f) ? 0.0f : rintf(x[w * 4 + i] / d);
          r = fminf(fmaxf(r, -127.0f), 127.0f);
          word |= ((uint32_t)(int32_t)r & 0xffu) << (8 * i);
        }
        o[w >> 2][w & 3] = word;
      }
      u32x4* dst = (u32x4*)(payload + vbase);
      dst[0] = o[0];
      dst[1] = o[1];
      ((uint16_t*)scales)[row * nbpr + blk] = dh;
    } else {  // EG_FMT_MXFP8
      const int ebits = (int)((__float_as_uint(amax) >> 23) & 0xffu);
      // smallest e with amax * 2^-e <= 448: floor(log2 amax) - 8, plus one
      // where that would saturate
      int e = (amax > 0.0f ? ebits - 127 : -127) - 8;
      e = min(max(e, -127), 127);
      if (amax * ldexpf(1.0f, -e) > 448.0f) e = min(e + 1, 127);
      const float inv = ldexpf(1.0f, -e);
      u32x4 o[2];
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float s = fminf(fmaxf(x[w * 4 + i] * inv, -448.0f), 448.0f);
          word |= f32_to_e4m3(s) << (8 * i);
        }
        o[w >> 2][w & 3] = word;
      }
      u32x4* dst = (u32x4*)(payload + vbase);
      dst[0] = o[0];
      dst[1] = o[1];
      scales[row * nbpr + blk] = (uint8_t)(e + 127);
    }
  }
}

}  // namespace eg

using namespace eg;

extern "C" int eg_synth_table(const eg_table* table, uint64_t seed, const float* qtable, int64_t row0,
                              int64_t n_rows, void* stream) {
  TableDev t;
  int rc = make_table(table, &t, "synth table");
  if (rc != EG_OK) return rc;
  EG_CHECK_ARG(qtable != nullptr, "qtable is NULL");
  EG_CHECK_ARG(row0 >= 0 && n_rows >= 0 && row0 + n_rows <= table->n_rows, "rows [%lld, %lld) outside the table",
               (long long)row0, (long long)(row0 + n_rows));
  if (n_rows == 0) return EG_OK;
  const int64_t n_blocks = n_rows * (table->dim / 32);
  const uint64_t base = seed * kSeedMul;
  int64_t grid = (n_blocks + 255) / 256;
  if (grid > 256 * 8) grid = 256 * 8;  // grid-stride: the LDS table load is amortised
  uint8_t* payload = (uint8_t*)table->payload;
  uint8_t* scales = (uint8_t*)table->scales;
  hipStream_t st = (hipStream_t)stream;
  switch (table->fmt) {
    case EG_FMT_BF16:
      hipLaunchKernelGGL(synth_kernel<EG_FMT_BF16>, dim3((unsigned)grid), dim3(256), 0, st, payload, scales,
                         table->dim, base, qtable, row0, n_blocks);
      break;
    case EG_FMT_Q8_0:
      hipLaunchKernelGGL(synth_kernel<EG_FMT_Q8_0>, dim3((unsigned)grid), dim3(256), 0, st, payload, scales,
                         table->dim, base, qtable, row0, n_blocks);
      break;
    case EG_FMT_MXFP8:
      hipLaunchKernelGGL(synth_kernel<EG_FMT_MXFP8>, dim3((unsigned)grid), dim3(256), 0, st, payload, scales,
                         table->dim, base, qtable, row0, n_blocks);
      break;
    default:
      return set_error(EG_ERR_UNSUPPORTED, "synthetic rows in format %d", table->fmt);
  }
  return launch_status("synth_kernel");
}
