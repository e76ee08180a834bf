// Modulation projection: mods[r][n] = sum_k silu(c[r][k]) W[n][k] + bias[n] for the rows r = (sample, Euler
// step) of one expert call — every AdaRMS scale, shift and gate of every layer and step in one product
// (MODW = 9 L H + 2 H columns; the reference's kernel reads these rows, src/mk_expert.py:336-340, and
// REKI's _step_modulations makes them, mk_expert.py:529).
//
// HBM-bound on W (bf16 [MODW, H]: 108.5 MB for L10 H768), so each weight byte is read once: a wave owns 16
// output columns and holds their whole K extent as MFMA fragments in registers (H / 32 fragments of 16
// bytes per lane), issued before anything else. The workgroup stages silu(c) of each 16-row tile once in
// LDS, split into bf16 hi + lo parts in fragment order (two MFMAs per fragment, as exact as fp32 to ~2^-16
// relative), and every wave sweeps the tile against its fragments. Computed per wave from global memory
// instead, the 24 dependent loads of c per tile made the kernel latency-bound (69 us for 10 rows; 31 us
// staged). Issuing the first tile's rows ahead of the weights changed nothing measurable.
#pragma once

#include "mkx.h"
#include "mkx_device.h"

namespace mkx {

constexpr int MODP_BLOCK = 256;
constexpr int MODP_MAX_KT = 32;  // H <= 1024

// silu(c) of one 16-row tile in bf16 hi + lo parts, in MFMA fragment order: [t][lane][8] per part
template <int KT>
__device__ __forceinline__ void modproj_stage(const mkx_modproj_args& a, int r0, char* lds) {
  constexpr int PIECES = KT * 64;
#pragma unroll 1
  for (int p = threadIdx.x; p < PIECES; p += MODP_BLOCK) {
    const int t = p >> 6, ln = p & 63;
    const int r = min(r0 + (ln & 15), a.R - 1);  // rows past R stage a valid row, never stored
    const float* cp = a.c + (int64_t)r * a.c_stride + 32 * t + 8 * (ln >> 4);
    const f32x4 x0 = *reinterpret_cast<const f32x4*>(cp);
    const f32x4 x1 = *reinterpret_cast<const f32x4*>(cp + 4);
    const float g[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
    u32x4 hi, lo;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float v0 = g[2 * e] / (1.f + __expf(-g[2 * e]));  // silu
      const float v1 = g[2 * e + 1] / (1.f + __expf(-g[2 * e + 1]));
      const bf16_t h0 = f2bf(v0), h1 = f2bf(v1);
      hi[e] = (uint32_t)h0 | ((uint32_t)h1 << 16);
      lo[e] = pack2(v0 - bf2f(h0), v1 - bf2f(h1));
    }
    *reinterpret_cast<u32x4*>(lds + p * 16) = hi;
    *reinterpret_cast<u32x4*>(lds + (PIECES + p) * 16) = lo;
  }
}

// grid: N / 64 workgroups (rounded up) of 4 waves, each wave 16 output columns
template <int KT>
__global__ __launch_bounds__(MODP_BLOCK) void modproj_kernel(mkx_modproj_args a) {
  extern __shared__ __align__(16) char lds[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * 4 + wave) * 16;
  const bool active = n0 < a.N;  // inactive waves still stage rows and meet the barriers
  const int K = a.K;
  // weight fragments: row n0 + (lane & 15), k = 32 t + 8 (lane >> 4), all issued before the first tile
  // (fragment order: one 1 KB contiguous block per load and wave; row-major: 16 rows x 64 B per load)
  const int g = active ? n0 / 16 : 0;
  const bool fo = a.w_fragment_order != 0;
  const bf16_t* wp = (const bf16_t*)a.w + (fo ? ((int64_t)g * KT * 64 + lane) * 8
                                              : (int64_t)(g * 16 + (lane & 15)) * K + 8 * (lane >> 4));
  const int wstep = fo ? 64 * 8 : 32;
  bf16x8 wf[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) wf[t] = __builtin_bit_cast(bf16x8, ld16(wp + (int64_t)t * wstep));
  const int nout = active ? n0 + 4 * (lane >> 4) : 0;
  const f32x4 bias = *reinterpret_cast<const f32x4*>(a.bias + nout);
  for (int r0 = 0; r0 < a.R; r0 += 16) {
    if (r0) __syncthreads();  // the previous tile's fragments have been read
    modproj_stage<KT>(a, r0, lds);
    __syncthreads();
    f32x4 acc_h = {0.f, 0.f, 0.f, 0.f}, acc_l = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      const bf16x8 hi = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(lds + (t * 64 + lane) * 16));
      const bf16x8 lo = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(lds + ((KT + t) * 64 + lane) * 16));
      acc_h = mfma16(wf[t], hi, acc_h);
      acc_l = mfma16(wf[t], lo, acc_l);
    }
    if (active && r0 + (lane & 15) < a.R) {
      f32x4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = acc_h[i] + acc_l[i] + bias[i];
      *reinterpret_cast<f32x4*>(a.out + (int64_t)(r0 + (lane & 15)) * a.out_stride + nout) = o;
    }
  }
}

}  // namespace mkx
