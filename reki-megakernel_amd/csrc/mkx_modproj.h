// Modulation projection: mods[r][n] = sum_k silu(c[r][k]) W[n][k] + bias[n] for the rows r = (sample, Euler
// step) of one expert call — every AdaRMS scale, shift and gate of every layer and step in one product
// (MODW = 9 L H + 2 H columns; the reference's kernel reads these rows, src/mk_expert.py:336-340, and
// REKI's _step_modulations makes them, mk_expert.py:529).
//
// HBM-bound on W (bf16 [MODW, H]: 108.5 MB for L10 H768), so each weight byte is read once: two waves own 16
// output columns, each holding half their K extent as MFMA fragments in registers (H / 64 fragments of 16
// bytes per lane), issued before anything else, and the second wave's partial sums are added through LDS. The
// workgroup stages silu(c) of each 16-row tile once in LDS, split into bf16 hi + lo parts in fragment order
// (two MFMAs per fragment, as exact as fp32 to ~2^-16 relative; silu with the hardware reciprocal and the
// split with the packed bf16 conversion, since every workgroup repeats this work for every tile), and every
// wave sweeps the tile against its fragments. Computed per wave from global memory instead, the 24 dependent
// loads of c per tile made the kernel latency-bound (69 us for 10 rows; 31 us staged).
#pragma once

#include "mkx.h"
#include "mkx_device.h"

namespace mkx {

constexpr int MODP_BLOCK = 256;
constexpr int MODP_MAX_KT = 32;  // H <= 1024
constexpr int MODP_KSPLIT = 2;   // waves sharing one 16-column tile, each over 1 / MODP_KSPLIT of K

typedef float modp_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 modp_bf16x2 __attribute__((ext_vector_type(2)));

// two floats rounded to nearest-even bf16 by the packed hardware conversion, low element in the low half
__device__ __forceinline__ uint32_t modp_cvt2(float x, float y) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((modp_f32x2){x, y}, modp_bf16x2));
}

// silu(c) of one 16-row tile in bf16 hi + lo parts, in MFMA fragment order: [t][lane][8] per part
template <int KT, int THREADS>
__device__ __forceinline__ void modproj_stage(const mkx_modproj_args& a, int r0, char* lds) {
  constexpr int PIECES = KT * 64;
#pragma unroll 1
  for (int p = threadIdx.x; p < PIECES; p += THREADS) {
    const int t = p >> 6, ln = p & 63;
    const int r = min(r0 + (ln & 15), a.R - 1);  // rows past R stage a valid row, never stored
    const float* cp = a.c + (int64_t)r * a.c_stride + 32 * t + 8 * (ln >> 4);
    const f32x4 x0 = *reinterpret_cast<const f32x4*>(cp);
    const f32x4 x1 = *reinterpret_cast<const f32x4*>(cp + 4);
    const float g[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
    u32x4 hi, lo;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float v0 = g[2 * e] * __builtin_amdgcn_rcpf(1.f + __expf(-g[2 * e]));  // silu
      const float v1 = g[2 * e + 1] * __builtin_amdgcn_rcpf(1.f + __expf(-g[2 * e + 1]));
      const uint32_t h = modp_cvt2(v0, v1);
      hi[e] = h;
      lo[e] = modp_cvt2(v0 - __uint_as_float(h << 16), v1 - __uint_as_float(h & 0xffff0000u));
    }
    *reinterpret_cast<u32x4*>(lds + p * 16) = hi;
    *reinterpret_cast<u32x4*>(lds + (PIECES + p) * 16) = lo;
  }
}

// dynamic LDS bytes of one projection workgroup: the staged tile (hi + lo)
template <int KT>
constexpr int modproj_lds_bytes() { return KT * 64 * 32; }

// grid: N / 64 workgroups (rounded up) of 4 column tiles x MODP_KSPLIT waves; wave w owns columns
// n0 .. n0 + 15 (tile w % 4) over k-blocks [KH (w / 4), KH (w / 4 + 1)), KH = KT / MODP_KSPLIT. Half the
// weight fragments per wave fit 4 waves per SIMD, two workgroups per CU, for H <= 768 (all K in one wave held
// 188 VGPRs: 2 waves), so more weight bytes are in flight and the waves finish in fewer rounds; H = 1024 keeps
// 2 waves per SIMD (4 would spill).
template <int KT>
__global__ __launch_bounds__(MODP_BLOCK * MODP_KSPLIT, KT <= 24 ? 4 : 2) void modproj_kernel(mkx_modproj_args a) {
  constexpr int KS = MODP_KSPLIT, KH = KT / KS, THREADS = MODP_BLOCK * KS;
  static_assert(KT % KS == 0, "k-blocks split evenly");
  extern __shared__ __align__(16) char lds[];
  __shared__ f32x4 part[(KS - 1) * 4 * 64];  // partial sums of the upper K parts: [ks - 1][tile][lane]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, ct = wave & 3, ks = wave >> 2;
  const int n0 = (blockIdx.x * 4 + ct) * 16;
  const bool active = n0 < a.N;  // inactive waves still stage rows and meet the barriers
  const int K = a.K;
  // weight fragments: row n0 + (lane & 15), k = 32 t + 8 (lane >> 4), t in this wave's half, all issued before
  // the first tile (fragment order: one 1 KB contiguous block per load and wave; row-major: 16 rows x 64 B)
  const int g = active ? n0 / 16 : 0;
  const bool fo = a.w_fragment_order != 0;
  const bf16_t* wp = (const bf16_t*)a.w + (fo ? ((int64_t)g * KT * 64 + lane) * 8
                                              : (int64_t)(g * 16 + (lane & 15)) * K + 8 * (lane >> 4));
  const int wstep = fo ? 64 * 8 : 32;
  bf16x8 wf[KH];
#pragma unroll
  for (int t = 0; t < KH; ++t) wf[t] = __builtin_bit_cast(bf16x8, ld16(wp + (int64_t)(ks * KH + t) * wstep));
  const int nout = active ? n0 + 4 * (lane >> 4) : 0;
  const f32x4 bias = *reinterpret_cast<const f32x4*>(a.bias + nout);
  for (int r0 = 0; r0 < a.R; r0 += 16) {
    if (r0) __syncthreads();  // the previous tile's fragments and partial sums have been read
    modproj_stage<KT, THREADS>(a, r0, lds);
    __syncthreads();
    f32x4 acc_h = {0.f, 0.f, 0.f, 0.f}, acc_l = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < KH; ++u) {
      const int t = ks * KH + u;
      const bf16x8 hi = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(lds + (t * 64 + lane) * 16));
      const bf16x8 lo = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(lds + ((KT + t) * 64 + lane) * 16));
      acc_h = mfma16(wf[u], hi, acc_h);
      acc_l = mfma16(wf[u], lo, acc_l);
    }
    f32x4 o = acc_h + acc_l;
    if (ks) part[((ks - 1) * 4 + ct) * 64 + lane] = o;
    __syncthreads();
    if (!ks && active && r0 + (lane & 15) < a.R) {
#pragma unroll
      for (int j = 1; j < KS; ++j) o += part[((j - 1) * 4 + ct) * 64 + lane];
      o += bias;
      *reinterpret_cast<f32x4*>(a.out + (int64_t)(r0 + (lane & 15)) * a.out_stride + nout) = o;
    }
  }
}

}  // namespace mkx

namespace mkx {

// The input of the modulation projection for an N-step Euler schedule (t_k = 1 - k / N):
// c[b][k] = silu(temb(t_k) W1^T + b1) W2^T + b2 + state_cond[b], temb(t) = [cos(1000 t f_i) | sin(1000 t f_i)]
// with f_i = 10000^(-i / (tdim / 2)) (the small MLP ahead of the projection in REKI's _step_modulations,
// mk_expert.py:529, as the synthetic expert defines it). One workgroup per 64 output columns of c, 4 waves of
// 16: each workgroup computes the whole hidden layer h1 = silu(temb W1^T + b1) for its (<= 16) steps on MFMAs
// (the embedding and h1 staged in LDS as bf16 hi + lo fragments, weights bf16, fp32 accumulation: fp32-exact to
// ~2^-16 relative), then its 64 columns of c for every sample. The embedding's arguments and cos / sin are
// computed in fp64 and rounded to fp32, as the fp32 eager expert computes them.
constexpr int MODIN_MAX_TKB = 16;  // tdim <= 512
constexpr int MODIN_MAX_HKB = 32;  // H <= 1024

// bf16 hi + lo of 8 fp32 values as the two 16-byte fragment halves
__device__ __forceinline__ void modin_split8(const float* g, u32x4& hi, u32x4& lo) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const bf16_t h0 = f2bf(g[2 * e]), h1 = f2bf(g[2 * e + 1]);
    hi[e] = (uint32_t)h0 | ((uint32_t)h1 << 16);
    lo[e] = pack2(g[2 * e] - bf2f(h0), g[2 * e + 1] - bf2f(h1));
  }
}

// acc (16 rows x 16 columns, D^T = W X^T: lane l holds columns 4 (l / 16) + i of row l % 16) of columns
// [n0, n0 + 16) of X W^T over KB k-blocks: X as split fragments in LDS ([kb][hi, lo][64 lanes] x 16 B), W row-major
// bf16 [*, ldw] from global memory
__device__ __forceinline__ f32x4 modin_mma(const char* xs, const bf16_t* w, int ldw, int n0, int KB, int lane) {
  f32x4 ah = {0.f, 0.f, 0.f, 0.f}, al = {0.f, 0.f, 0.f, 0.f};
  const bf16_t* wr = w + (int64_t)(n0 + (lane & 15)) * ldw + 8 * (lane >> 4);
  for (int kb = 0; kb < KB; ++kb) {
    const bf16x8 wf = __builtin_bit_cast(bf16x8, ld16(wr + 32 * kb));
    const bf16x8 hi = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(xs + ((kb * 2 + 0) * 64 + lane) * 16));
    const bf16x8 lo = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(xs + ((kb * 2 + 1) * 64 + lane) * 16));
    ah = mfma16(wf, hi, ah);
    al = mfma16(wf, lo, al);
  }
  return ah + al;
}

__global__ __launch_bounds__(MODP_BLOCK) void modin_kernel(mkx_modin_args a) {
  __shared__ __attribute__((aligned(16))) char es[MODIN_MAX_TKB * 2 * 1024];   // temb, split fragments
  __shared__ __attribute__((aligned(16))) char hs[MODIN_MAX_HKB * 2 * 1024];   // h1, split fragments
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int H = a.H, TKB = a.tdim / 32, HKB = H / 32, half = a.tdim / 2;
  const int n0 = (blockIdx.x * 4 + wave) * 16;  // this wave's 16 columns of c
  for (int k0 = 0; k0 < a.N; k0 += 16) {
    if (k0) __syncthreads();  // the previous row tile's fragments have been read
    // temb of steps k0 .. k0 + 15 (steps past N repeat the last one and are never stored)
    for (int pc = threadIdx.x; pc < TKB * 64; pc += MODP_BLOCK) {
      const int kb = pc >> 6, ln = pc & 63, k = min(k0 + (ln & 15), a.N - 1);
      const double t = 1.0 - (double)k / (double)a.N;
      float g[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int i = 32 * kb + 8 * (ln >> 4) + e;  // embedding column: cos for i < half, sin after
        const int fi = i < half ? i : i - half;
        const double arg = t * 1000.0 * exp(-log(10000.0) * (double)fi / (double)half);
        g[e] = (float)(i < half ? cos(arg) : sin(arg));
      }
      u32x4 hi, lo;
      modin_split8(g, hi, lo);
      *reinterpret_cast<u32x4*>(es + ((kb * 2 + 0) * 64 + ln) * 16) = hi;
      *reinterpret_cast<u32x4*>(es + ((kb * 2 + 1) * 64 + ln) * 16) = lo;
    }
    __syncthreads();
    // h1 = silu(temb W1^T + b1), all H columns (wave w: tiles w, w + 4, ...), into LDS as split fragments: the
    // lane's 4 columns c0 .. c0 + 3 of row l % 16 are elements 4 (j % 2) .. of 8-column group j / 2 of k-block
    // c0 / 32 (fragment lane l % 16 + 16 ((c0 % 32) / 8))
    for (int tile = wave; tile < H / 16; tile += 4) {
      const f32x4 acc = modin_mma(es, (const bf16_t*)a.t1_w, a.tdim, tile * 16, TKB, lane);
      const int c0 = tile * 16 + 4 * (lane >> 4);
      const f32x4 b1 = *reinterpret_cast<const f32x4*>(a.t1_b + c0);
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float x = acc[i] + b1[i];
        v[i] = x / (1.f + __expf(-x));
      }
      const int kb = c0 >> 5, fl = (lane & 15) + 16 * ((c0 & 31) >> 3), half8 = (c0 >> 2) & 1;
      uint32_t hi2[2], lo2[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const bf16_t h0 = f2bf(v[2 * e]), h1 = f2bf(v[2 * e + 1]);
        hi2[e] = (uint32_t)h0 | ((uint32_t)h1 << 16);
        lo2[e] = pack2(v[2 * e] - bf2f(h0), v[2 * e + 1] - bf2f(h1));
      }
      *reinterpret_cast<u32x2*>(hs + ((kb * 2 + 0) * 64 + fl) * 16 + half8 * 8) = u32x2{hi2[0], hi2[1]};
      *reinterpret_cast<u32x2*>(hs + ((kb * 2 + 1) * 64 + fl) * 16 + half8 * 8) = u32x2{lo2[0], lo2[1]};
    }
    __syncthreads();
    if (n0 < H) {
      const f32x4 acc = modin_mma(hs, (const bf16_t*)a.t2_w, H, n0, HKB, lane);
      const int k = k0 + (lane & 15), c0 = n0 + 4 * (lane >> 4);
      const f32x4 b2 = *reinterpret_cast<const f32x4*>(a.t2_b + c0);
      if (k < a.N) {
        for (int b = 0; b < a.B; ++b) {
          const f32x4 sc = *reinterpret_cast<const f32x4*>(a.state_cond + (int64_t)b * a.sc_stride + c0);
          f32x4 o;
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = (acc[i] + b2[i]) + sc[i];
          *reinterpret_cast<f32x4*>(a.out + (int64_t)b * a.out_stride_b + (int64_t)k * a.out_stride_k + c0) = o;
        }
      }
    }
  }
}

}  // namespace mkx
