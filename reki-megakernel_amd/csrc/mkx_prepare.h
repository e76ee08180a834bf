// Cross-attention source K/V preparation: per layer, the VLM context projected onto the expert's
// cross-attention K and V, K normed per head (weight 1 + w) and rotated (rotate-half RoPE at the source
// positions), bf16 [B, SP, NH, 64] with rows >= ca_len zero — the caches the megakernel reads as
// past.cross_attn_kv (src/mk_expert.py:491-492), produced by REKI's register_prepare (README.md:279-281:
// "the cross-attention K/V projections of the VLM source (31 M weights)").
//
// One workgroup = 64 source rows x one head (64 columns) of K or V of one layer; 4 waves of 16 rows. The
// product runs on v_mfma_f32_16x16x32_bf16 with the weight rows as the first operand, so a lane ends with
// 4 consecutive columns of each 16-column group for one source row: the RMS of a row is a sum over the
// lane's 16 values and two cross-lane swaps, and each column's RoPE partner (d +- 32) sits in the same
// lane. Both operands are read in fragment order, one 1 KB contiguous block per wave and load: the
// weights are packed so once at creation and the context at each call (pack_rows_kernel). Read in place,
// the rows of a fragment sit C * 2 bytes apart and the same kernel ran 2.6x slower (221 us against 84 us
// for 10 layers of a 300 x 2048 context). Chunks of 2 k-steps keep it at 80 VGPRs, so a whole grid of that
// size is resident at once (75 us; chunks of 4: 132 VGPRs, 83 us).
#pragma once

#include "mkx.h"
#include "mkx_device.h"

namespace mkx {

constexpr int PREP_BLOCK = 256;

// Fragment-order packing of a row-major bf16 matrix [rows, C]: out[g][t][j][lane][8] = in[row][k .. k + 8)
// with row = (g * S + j) * 16 + (lane & 15), k = 32 t + 8 (lane >> 4); rows >= nrows are zero. One thread
// per 16-byte output piece (n_out pieces).
__global__ __launch_bounds__(256) void pack_rows_kernel(const bf16_t* __restrict__ in, bf16_t* __restrict__ out,
                                                        int nrows, int C, int S, long long n_out) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n_out) return;
  const int lane = (int)(i & 63);
  const long long q = i >> 6;
  const int T = C / 32;
  const int j = (int)(q % S);
  const long long gt = q / S;
  const int t = (int)(gt % T);
  const long long g = gt / T;
  const long long row = (g * S + j) * 16 + (lane & 15);
  u32x4 v = {0u, 0u, 0u, 0u};
  if (row < nrows) v = ld16(in + row * C + 32 * t + 8 * (lane >> 4));
  *reinterpret_cast<u32x4*>(out + i * 8) = v;
}

struct SourceParams {
  int L, NH, C, B, SP;
  const bf16_t* ctxp;   // context in fragment order, S = 1, rows padded to a multiple of 64
  const bf16_t* wkp;    // K weights in fragment order, S = 4 (16-row groups of one head)
  const bf16_t* wvp;
  const bf16_t* k_norm; // [L, 64]
  const int32_t* ca_len;
  const float* cos; const float* sin;
  void* kca[MKX_MAX_LAYERS]; void* vca[MKX_MAX_LAYERS];
  long long src_sb;
  float eps;
};

// grid: x = ceil(B * SP / 64) row tiles, y = (layer * 2 + (0: K, 1: V)) * NH + head
__global__ __launch_bounds__(PREP_BLOCK) void prepare_source_kernel(SourceParams a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int NH = a.NH, C = a.C;
  const int h = blockIdx.y % NH, lk = blockIdx.y / NH, l = lk >> 1, is_v = lk & 1;
  const int nrows = a.B * a.SP;
  const int row = blockIdx.x * 64 + wave * 16 + (lane & 15);
  const int rowc = min(row, nrows - 1);  // rows past the end (zero in the packed context) are not stored
  const int T = C / 32;
  const bf16_t* xp = a.ctxp + ((int64_t)(blockIdx.x * 4 + wave) * T * 64 + lane) * 8;
  const bf16_t* wbase = (is_v ? a.wvp : a.wkp) + ((int64_t)(l * NH + h) * T * 4 * 64 + lane) * 8;
  f32x4 acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // k in chunks of KU steps of 32, two chunks in flight: the loads of chunk c + 1 are issued before the
  // MFMAs of chunk c. Steps past C load the last valid step (in bounds) and multiply a zeroed context
  // fragment, so every wave runs the same straight-line code.
  constexpr int KU = 2;
  u32x4 xs[2][KU], ws[2][KU][4];
  auto load = [&](int buf, int k0) {
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int k = min(k0 + 32 * u, C - 32);
      xs[buf][u] = ld16(xp + (int64_t)(k / 32) * 64 * 8);
#pragma unroll
      for (int j = 0; j < 4; ++j) ws[buf][u][j] = ld16(wbase + ((int64_t)(k / 32) * 4 + j) * 64 * 8);
    }
  };
  auto mma = [&](int buf, int k0) {
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const bool in = k0 + 32 * u < C;
      u32x4 xv = xs[buf][u];
#pragma unroll
      for (int e = 0; e < 4; ++e) xv[e] = in ? xv[e] : 0u;
      const bf16x8 xf = __builtin_bit_cast(bf16x8, xv);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = mfma16(__builtin_bit_cast(bf16x8, ws[buf][u][j]), xf, acc[j]);
    }
  };
  constexpr int CH = 32 * KU;
  load(0, 0);
  for (int k0 = 0; k0 < C; k0 += 2 * CH) {
    load(1, k0 + CH);
    mma(0, k0);
    load(0, k0 + 2 * CH);
    mma(1, k0 + CH);
  }
  // lane holds columns d = 16 j + 4 (lane >> 4) + i of source row `row`
  const int b = rowc / a.SP, s = rowc - b * a.SP;
  const bool live = s < min(max(a.ca_len[b], 0), a.SP);
  float y[4][4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) y[j][i] = rbf(acc[j][i]);
  if (!is_v) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) ss += y[j][i] * y[j][i];
    ss = xor32_sum(xor16_sum(ss));
    const float r = rsqrtf(ss / 64.f + a.eps);
    const bf16_t* wn = a.k_norm + l * 64;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 16 * j + 4 * (lane >> 4) + i;
        y[j][i] = rbf(y[j][i] * r * (1.f + bf2f(wn[d])));
      }
    const float* cs = a.cos + (int64_t)s * 64;
    const float* sn = a.sin + (int64_t)s * 64;
    float z[4][4];
    {
#pragma clang fp contract(off)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = 16 * j + 4 * (lane >> 4) + i;
          const float rot = j < 2 ? -y[j + 2][i] : y[j - 2][i];
          z[j][i] = rbf(y[j][i] * cs[d] + rot * sn[d]);
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) y[j][i] = z[j][i];
  }
  if (row >= nrows) return;
  bf16_t* out = (bf16_t*)(is_v ? a.vca[l] : a.kca[l]) + (int64_t)b * a.src_sb + ((int64_t)s * NH + h) * 64;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    u32x2 v;
    v[0] = live ? pack2(y[j][0], y[j][1]) : 0u;
    v[1] = live ? pack2(y[j][2], y[j][3]) : 0u;
    *reinterpret_cast<u32x2*>(out + 16 * j + 4 * (lane >> 4)) = v;
  }
}

}  // namespace mkx
