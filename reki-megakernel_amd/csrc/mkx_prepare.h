// Cross-attention source K/V preparation: per layer, the VLM context projected onto the expert's
// cross-attention K and V, K normed per head (weight 1 + w) and rotated (rotate-half RoPE at the source
// positions), bf16 [B, SP, NH, 64] with rows >= ca_len zero — the caches the megakernel reads as
// past.cross_attn_kv (src/mk_expert.py:491-492), produced by REKI's register_prepare (README.md:279-281:
// "the cross-attention K/V projections of the VLM source (31 M weights)").
//
// The product runs on v_mfma_f32_16x16x32_bf16 with the weight rows as the first operand, so a lane ends
// with 4 consecutive columns of each 16-column group for one source row: the RMS of a row is a sum over the
// lane's 16 values and two cross-lane swaps, and each column's RoPE partner (d +- 32) sits in the same
// lane. Both operands are read in fragment order, one contiguous 1 KB block per fragment: the weights are
// packed so once at creation and the context at each call (pack_rows_kernel). A workgroup stages the
// fragments of each k-block in LDS once and shares them between its waves (below); when every wave streamed
// its own weight fragments from memory (64 rows x one head per workgroup, no LDS), the four waves of a
// workgroup read each weight fragment four times and the kernel took 75 us for 10 layers of a 300 x 2048
// context, 10 % of the MFMA peak.
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
  const bf16_t* ctxp;   // context in fragment order, S = 2 RTW (one group per workgroup), rows padded to whole groups
  const bf16_t* wkp;    // K weights in fragment order, S = 4 (16-row groups of one head)
  const bf16_t* wvp;
  const bf16_t* k_norm; // [L, 64]
  const int32_t* ca_len;
  const float* cos; const float* sin;
  void* kca[MKX_MAX_LAYERS]; void* vca[MKX_MAX_LAYERS];
  long long src_sb;
  float eps;
};

// Row tiles of 16 per wave (the workgroup covers 2 * RTW of them, 32 * RTW rows): the packed context is padded
// to PREP_ROW_PAD more rows than the largest workgroup covers.
constexpr int PREP_ROW_PAD = 32 * 5;
constexpr int PREP_XCDS = 8;  // XCDs the dispatcher deals consecutive workgroups to

// grid: x = row groups of 32 * RTW rows, y = (layer * 2 + (0: K, 1: V)) * ceil(NH / 2) + head pair.
// Workgroup = 32 RTW source rows x two heads (128 columns) of K or V of one layer; wave (wr, wc) computes
// rows [16 RTW wr, 16 RTW (wr + 1)) of head 2 * pair + wc. Each k-block's operand fragments (2 RTW context
// fragments, 8 weight fragments, each a contiguous 1 KB block) are loaded into registers PV k-blocks ahead,
// each wave 16 bytes per lane of its share, then written to one of two LDS stages and shared by the waves:
// each weight fragment is read from memory once per workgroup and shared by its 2 RTW row tiles, and each
// context fragment serves the two heads. Per k-block a wave reads RTW + 4 fragments from LDS for 4 RTW
// MFMAs. The products are accumulated over k in order, exactly as a single wave streaming its operands would.
// TK > 0: the k-loop over TK k-blocks fully unrolled (the production context width), so that the compiler's
// wait counts follow each k-block's loads instead of draining them at a loop head; TK = 0: any C / 32.
template <int RTW, int TK>
__global__ __launch_bounds__(PREP_BLOCK) void prepare_source_kernel(SourceParams a) {
  constexpr int NXF = 2 * RTW, NF = NXF + 8;      // fragments per k-block: context, then weights
  constexpr int ND = (NF + 3) / 4;                // fragments per wave and k-block (past NF: repeats of fragment 0)
  constexpr int STAGE = (4 * ND) * 1024;          // bytes per LDS stage (a repeat lands past the real fragments)
  constexpr int PV = 4;                           // k-blocks of loads in flight
  __shared__ __attribute__((aligned(1024))) char sm[2 * STAGE];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, wr = wave >> 1, wc = wave & 1;
  const int NH = a.NH, C = a.C, T = TK > 0 ? TK : C / 32, NP = (NH + 1) / 2;
  // XCD-aware order: consecutive workgroups run on different XCDs (round-robin dispatch), so the linear index
  // is regrouped to give each XCD a contiguous run of (column group, row group) tiles, row group fastest: the
  // row groups of one column group then share its weight fragments (and the context rows) in their XCD's L2.
  const int ngr = gridDim.x, nwg = ngr * gridDim.y, lin = blockIdx.y * ngr + blockIdx.x;
  const int nfull = nwg - nwg % PREP_XCDS, per = nfull / PREP_XCDS;
  const int tix = lin < nfull ? (lin % PREP_XCDS) * per + lin / PREP_XCDS : lin;
  const int rg = tix % ngr, cgp = tix / ngr;
  const int pair = cgp % NP, lk = cgp / NP, l = lk >> 1, is_v = lk & 1;
  const int h = min(2 * pair + wc, NH - 1);
  const bool head_ok = 2 * pair + wc < NH;
  const int nrows = a.B * a.SP;
  const int g0 = rg * NXF;  // first 16-row tile of the workgroup
  const bf16_t* wsrc = is_v ? a.wvp : a.wkp;
  // this wave's fragment sources at k-block 0 (fragment f = wave + 4 i; f >= NF: a repeat of fragment 0) and
  // the element stride between consecutive k-blocks
  const bf16_t* src[ND];
  int kstride[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i) {
    const int f = wave + 4 * i;
    if (f < NXF) {
      src[i] = a.ctxp + (((int64_t)rg * T * NXF + f) * 64 + lane) * 8;
      kstride[i] = NXF * 64 * 8;
    } else if (f < NF) {
      const int hw = min(2 * pair + (f - NXF) / 4, NH - 1), j = (f - NXF) & 3;
      src[i] = wsrc + (((int64_t)(l * NH + hw) * T * 4 + j) * 64 + lane) * 8;
      kstride[i] = 4 * 64 * 8;
    } else {
      src[i] = a.ctxp + ((int64_t)rg * T * NXF * 64 + lane) * 8;
      kstride[i] = NXF * 64 * 8;
    }
  }
  u32x4 rgb[PV][ND];
  auto load = [&](int slot, int kb) {
    const int k = min(kb, T - 1);  // k-blocks past the end reload the last one, never stored
#pragma unroll
    for (int i = 0; i < ND; ++i) rgb[slot][i] = ld16(src[i] + (int64_t)k * kstride[i]);
  };
#pragma unroll
  for (int s = 0; s < PV; ++s) load(s, s);
  f32x4 acc[RTW][4];
#pragma unroll
  for (int rt = 0; rt < RTW; ++rt)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[rt][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // k-block kb: its fragments (loaded PV k-blocks earlier) into LDS stage kb % 2, the slot's next loads, a
  // barrier (every wave's fragments of kb are in LDS; the stage written was last read at kb - 2, before the
  // previous barrier), then the MFMAs
  auto step = [&](int slot, int kb) {
    char* st = sm + (kb & 1) * STAGE;
#pragma unroll
    for (int i = 0; i < ND; ++i) *reinterpret_cast<u32x4*>(st + (wave + 4 * i) * 1024 + lane * 16) = rgb[slot][i];
    load(slot, kb + PV);
    __syncthreads();
    bf16x8 xf[RTW], wf[4];
#pragma unroll
    for (int rt = 0; rt < RTW; ++rt) xf[rt] = *reinterpret_cast<const bf16x8*>(st + (wr * RTW + rt) * 1024 + lane * 16);
#pragma unroll
    for (int j = 0; j < 4; ++j) wf[j] = *reinterpret_cast<const bf16x8*>(st + (NXF + wc * 4 + j) * 1024 + lane * 16);
#pragma unroll
    for (int rt = 0; rt < RTW; ++rt)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[rt][j] = mfma16(wf[j], xf[rt], acc[rt][j]);
  };
  if constexpr (TK > 0) {
#pragma unroll
    for (int kb = 0; kb < TK; ++kb) step(kb % PV, kb);
  } else {
    for (int kb0 = 0; kb0 < T; kb0 += PV) {
#pragma unroll
      for (int u = 0; u < PV; ++u)
        if (kb0 + u < T) step(u, kb0 + u);
    }
  }
  wait_vm0();  // no load is in flight when the workgroup ends
  // the K norm weights of this lane's 16 columns d = 16 j + 4 (lane >> 4) + i (4 bf16 per j)
  uint2 wnv[4];
  if (!is_v) {
#pragma unroll
    for (int j = 0; j < 4; ++j) wnv[j] = *reinterpret_cast<const uint2*>(a.k_norm + l * 64 + 16 * j + 4 * (lane >> 4));
  }
#pragma unroll
  for (int rt = 0; rt < RTW; ++rt) {
    // lane holds columns d = 16 j + 4 (lane >> 4) + i of source row `row`
    const int row = (g0 + wr * RTW + rt) * 16 + (lane & 15);
    const int rowc = min(row, nrows - 1);  // rows past the end (zero in the packed context) are not stored
    const int b = rowc / a.SP, s = rowc - b * a.SP;
    // the row's loads are issued together: its sample's valid length and its RoPE table entries
    const int cal = a.ca_len[b];
    f32x4 csv[4], snv[4];
    if (!is_v) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        csv[j] = *reinterpret_cast<const f32x4*>(a.cos + (int64_t)s * 64 + 16 * j + 4 * (lane >> 4));
        snv[j] = *reinterpret_cast<const f32x4*>(a.sin + (int64_t)s * 64 + 16 * j + 4 * (lane >> 4));
      }
    }
    float y[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) y[j][i] = rbf(acc[rt][j][i]);
    if (!is_v) {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) ss += y[j][i] * y[j][i];
      ss = xor32_sum(xor16_sum(ss));
      const float r = rsqrtf(ss / 64.f + a.eps);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float wv[4] = {__uint_as_float(wnv[j].x << 16), __uint_as_float(wnv[j].x & 0xffff0000u),
                             __uint_as_float(wnv[j].y << 16), __uint_as_float(wnv[j].y & 0xffff0000u)};
#pragma unroll
        for (int i = 0; i < 4; ++i) y[j][i] = rbf(y[j][i] * r * (1.f + wv[i]));
      }
      float z[4][4];
      {
#pragma clang fp contract(off)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float rot = j < 2 ? -y[j + 2][i] : y[j - 2][i];
            z[j][i] = rbf(y[j][i] * csv[j][i] + rot * snv[j][i]);
          }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) y[j][i] = z[j][i];
    }
    const bool live = s < min(max(cal, 0), a.SP);
    if (row >= nrows || !head_ok) continue;
    bf16_t* out = (bf16_t*)(is_v ? a.vca[l] : a.kca[l]) + (int64_t)b * a.src_sb + ((int64_t)s * NH + h) * 64;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x2 v;
      v[0] = live ? pack2(y[j][0], y[j][1]) : 0u;
      v[1] = live ? pack2(y[j][2], y[j][3]) : 0u;
      *reinterpret_cast<u32x2*>(out + 16 * j + 4 * (lane >> 4)) = v;
    }
  }
}

}  // namespace mkx
