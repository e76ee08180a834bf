// Register-memory ring append: the step after an expert call moves the call's register rows into the
// memory rows the next call attends to.
//
// Memory of one sample and layer is PM rows [PM, NH, 64] bf16, rows [kv_start, PM) valid, K normed and
// rotated at its row index. Appending R rows drops the oldest R: new row j is old row j + R for
// j < PM - R (K turned back by R positions), or the call's register row j - (PM - R) (K turned from its
// position in the call to row j); kv_start becomes max(kv_start - R, 0) and rows below it are zeroed.
// With PM = F R this keeps the register rows of the last F calls (frames). Reference: the memory fields
// the expert reads (src/mk_expert.py:489-490, kv_start = cu_kv[0] at :321) and the per-frame append
// REKI's register cache performs after each call (results/opt/breakdown_mk_fasthost_cprefill.json:116).
//
// The kernel is a streaming copy (HBM-bound): 4 lanes per 64-element head row, each moving the 16-byte
// chunk at d = 8q and its RoPE partner at d + 32, so a rotation needs no exchange between lanes.
#pragma once

#include "mkx.h"
#include "mkx_kernel.h"  // unpack8 (8 bf16 -> fp32)

namespace mkx {

constexpr int RING_BLOCK = 256;

// Rotate-half RoPE by a fixed angle per dimension, in fp32 without contraction (two products, then one
// sum), the order an fp32 restatement x * cos + rotate_half(x) * sin evaluates it in.
__device__ __forceinline__ void ring_rotate(float* lo, float* hi, const float* c, const float* s, int d0) {
#pragma clang fp contract(off)
  for (int i = 0; i < 8; ++i) {
    const float a = lo[i], b = hi[i];
    const float pa = a * c[d0 + i], pb = b * s[d0 + i];
    const float qb = b * c[d0 + 32 + i], qa = a * s[d0 + 32 + i];
    lo[i] = pa - pb;
    hi[i] = qb + qa;
  }
}

__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 v;
  for (int i = 0; i < 4; ++i) v[i] = pack2(f[2 * i], f[2 * i + 1]);
  return v;
}

// grid: x over PM * NH * 4 lanes, y = layer * 2 + (0: K, 1: V), z = sample
__global__ __launch_bounds__(RING_BLOCK) void ring_append_kernel(mkx_ring_args a) {
  const int lane = blockIdx.x * RING_BLOCK + threadIdx.x;
  const int l = blockIdx.y >> 1, is_v = blockIdx.y & 1, b = blockIdx.z;
  const int NH = a.NH, PM = a.PM, R = a.R;
  if (lane >= PM * NH * 4) return;
  const int q = lane & 3, hr = lane >> 2;
  const int h = hr % NH, j = hr / NH;
  const int ks_new = max(min(max(a.kv_start_in[b], 0), PM) - R, 0);  // kv_start outside [0, PM] is clamped
  const int64_t row = (int64_t)NH * 64;
  bf16_t* out = (bf16_t*)(is_v ? a.memv_out[l] : a.memk_out[l]) + b * a.mem_stride_b + j * row + h * 64;
  if (l == 0 && !is_v && lane == 0) a.kv_start_out[b] = ks_new;
  if (j < ks_new) {
    const u32x4 z = {0u, 0u, 0u, 0u};
    *reinterpret_cast<u32x4*>(out + 8 * q) = z;
    *reinterpret_cast<u32x4*>(out + 32 + 8 * q) = z;
    return;
  }
  const bf16_t* src;
  const float *c, *s;
  if (j < PM - R) {
    src = (const bf16_t*)(is_v ? a.memv_in[l] : a.memk_in[l]) + b * a.mem_stride_b + (j + R) * row + h * 64;
    c = a.shift_cos;
    s = a.shift_sin;
  } else {
    const int r = j - (PM - R);
    src = (const bf16_t*)(is_v ? a.cur_v : a.cur_k) + (((int64_t)(l * a.B + b) * R + r) * NH + h) * 64;
    c = a.new_cos;
    s = a.new_sin;
  }
  u32x4 vlo = ld16(src + 8 * q), vhi = ld16(src + 32 + 8 * q);
  if (!is_v && c != nullptr) {
    float lo[8], hi[8];
    unpack8(vlo, lo);
    unpack8(vhi, hi);
    ring_rotate(lo, hi, c, s, 8 * q);
    vlo = pack8(lo);
    vhi = pack8(hi);
  }
  *reinterpret_cast<u32x4*>(out + 8 * q) = vlo;
  *reinterpret_cast<u32x4*>(out + 32 + 8 * q) = vhi;
}

}  // namespace mkx
