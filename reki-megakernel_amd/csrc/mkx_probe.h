// Micro-benchmarks of the megakernel's synchronisation primitives, run through mkx_probe (include/mkx.h):
// the reference times a barrier-only kernel to price its grid barrier (_barrier_only, src/tune_mk.py:28-33,
// timed at :66-68); the megakernel orders its stages with per-task ready epochs instead, so the second probe
// prices one producer -> consumer hand-off, the unit every stage boundary of a layer costs.
#pragma once
#include "mkx_device.h"

namespace mkx {

struct ProbeParams {
  BarState* bar;              // zeroed before each launch
  unsigned long long* flags;  // [FLAG_MAX][FLAG_STRIDE] ready epochs (kind 0), zeroed before each launch
  char* data;                 // hand-off buffers: hand-off i at data + i * bytes
  long long* out;             // [0] 100 MHz ticks of the timed region on workgroup 0, [1] checksum,
                              // [2], [3] the XCDs of workgroups 0 and 1
  unsigned nx[MAX_XCD];
  unsigned xmask;
  int n, fan;
  unsigned spin_limit;
};

__device__ __forceinline__ BarCtx probe_ctx(const ProbeParams& p) {
  BarCtx bc;
  bc.bs = p.bar;
  bc.flags = p.flags;
  bc.base = 0;
  bc.x = xcc_id();
  bc.nx = p.nx[bc.x];
  bc.xmask = p.xmask;
  bc.spin_limit = p.spin_limit;
  bc.failed = false;
  return bc;
}

// Every workgroup of the grid passes one aligning barrier, then n timed grid barriers (bar_arrive /
// bar_wait, the megakernel's barrier) with nothing between them.
__global__ void __launch_bounds__(NTHREADS, 1) barrier_probe_kernel(ProbeParams p) {
  BarCtx bc = probe_ctx(p);
  bar_arrive(bc, 1);
  bar_wait(bc, 1);
  const long long t0 = clock100();
  for (int i = 0; i < p.n; ++i) {
    bar_arrive(bc, 2 + (unsigned long long)i);
    bar_wait(bc, 2 + (unsigned long long)i);
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    p.out[0] = clock100() - t0;
    p.out[1] = 0;
  }
}

// A chain of n hand-offs between two groups of `fan` workgroups: workgroup 2 m + g is member m of group g
// (consecutive workgroups are dispatched to different XCDs, so producer and consumers never share an L2).
// Hand-off i: member 0 of group i % 2, the producer, stores PIECES x 4 KB write-through and publishes ready
// epoch 1 in flag i (flag_publish: its stores acknowledged first); every member of the other group waits
// for that flag (flag_wait: wave 0 polls, device-scope loads) and then loads all PIECES x 4 KB with ordinary
// loads, as a megakernel stage loads its operand. The consumer that is member 0 of its group produces
// hand-off i + 1 from what it loaded, so each hand-off starts when the previous one has been consumed.
// Workgroup 0 (member 0 of group 0) times the whole chain. Every wait is bounded, so the grid always drains.
template <int PIECES>
__global__ void __launch_bounds__(NTHREADS, 1) handoff_probe_kernel(ProbeParams p) {
  const int wg = blockIdx.x, tid = threadIdx.x;
  if (wg >= 2 * p.fan) return;
  const int grp = wg & 1, member = wg >> 1;
  BarCtx bc = probe_ctx(p);
  // no line of an earlier launch's hand-off buffers stays cached in this XCD's L2
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  __syncthreads();
  constexpr int BYTES = PIECES * NTHREADS * 16;
  u32x4 acc = {(unsigned)tid, 1u, 2u, 3u};
  const long long t0 = clock100();
  for (int i = 0; i < p.n; ++i) {
    char* d = p.data + (long long)i * BYTES;
    if (grp == (i & 1)) {
      if (member == 0) {
#pragma unroll
        for (int k = 0; k < PIECES; ++k) st_sc1(d, (uint32_t)((k * NTHREADS + tid) * 16), acc + (unsigned)k);
        flag_publish(bc, 0, i, 1);
      }
    } else {
      flag_wait<1>(bc, 0, 1, [&](int) { return i; }, 1);
      u32x4 v[PIECES];
#pragma unroll
      for (int k = 0; k < PIECES; ++k) v[k] = ld16(d + (k * NTHREADS + tid) * 16);
      u32x4 s = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int k = 0; k < PIECES; ++k) s += v[k];
      acc = s;
    }
  }
  if (wg == 0 && tid == 0) {
    p.out[0] = clock100() - t0;
    p.out[1] = (long long)(acc[0] ^ acc[3]);
  }
  if (wg < 2 && tid == 0) p.out[2 + wg] = (long long)bc.x;
}

}  // namespace mkx
