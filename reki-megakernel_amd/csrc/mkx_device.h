// Device primitives for the mkx megakernel (gfx950 / CDNA4).
//
// Memory-coherence scheme (MI355X has 8 XCDs, each with its own L2; the L2s are not coherent with
// each other):
//  * Activations cross workgroups through write-once "frames": a producer writes with sc1 (device-scope,
//    write-through past its XCD's L2), and every frame address is written at most once per launch and
//    only read after every task that writes its cache line has published its ready epoch (below).
//    Consumers therefore read with ordinary loads: no L2 can hold a stale copy of a line that was never
//    read before all of its writers were done, and the L2 of each XCD de-duplicates the 32 CUs' reads of
//    the same activation rows. No cache writeback or invalidate (buffer_wbl2 / buffer_inv) is executed on
//    the hot path.
//  * Stages are ordered by per-task ready epochs (flag_publish / flag_wait): a consumer waits only for the
//    producer tasks whose output it reads. One grid barrier per launch remains, after the launch's first
//    stage (whose per-launch copies every later stage reads).
//  * The grid barrier is hierarchical and fence-free: each workgroup waits for its own stores to be
//    acknowledged, bumps its XCD's arrival counter with a device-scope atomic (the counter is shared by the
//    XCD's workgroups, so the HIP memory model asks for agent scope; it runs once per launch), the last
//    arrival of an XCD publishes the epoch with a device-scope store, and every workgroup polls the eight
//    per-XCD flags with device-scope loads. Counters are 64-bit and monotonic across launches, so nothing
//    is reset.
//  * Waits are bounded: a wait that exceeds its spin bound sets an error flag, and every later wait of the
//    launch returns immediately, so a broken launch still drains.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mkx {

typedef uint16_t bf16_t;
typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int NTHREADS = 256;
constexpr int NWAVES = 4;
constexpr int HD = 64;
constexpr int MAX_LAYERS = 32;
constexpr int MAX_BATCH = 16;
constexpr int MAX_XCD = 16;

// cache-policy bits of buffer / LDS-DMA instructions on gfx950
constexpr int CPOL_NONE = 0;
constexpr int CPOL_NT = 2;
constexpr int CPOL_SC1 = 16;

__device__ __forceinline__ float bf2f(bf16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ bf16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (bf16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);                                          // round to nearest even
  return (bf16_t)(u >> 16);
}
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }
__device__ __forceinline__ uint32_t pack2(float lo, float hi) { return (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
}
// 16-byte store, written through to the device coherence point (base must be wave-uniform)
__device__ __forceinline__ void st_sc1(void* base, uint32_t byte_off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, rsrc(base), byte_off, 0, CPOL_SC1);
}
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void st_sc1_b64(void* base, uint32_t byte_off, u32x2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(v, rsrc(base), byte_off, 0, CPOL_SC1);
}
__device__ __forceinline__ void st_sc1_b32(void* base, uint32_t byte_off, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, rsrc(base), byte_off, 0, CPOL_SC1);
}
__device__ __forceinline__ void st_sc1_b16(void* base, uint32_t byte_off, uint16_t v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, rsrc(base), byte_off, 0, CPOL_SC1);
}
// 16-byte device-coherent load
__device__ __forceinline__ u32x4 ld_sc1(const void* base, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(rsrc(base), byte_off, 0, CPOL_SC1);
}
// 16-byte ordinary load (frames, read-only inputs)
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

// LDS DMA: each lane copies 16 bytes from `src` to lds_base + 16 * lane (lds_base wave-uniform).
template <int CPOL = CPOL_NONE>
__device__ __forceinline__ void dma16(const void* src, void* lds_base) {
  __builtin_amdgcn_global_load_lds(src, (lds_void*)lds_base, 16, 0, CPOL);
}
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(0); }
// Waits until at most N of this wave's vector memory operations are outstanding: they complete in issue
// order, so every operation issued before the last N has completed (LDS DMAs included). Written as the
// builtin (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt and lgkmcnt at their no-wait maxima) so that
// the compiler's own wait-count tracking knows which loads are still pending and waits for the later ones
// one by one where they are used; the empty asm statements keep memory accesses from moving across it.
template <int N>
__device__ __forceinline__ void wait_vm_le() {
  static_assert(N >= 0 && N <= 63, "vmcnt is a 6-bit counter");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ unsigned xcc_id() {
  unsigned v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xf;
}
__device__ __forceinline__ long long clock100() { return (long long)__builtin_amdgcn_s_memrealtime(); }

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ f32x4 mfma16h(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Cross-lane sums and maxima in registers (no LDS round trip): DPP within a 16-lane row, the gfx950
// permlane swaps across rows. Each step adds a lane's value and its partner's, so both partners (and, at the
// end, all lanes of the group) hold bitwise the same result.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float lane_xor8(float v) { return dpp<0x128>(v); }  // row_ror:8 = lane ^ 8 within a row
__device__ __forceinline__ float quad_sum(float v) {
  v += dpp<0xB1>(v);  // quad_perm [1, 0, 3, 2]: lane ^ 1
  return v + dpp<0x4E>(v);  // quad_perm [2, 3, 0, 1]: lane ^ 2
}
__device__ __forceinline__ float row_sum16(float v) {
  v = quad_sum(v);
  v += dpp<0x141>(v);  // row_half_mirror: a lane of the other quad of the half-row (quads are uniform)
  return v + dpp<0x140>(v);  // row_mirror: a lane of the other half-row
}
__device__ __forceinline__ float xor16_sum(float v) {  // v[l] + v[l ^ 16]
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {  // v[l] + v[l ^ 32]
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float wave_sum(float v) { return xor32_sum(xor16_sum(row_sum16(v))); }

// ---------------------------------------------------------------------------------------------
// Error bits of BarState::err, each set with an atomic OR so that neither clears the other: a wait exceeded
// its spin bound (the launch's synchronisation is broken), or a GEMM operand exceeded the fp16 range (the
// launch completes and returns NaN).
constexpr int ERR_TIMEOUT = 1;
constexpr int ERR_RANGE = 2;

// grid barrier state (device memory, zeroed at handle creation)
struct BarState {
  unsigned long long arrive[MAX_XCD][32];   // per-XCD arrival counters (L2 atomics), 256 B apart
  unsigned long long done[MAX_XCD][512];    // per-XCD published epochs (device scope), 4 KB apart
  unsigned long long gen;                   // epoch base: stage boundaries passed by earlier launches
  unsigned long long pad0[15];
  int err;                                  // ERR_TIMEOUT | ERR_RANGE bits, set with atomic OR
  int pad1[31];
  unsigned long long arrivals_last;         // barriers x workgroups recorded by the last launch
};

// Ready epochs: flags[kind][task] holds the epoch (gen at launch start + stage + 1) of the last stage in
// which that producer task completed; a consumer task waits until the flags of exactly the producer tasks
// whose output lines it reads have reached its stage. 64-bit and monotonic across launches (a launch of
// `total` stages advances gen by total, so no flag of an earlier launch satisfies a later wait).
constexpr int FLAG_MAX = 2048;
constexpr int FLAG_STRIDE = 16;  // one 128-byte line per flag: no two writers share a line
enum FlagKind { F_TAIL_IN = 0, F_TAIL_OUT, F_QKV, F_SA, F_O, F_CA, F_CAO, F_GU, F_DPART, F_DOWN, FLAG_KINDS };

struct BarCtx {
  BarState* bs;
  unsigned long long* flags;  // [FLAG_KINDS][FLAG_MAX][FLAG_STRIDE]
  unsigned long long base;    // gen at launch start
  unsigned x;               // this workgroup's XCD
  unsigned nx;              // workgroups on this XCD
  unsigned xmask;           // XCDs that have workgroups
  unsigned spin_limit;
  bool failed;
};

__device__ __forceinline__ void bar_arrive(BarCtx& c, unsigned long long e) {
  wait_vm0();  // this wave's stores are acknowledged (sc1 stores have reached the coherence point)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long t = c.base + e;
    unsigned long long old =
        __hip_atomic_fetch_add(&c.bs->arrive[c.x][0], 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old + 1 == t * c.nx) __hip_atomic_store(&c.bs->done[c.x][0], t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

__device__ __forceinline__ void bar_wait(BarCtx& c, unsigned long long e) {
  if (threadIdx.x < 64 && !c.failed) {
    const unsigned long long t = c.base + e;
    const unsigned lane = threadIdx.x;
    unsigned n = 0;
    while (true) {
      bool ok = true;
      if (lane < MAX_XCD && ((c.xmask >> lane) & 1u))
        ok = __hip_atomic_load(&c.bs->done[lane][0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= t;
      if (__all(ok)) break;
      if (++n > c.spin_limit) {
        if (lane == 0) __hip_atomic_fetch_or(&c.bs->err, ERR_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        c.failed = true;
        break;
      }
    }
  }
  __syncthreads();
  // every wave learns whether wave 0 gave up (so later waits are skipped uniformly)
  __shared__ int s_failed;
  if (threadIdx.x == 0) s_failed = c.failed ? 1 : 0;
  __syncthreads();
  c.failed = s_failed != 0;
}

// Execution barrier of the workgroup that orders no memory operation: waves whose LDS DMAs (the prefetch of
// a later phase) are still in flight pass it without waiting for them (__syncthreads' workgroup fences make
// every wave wait for its outstanding DMAs first). The empty asm statements keep the compiler from moving
// memory accesses across it.
__device__ __forceinline__ void exec_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// publish: every wave's stores of the task have been acknowledged (write-through, so they are at the
// device coherence point), then one device-scope store of the task's ready epoch
__device__ __forceinline__ void flag_publish(BarCtx& c, int kind, int idx, unsigned long long e) {
  wait_vm0();
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_store(&c.flags[((long long)kind * FLAG_MAX + idx) * FLAG_STRIDE], c.base + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// wait until flags[kind][idx(i)] >= base + e for every i < n (n <= 64 NCH): wave 0 polls them all, 64 per
// device-scope load, each poll one round trip; the workgroup proceeds together. Bounded like bar_wait (only
// wave 0 polls, so only wave 0 tracks whether a wait gave up). Waits whose n is bounded by 64 use NCH = 1.
template <int NCH = 4, class F>
__device__ __forceinline__ void flag_wait(BarCtx& c, int kind, int n, F idx, unsigned long long e) {
  if (threadIdx.x < 64 && !c.failed) {
    const unsigned long long t = c.base + e;
    const int lane = (int)threadIdx.x;
    const unsigned long long* fp[NCH];
#pragma unroll
    for (int k = 0; k < NCH; ++k) fp[k] = c.flags + ((long long)kind * FLAG_MAX + idx(min(k * 64 + lane, n - 1))) * FLAG_STRIDE;
    const int nch = (n + 63) / 64;
    unsigned spins = 0;
    while (true) {
      unsigned long long v[NCH];
#pragma unroll
      for (int k = 0; k < NCH; ++k)
        v[k] = k < nch ? __hip_atomic_load(fp[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : t;
      bool ok = true;
#pragma unroll
      for (int k = 0; k < NCH; ++k) ok = ok && v[k] >= t;
      if (__all(ok)) break;
      if (++spins > c.spin_limit) {
        if (lane == 0) __hip_atomic_fetch_or(&c.bs->err, ERR_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        c.failed = true;
        break;
      }
    }
  }
  exec_barrier();
}

}  // namespace mkx
