// The persistent megakernel: Euler steps of the flow-matching action expert in one launch.
//
// Schedule (mirrors expert_megakernel, src/mk_expert.py:302-426): an in-projection tail, then for each
// step and layer eight stages (QKV, self-attention, out-proj + gated residual, cross-attention query,
// cross-attention, out-proj + gated residual, gate/up, down + gated residual) and a step tail, each
// followed by a grid barrier: 1 + n_steps * (8 L + 1) barriers.
//
// Work decomposition for 256 CUs: every linear layer is cut into 16-column output tiles (one task per
// workgroup, K = H per task; the down projection is split over K into I/H tasks per tile whose fp32
// partials are summed in a fixed order by the last-arriving task). A workgroup prefetches the packed
// weight tile of its next task into LDS with 16-byte LDS DMA between arriving at a barrier and waiting on
// it, so weight streaming overlaps the barrier. GEMM A operands go straight from the activation frame
// into VGPRs (the AdaRMS prologue runs in registers) and the MFMA reads its B operand from LDS.
// Attention runs one workgroup per (sample, head).
//
// Numerics: bf16 MFMA inputs with fp32 accumulation; the residual stream (h0, h2, h3, h_l) and the gated
// branch added to it stay fp32 (the reference rounds both to bf16; keeping them fp32 halves the distance
// to the fp32 eager expert). q/k norms, RoPE, softmax probabilities, attention outputs and the MLP
// hidden are rounded to bf16 where the reference rounds them.
#pragma once
#include "mkx_device.h"

namespace mkx {

struct Params {
  // packed weights; per-layer strides in elements
  const bf16_t* wqkv; const bf16_t* wo; const bf16_t* wqca; const bf16_t* woca; const bf16_t* wgu; const bf16_t* wd;
  long long s_qkv, s_o, s_gu, s_d;
  const bf16_t* qn; const bf16_t* kn; const bf16_t* qcan;  // [L][64]
  const float* win; const float* bin; const float* wout; const float* bout;  // [A][H], [H], [A][H], [A]
  // call inputs
  const float* x_in; float* x_out;
  const float* mods; long long mods_sb, mods_ss; int mod_row0;
  const float* dt;
  const bf16_t* memk[MAX_LAYERS]; const bf16_t* memv[MAX_LAYERS]; long long mem_sb;
  const bf16_t* kca[MAX_LAYERS]; const bf16_t* vca[MAX_LAYERS]; long long src_sb;
  const int* kv_start; const int* ca_len;
  const float* sa_cos; const float* sa_sin; const float* ca_cos; const float* ca_sin;
  const bf16_t* reg_tok; bf16_t* cur_k; bf16_t* cur_v;
  int n_steps, action_dim, T, R, B, PM, SP, L, Mq, Mqp, NR, NRP, A, act;
  float eps, qk_eps, sm_scale;
  // scratch
  char* frames; long long frame_bytes;   // [n_steps * L] layer frames
  char* steps; long long step_bytes;     // [n_steps] step areas: h0 (fp32, tile-major) + x (fp32)
  unsigned* dcnt;                        // [H/16] split-K arrival counters
  BarState* bar; unsigned nx[MAX_XCD]; unsigned xmask;
  long long* prof; int profile;
  unsigned spin_limit;
};

// the kernel reads its parameters in place from the kernarg segment (constant address space), so the
// per-layer pointer tables are indexed with scalar loads and never copied to scratch
typedef const __attribute__((address_space(4))) Params CP;

__host__ __device__ constexpr int ceil_to(int a, int m) { return (a + m - 1) / m * m; }

template <int H_, int I_>
struct Shape {
  static constexpr int H = H_, I = I_, NH = H / HD, NKB = H / 32, HT = H / 16, IT = I / 16, SK = I / H;
  static constexpr int KPW = NKB / NWAVES;  // 32-wide k-blocks per wave
  static constexpr int WBUF = 0, WBUF_BYTES = 64 * 1024;
  static constexpr int ABUF = WBUF_BYTES, ABUF_BYTES = 72 * 1024;
  static constexpr int SMALL = ABUF + ABUF_BYTES, SMALL_BYTES = 4 * 1024;
  static constexpr int LDS = SMALL + SMALL_BYTES;
  static constexpr int RB_FIT = 144 / (KPW * 8);          // row tiles per GEMM pass held in VGPRs
  static constexpr int RBMAX = RB_FIT > 8 ? 8 : RB_FIT;
  static constexpr int MAXKT = (256 + 128) / 16;          // SA key tiles (PM <= 256, M_q <= 128)
  static_assert(H % 128 == 0 && I % H == 0, "H must be a multiple of 128 and I a multiple of H");
  static_assert(RBMAX >= 1, "row tile does not fit registers");
  static_assert(NKB * 1024 * 2 <= WBUF_BYTES, "gate/up weight tile pair must fit the weight buffer");
  static_assert(NWAVES * RBMAX * 2 * 1024 <= ABUF_BYTES, "cross-wave reduction must fit LDS");
  // frame layout (bytes), tile-major buffers [cols/16][NRP][16]; h2, h3, hl fp32, the rest bf16
  __host__ __device__ static long long qkv_off(int) { return 0; }
  __host__ __device__ static long long ysa_off(int nrp) { return (long long)nrp * 3 * H * 2; }
  __host__ __device__ static long long h2_off(int nrp) { return ysa_off(nrp) + (long long)nrp * H * 2; }
  __host__ __device__ static long long qca_off(int nrp) { return h2_off(nrp) + (long long)nrp * H * 4; }
  __host__ __device__ static long long yca_off(int nrp) { return qca_off(nrp) + (long long)nrp * H * 2; }
  __host__ __device__ static long long h3_off(int nrp) { return yca_off(nrp) + (long long)nrp * H * 2; }
  __host__ __device__ static long long g_off(int nrp) { return h3_off(nrp) + (long long)nrp * H * 4; }
  __host__ __device__ static long long hl_off(int nrp) { return g_off(nrp) + (long long)nrp * I * 2; }
  __host__ __device__ static long long part_off(int nrp) { return hl_off(nrp) + (long long)nrp * H * 4; }
  __host__ __device__ static long long frame_bytes(int nrp) { return part_off(nrp) + (long long)SK * nrp * H * 4; }
};

enum Stage { ST_QKV = 0, ST_SA, ST_O, ST_CAQ, ST_CA, ST_CAO, ST_GU, ST_DOWN, ST_TAIL };

template <class S>
struct Ctx {
  CP& p;
  char* smem;
  int wg, G, wave, lane, tid;
  float dt;
  __device__ Ctx(CP& p_, char* smem_) : p(p_), smem(smem_) {
    wg = blockIdx.x; G = gridDim.x; tid = threadIdx.x; wave = tid >> 6; lane = tid & 63;
  }
  __device__ char* frame(int s, int l) const { return p.frames + (long long)(s * p.L + l) * p.frame_bytes; }
  __device__ float* h0(int s) const { return (float*)(p.steps + (long long)s * p.step_bytes); }
  __device__ float* xstep(int s) const { return (float*)(p.steps + (long long)s * p.step_bytes + (long long)p.NRP * S::H * 4); }
  __device__ const float* h_in(int s, int l) const {
    return l == 0 ? h0(s) : (const float*)(frame(s, l - 1) + S::hl_off(p.NRP));
  }
  __device__ const float* modrow(int b, int s) const {
    return p.mods + (long long)b * p.mods_sb + (long long)(p.mod_row0 + s) * p.mods_ss;
  }
  __device__ int sample_of(int grow) const {
    int b = grow / p.Mqp;
    return b < p.B ? b : p.B - 1;
  }
};

// ------------------------------------------------------------------------------------------------
// helpers

// Weight chunks: packed 1 KB chunks, contiguous in HBM, copied to dst chunk by chunk.
template <class S>
__device__ __forceinline__ void dma_w(Ctx<S>& c, char* dst, const bf16_t* src, int nchunks) {
  for (int k = c.wave; k < nchunks; k += NWAVES) dma16(src + (long long)k * 512 + c.lane * 8, dst + k * 1024);
}

__device__ __forceinline__ void unpack8(u32x4 v, float* f) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f[2 * j] = __uint_as_float(v[j] << 16);
    f[2 * j + 1] = __uint_as_float(v[j] & 0xffff0000u);
  }
}
__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 v;
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = pack2(f[2 * j], f[2 * j + 1]);
  return v;
}
__device__ __forceinline__ u32x4 lds16(const char* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void sts16(char* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ void load8f(const float* p, float* f) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
  f[0] = a[0]; f[1] = a[1]; f[2] = a[2]; f[3] = a[3]; f[4] = b[0]; f[5] = b[1]; f[6] = b[2]; f[7] = b[3];
}
// 8 fp32 values (32 bytes) at element offset `off` of a frame buffer, written through (sc1)
__device__ __forceinline__ void st8f_sc1(float* base, long long off, const float* v) {
  st_sc1(base, (uint32_t)(off * 4), u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])});
  st_sc1(base, (uint32_t)(off * 4 + 16), u32x4{__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7])});
}

__device__ __forceinline__ float act_fn(float x, int gelu) {
  if (gelu) {
    const float k0 = 0.7978845608028654f, k1 = 0.044715f;
    return 0.5f * x * (1.0f + tanhf(k0 * (x + k1 * x * x * x)));
  }
  return x / (1.0f + __expf(-x));
}

// ------------------------------------------------------------------------------------------------
// GEMM stage: out tile (16 columns, all rows) = A @ W_tile^T for each task of this workgroup.
//   ADARMS: A = bf16(h * rstd(h) * (1 + scale) + shift) from the fp32 residual stream h
//           (src/mk_expert.py:93-122); otherwise A is a bf16 activation buffer.
//   KIND PLAIN: bf16 store (qkv, cross-attention query); RES: fp32 h_out = res + acc * gate
//   (src/mk_expert.py:162-172 without the roundings); GU: bf16 act(bf16 gate) * bf16 up
//   (:404-413); SPLIT: fp32 K-split partial, the last split of a tile sums the partials in split order
//   and applies RES.
// K (= H per task) is split over the 4 waves; the wave partials are summed through LDS.
enum { K_PLAIN = 0, K_RES = 1, K_GU = 2, K_SPLIT = 3 };

template <class S, int NT>
__device__ __forceinline__ void red_sum8(Ctx<S>& c, int r, int nt, int half, float* out) {
  const float* red = (const float*)(c.smem + S::ABUF);
  const int rt = r >> 4, rr = r & 15;
#pragma unroll
  for (int j = 0; j < 8; ++j) out[j] = 0.f;
#pragma unroll
  for (int w = 0; w < NWAVES; ++w) {
    const float* src = red + ((w * S::RBMAX + rt) * NT + nt) * 256 + rr * 16 + half * 8;
    const f32x4 a = *reinterpret_cast<const f32x4*>(src), b = *reinterpret_cast<const f32x4*>(src + 4);
    out[0] += a[0]; out[1] += a[1]; out[2] += a[2]; out[3] += a[3];
    out[4] += b[0]; out[5] += b[1]; out[6] += b[2]; out[7] += b[3];
  }
}

template <class S, int NT, int KIND, bool ADARMS>
__device__ void gemm_stage(Ctx<S>& c, int s, int ntask, const bf16_t* wbase, long long wtask_stride, const void* asrc,
                           int mod_off, void* out, const float* res, int gate_off, float* part, int split_tiles) {
  constexpr int KPW = S::KPW, RB = S::RBMAX;
  const int NRP = c.p.NRP;
  const int RT = NRP / 16;
  for (int t = c.wg; t < ntask; t += c.G) {
    int tile = t, split = 0;
    if (KIND == K_SPLIT) { tile = t % split_tiles; split = t / split_tiles; }
    if (t != c.wg) {  // later tasks of this workgroup: load their weights now (the first was prefetched)
      __syncthreads();
      const long long woff = KIND == K_SPLIT ? ((long long)tile * S::SK + split) * S::NKB * 512 : (long long)t * wtask_stride;
      dma_w(c, c.smem + S::WBUF, wbase + woff, NT * S::NKB);
    }
    const int k0 = split * S::H;
    for (int rt0 = 0; rt0 < RT; rt0 += RB) {
      const int nrt = min(RB, RT - rt0);
      const int row0 = rt0 * 16;
      bf16x8 a[RB][KPW];
      if (ADARMS) {
        const float* src = (const float*)asrc;
        float x[RB][KPW][8];
#pragma unroll
        for (int rt = 0; rt < RB; ++rt)
          if (rt < nrt) {
#pragma unroll
            for (int i = 0; i < KPW; ++i) {
              const int row = row0 + rt * 16 + (c.lane & 15);
              const int col = k0 + (c.wave + NWAVES * i) * 32 + 8 * (c.lane >> 4);
              load8f(src + ((long long)(col >> 4) * NRP + row) * 16 + (col & 15), x[rt][i]);
            }
          }
        float* ssq = (float*)(c.smem + S::SMALL);  // [4][RB*16]
#pragma unroll
        for (int rt = 0; rt < RB; ++rt)
          if (rt < nrt) {
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < KPW; ++i)
#pragma unroll
              for (int j = 0; j < 8; ++j) ss += x[rt][i][j] * x[rt][i][j];
            ss += __shfl_xor(ss, 16);
            ss += __shfl_xor(ss, 32);
            if (c.lane < 16) ssq[c.wave * RB * 16 + rt * 16 + c.lane] = ss;
          }
        wait_vm0();  // the weight tile (LDS DMA) has landed too
        __syncthreads();
#pragma unroll
        for (int rt = 0; rt < RB; ++rt)
          if (rt < nrt) {
            const int r = rt * 16 + (c.lane & 15);
            float tot = 0.f;
#pragma unroll
            for (int w = 0; w < NWAVES; ++w) tot += ssq[w * RB * 16 + r];
            const float rs = rsqrtf(tot / (float)S::H + c.p.eps);
            const float* mrow = c.modrow(c.sample_of(row0 + r), s) + mod_off;
#pragma unroll
            for (int i = 0; i < KPW; ++i) {
              const int col = (c.wave + NWAVES * i) * 32 + 8 * (c.lane >> 4);
              float sc[8], sh[8], v[8];
              load8f(mrow + col, sc);
              load8f(mrow + S::H + col, sh);
#pragma unroll
              for (int j = 0; j < 8; ++j) v[j] = x[rt][i][j] * rs * (1.0f + sc[j]) + sh[j];
              const u32x4 pk = pack8(v);
              a[rt][i] = *reinterpret_cast<const bf16x8*>(&pk);
            }
          }
      } else {
        const bf16_t* src = (const bf16_t*)asrc;
#pragma unroll
        for (int rt = 0; rt < RB; ++rt)
          if (rt < nrt) {
#pragma unroll
            for (int i = 0; i < KPW; ++i) {
              const int row = row0 + rt * 16 + (c.lane & 15);
              const int col = k0 + (c.wave + NWAVES * i) * 32 + 8 * (c.lane >> 4);
              a[rt][i] = *reinterpret_cast<const bf16x8*>(src + ((long long)(col >> 4) * NRP + row) * 16 + (col & 15));
            }
          }
        wait_vm0();
        __syncthreads();
      }
      f32x4 acc[RB][NT];
#pragma unroll
      for (int rt = 0; rt < RB; ++rt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[rt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < KPW; ++i) {
        const int kb = c.wave + NWAVES * i;
        bf16x8 w[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          w[nt] = *reinterpret_cast<const bf16x8*>(c.smem + S::WBUF + (nt * S::NKB + kb) * 1024 + c.lane * 16);
#pragma unroll
        for (int rt = 0; rt < RB; ++rt)
          if (rt < nrt) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) acc[rt][nt] = mfma16(a[rt][i], w[nt], acc[rt][nt]);
          }
      }
      // cross-wave reduction through LDS: red[w][rt][nt][16 rows][16 cols]
      float* red = (float*)(c.smem + S::ABUF);
#pragma unroll
      for (int rt = 0; rt < RB; ++rt)
        if (rt < nrt) {
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            float* base = red + ((c.wave * RB + rt) * NT + nt) * 256;
#pragma unroll
            for (int i = 0; i < 4; ++i) base[(4 * (c.lane >> 4) + i) * 16 + (c.lane & 15)] = acc[rt][nt][i];
          }
        }
      __syncthreads();
      // epilogue: one item = (row, 8 columns) of the task's 16-column tile
      for (int it = c.tid; it < nrt * 16 * 2; it += NTHREADS) {
        const int r = it >> 1, half = it & 1;
        const int grow = row0 + r;
        const int b = c.sample_of(grow);
        const long long ooff = ((long long)tile * NRP + grow) * 16 + half * 8;  // elements
        float v[8];
        red_sum8<S, NT>(c, r, 0, half, v);
        if (KIND == K_GU) {
          float u[8];
          red_sum8<S, NT>(c, r, NT - 1, half, u);
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = act_fn(rbf(v[j]), c.p.act) * rbf(u[j]);
          st_sc1(out, (uint32_t)(ooff * 2), pack8(v));
        } else if (KIND == K_PLAIN) {
          st_sc1(out, (uint32_t)(ooff * 2), pack8(v));
        } else if (KIND == K_RES) {
          float rv[8], g[8];
          load8f(res + ooff, rv);
          load8f(c.modrow(b, s) + gate_off + tile * 16 + half * 8, g);
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = rv[j] + v[j] * g[j];
          st8f_sc1((float*)out, ooff, v);
        } else {
          st8f_sc1(part, (((long long)split * split_tiles + tile) * NRP + grow) * 16 + half * 8, v);
        }
      }
      __syncthreads();  // red and ssq are reused by the next pass
    }
    if (KIND == K_SPLIT) {
      // the last-arriving split task of this tile sums the partials in split order and applies the residual
      const int SK = ntask / split_tiles;
      int* flag = (int*)(c.smem + S::SMALL + 3 * 1024);
      wait_vm0();
      __syncthreads();
      if (c.tid == 0) {
        const unsigned old = __hip_atomic_fetch_add(&c.p.dcnt[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = (old == (unsigned)(SK - 1));
        if (last) __hip_atomic_store(&c.p.dcnt[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = last;
      }
      __syncthreads();
      if (*flag) {
        for (int it = c.tid; it < NRP * 2; it += NTHREADS) {
          const int grow = it >> 1, half = it & 1;
          const int b = c.sample_of(grow);
          float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
          for (int j = 0; j < SK; ++j) {
            const long long poff = (((long long)j * split_tiles + tile) * NRP + grow) * 16 + half * 8;
            const u32x4 x0 = ld_sc1(part, (uint32_t)(poff * 4)), x1 = ld_sc1(part, (uint32_t)(poff * 4 + 16));
#pragma unroll
            for (int q = 0; q < 4; ++q) { v[q] += __uint_as_float(x0[q]); v[4 + q] += __uint_as_float(x1[q]); }
          }
          const long long ooff = ((long long)tile * NRP + grow) * 16 + half * 8;
          float rv[8], g[8];
          load8f(res + ooff, rv);
          load8f(c.modrow(b, s) + gate_off + tile * 16 + half * 8, g);
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = rv[j] + v[j] * g[j];
          st8f_sc1((float*)out, ooff, v);
        }
      }
    }
  }
}

// ------------------------------------------------------------------------------------------------
// Attention. Q/K chunk layout (rows x 64 d) -> chunk (rt, db) 1 KB, lane l = row rt*16 + l%16,
// d = db*32 + 8(l/16). Vt chunk (kb, dt): lane l holds V[key kb*32 + 8(l/16) + j][d = dt*16 + l%16], j < 8.

__device__ __forceinline__ int qk_chunk_off(int row, int d) {  // byte offset of 8 d-values (d % 8 == 0)
  return ((row >> 4) * 2 + (d >> 5)) * 1024 + ((row & 15) + 16 * ((d & 31) >> 3)) * 16;
}
__device__ __forceinline__ int vt_off(int key, int d) {  // byte offset of one bf16
  return ((key >> 5) * 4 + (d >> 4)) * 1024 + ((d & 15) + 16 * ((key & 31) >> 3)) * 16 + (key & 7) * 2;
}

// q/k head row (64 values in x): RMSNorm with weight 1 + w, bf16, rotate-half RoPE, bf16
// (src/mk_expert.py:175-193).
__device__ __forceinline__ void norm_rope64(float* x, const bf16_t* w, const float* cs, const float* sn, float eps) {
  float ss = 0.f;
#pragma unroll
  for (int d = 0; d < 64; ++d) ss += x[d] * x[d];
  const float r = rsqrtf(ss / 64.f + eps);
  float xn[64];
#pragma unroll
  for (int d = 0; d < 64; ++d) xn[d] = rbf(x[d] * r * (1.0f + bf2f(w[d])));
#pragma unroll
  for (int d = 0; d < 64; ++d) {
    const float rot = d < 32 ? -xn[d + 32] : xn[d - 32];
    x[d] = rbf(xn[d] * cs[d] + rot * sn[d]);
  }
}

// load 64 bf16 of row `grow`, columns [col0, col0+64) of a tile-major buffer
template <class S>
__device__ __forceinline__ void load_row64(Ctx<S>& c, const bf16_t* buf, int grow, int col0, float* x) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bf16_t* p = buf + ((long long)((col0 >> 4) + j) * c.p.NRP + grow) * 16;
    unpack8(ld16(p), x + 16 * j);
    unpack8(ld16(p + 8), x + 16 * j + 8);
  }
}

template <class S>
__device__ void sa_prefetch(Ctx<S>& c, int l, int b, int hd) {
  const int PM = c.p.PM, PMP = ceil_to(PM, 16);
  char* memK = c.smem + S::WBUF;
  char* memV = memK + PMP * 128;
  const bf16_t* mk = c.p.memk[l] + (long long)b * c.p.mem_sb;
  const bf16_t* mv = c.p.memv[l] + (long long)b * c.p.mem_sb;
  const int nk = (PMP / 16) * 2, nv = (PM + 7) / 8;
  for (int k = c.wave; k < nk + nv; k += NWAVES) {
    if (k < nk) {
      const int kt = k >> 1, db = k & 1;
      const int key = min(kt * 16 + (c.lane & 15), PM - 1);
      const int d = db * 32 + 8 * (c.lane >> 4);
      dma16(mk + ((long long)key * S::NH + hd) * HD + d, memK + k * 1024);
    } else {
      const int i = k - nk;
      const int key = min(i * 8 + (c.lane >> 3), PM - 1);
      dma16(mv + ((long long)key * S::NH + hd) * HD + (c.lane & 7) * 8, memV + i * 1024);
    }
  }
}

template <class S>
__device__ void sa_task(Ctx<S>& c, int s, int l, int b, int hd, const bf16_t* qkv, bf16_t* y, int kvs) {
  CP& p = c.p;
  const int M = p.Mq, PM = p.PM, PMP = ceil_to(PM, 16), NOWN = ceil_to(M, 16), NK = PMP + NOWN, NKP = ceil_to(NK, 32);
  char* memK = c.smem + S::WBUF;
  char* memV = memK + PMP * 128;
  char* Qc = c.smem + S::ABUF;
  char* Kown = Qc + NOWN * 128;
  char* Vt = Kown + NOWN * 128;
  char* Pst = Vt + NKP * 128 + c.wave * 1024;
  const bool want_kv = (s == 0 && p.cur_k != nullptr && p.R > 0);
  // own rows: q, k normed + rotated; v transposed
  for (int it = c.tid; it < 3 * M; it += NTHREADS) {
    const int kind = it / M, i = it % M;
    const int grow = b * p.Mqp + i;
    float x[64];
    load_row64(c, qkv, grow, kind * S::H + hd * HD, x);
    if (kind < 2) {
      norm_rope64(x, (kind == 0 ? p.qn : p.kn) + l * HD, p.sa_cos + i * HD, p.sa_sin + i * HD, p.qk_eps);
      char* dst = kind == 0 ? Qc : Kown;
#pragma unroll
      for (int d = 0; d < 64; d += 8) sts16(dst + qk_chunk_off(i, d), pack8(x + d));
      if (kind == 1 && want_kv && i >= p.T) {
        bf16_t* o = p.cur_k + ((((long long)l * p.B + b) * p.R + (i - p.T)) * S::NH + hd) * HD;
#pragma unroll
        for (int d = 0; d < 64; d += 8) *reinterpret_cast<u32x4*>(o + d) = pack8(x + d);
      }
    } else {
      if (want_kv && i >= p.T) {
        bf16_t* o = p.cur_v + ((((long long)l * p.B + b) * p.R + (i - p.T)) * S::NH + hd) * HD;
#pragma unroll
        for (int d = 0; d < 64; d += 8) *reinterpret_cast<u32x4*>(o + d) = pack8(x + d);
      }
      const int key = PMP + i;
#pragma unroll
      for (int d = 0; d < 64; ++d) *reinterpret_cast<bf16_t*>(Vt + vt_off(key, d)) = f2bf(x[d]);
    }
  }
  // memory V -> Vt (rows below kv_start are zero), zero the padded key slots
  for (int it = c.tid; it < NKP * 8; it += NTHREADS) {
    const int key = it >> 3, dg = (it & 7) * 8;
    if (key >= PMP && key < PMP + M) continue;
    float f[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (key < PM && key >= kvs) unpack8(lds16(memV + key * 128 + dg * 2), f);
#pragma unroll
    for (int j = 0; j < 8; ++j) *reinterpret_cast<bf16_t*>(Vt + vt_off(key, dg + j)) = f2bf(f[j]);
  }
  __syncthreads();
  const float scale = p.sm_scale;
  const int nkt = NK / 16;
  for (int qt = c.wave; qt < NOWN / 16; qt += NWAVES) {
    const bf16x8 qa0 = *reinterpret_cast<const bf16x8*>(Qc + (qt * 2 + 0) * 1024 + c.lane * 16);
    const bf16x8 qa1 = *reinterpret_cast<const bf16x8*>(Qc + (qt * 2 + 1) * 1024 + c.lane * 16);
    f32x4 sreg[S::MAXKT];
    float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
    for (int kt = 0; kt < S::MAXKT; ++kt) {
      if (kt < nkt) {
        const char* kc = kt < PMP / 16 ? memK + kt * 2048 : Kown + (kt - PMP / 16) * 2048;
        f32x4 sc = {0.f, 0.f, 0.f, 0.f};
        sc = mfma16(qa0, *reinterpret_cast<const bf16x8*>(kc + c.lane * 16), sc);
        sc = mfma16(qa1, *reinterpret_cast<const bf16x8*>(kc + 1024 + c.lane * 16), sc);
        const int key = kt * 16 + (c.lane & 15);
        const bool valid = (key >= kvs && key < PM) || (key >= PMP && key < PMP + M);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sc[i] = valid ? sc[i] * scale : -INFINITY;
          mx[i] = fmaxf(mx[i], sc[i]);
        }
        sreg[kt] = sc;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) mx[i] = fmaxf(mx[i], __shfl_xor(mx[i], o));
    float den[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < S::MAXKT; ++kt) {
      if (kt < nkt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float e = __expf(sreg[kt][i] - mx[i]);
          sreg[kt][i] = e;
          den[i] += e;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) den[i] += __shfl_xor(den[i], o);
    f32x4 acc[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < S::MAXKT / 2; ++kb) {
      if (kb < NKP / 32) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int kt = 2 * kb + h;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float pv = kt < nkt ? sreg[kt][i] : 0.f;
            *reinterpret_cast<bf16_t*>(Pst + (4 * (c.lane >> 4) + i) * 64 + (h * 16 + (c.lane & 15)) * 2) = f2bf(pv);
          }
        }
        const bf16x8 pa = *reinterpret_cast<const bf16x8*>(Pst + (c.lane & 15) * 64 + (c.lane >> 4) * 16);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
          acc[dt] = mfma16(pa, *reinterpret_cast<const bf16x8*>(Vt + (kb * 4 + dt) * 1024 + c.lane * 16), acc[dt]);
      }
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int q = qt * 16 + 4 * (c.lane >> 4) + i;
        if (q < M) {
          const int grow = b * p.Mqp + q;
          const long long off = ((long long)(hd * 4 + dt) * p.NRP + grow) * 16 + (c.lane & 15);
          st_sc1_b16(y, (uint32_t)(off * 2), f2bf(acc[dt][i] / den[i]));
        }
      }
    }
  }
}

// Cross-attention: K/V streamed in blocks of 64 source rows through a 4-slot LDS ring (16 KB per slot:
// K chunks then raw V rows), online softmax (src/mk_expert.py:225-251).
template <class S>
__device__ void ca_dma_block(Ctx<S>& c, int l, int b, int hd, int j) {
  const int SP = c.p.SP;
  char* slot = c.smem + S::WBUF + (j & 3) * 16384;
  const bf16_t* kb_ = c.p.kca[l] + (long long)b * c.p.src_sb;
  const bf16_t* vb_ = c.p.vca[l] + (long long)b * c.p.src_sb;
  for (int k = c.wave; k < 16; k += NWAVES) {
    if (k < 8) {
      const int kt = k >> 1, db = k & 1;
      const int key = min(j * 64 + kt * 16 + (c.lane & 15), SP - 1);
      dma16(kb_ + ((long long)key * S::NH + hd) * HD + db * 32 + 8 * (c.lane >> 4), slot + k * 1024);
    } else {
      const int i = k - 8;
      const int key = min(j * 64 + i * 8 + (c.lane >> 3), SP - 1);
      dma16(vb_ + ((long long)key * S::NH + hd) * HD + (c.lane & 7) * 8, slot + 8192 + i * 1024);
    }
  }
}

template <class S>
__device__ void ca_prefetch(Ctx<S>& c, int l, int b, int hd, int S_len) {
  const int nblk = (S_len + 63) / 64;
  for (int j = 0; j < min(nblk, 4); ++j) ca_dma_block(c, l, b, hd, j);
}

__device__ __forceinline__ void wait_vm_blocks(int younger) {
  // each ring block is 4 DMA instructions per wave
  switch (younger) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
  }
}

template <class S>
__device__ void ca_task(Ctx<S>& c, int s, int l, int b, int hd, const bf16_t* qca, bf16_t* y, int S_len) {
  CP& p = c.p;
  const int M = p.Mq, NOWN = ceil_to(M, 16);
  char* Qc = c.smem + S::ABUF;
  char* Vt = Qc + NOWN * 128;              // one block: 2 kb x 4 dt chunks = 8 KB
  char* Pst = Vt + 8192 + c.wave * 1024;
  for (int i = c.tid; i < M; i += NTHREADS) {
    float x[64];
    load_row64(c, qca, b * p.Mqp + i, hd * HD, x);
    norm_rope64(x, p.qcan + l * HD, p.ca_cos + i * HD, p.ca_sin + i * HD, p.qk_eps);
#pragma unroll
    for (int d = 0; d < 64; d += 8) sts16(Qc + qk_chunk_off(i, d), pack8(x + d));
  }
  const int nblk = (S_len + 63) / 64;
  constexpr int MAXQT = 2;  // query tiles per wave (M_q <= 128)
  float mrun[MAXQT][4], den[MAXQT][4];
  f32x4 acc[MAXQT][4];
#pragma unroll
  for (int u = 0; u < MAXQT; ++u)
#pragma unroll
    for (int i = 0; i < 4; ++i) { mrun[u][i] = -INFINITY; den[u][i] = 0.f; acc[u][i] = f32x4{0.f, 0.f, 0.f, 0.f}; }
  const float scale = p.sm_scale;
  for (int j = 0; j < nblk; ++j) {
    wait_vm_blocks(min(nblk, j + 4) - j - 1);
    __syncthreads();
    char* slot = c.smem + S::WBUF + (j & 3) * 16384;
    for (int it = c.tid; it < 64 * 8; it += NTHREADS) {
      const int kl = it >> 3, dg = (it & 7) * 8;
      float f[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      if (j * 64 + kl < S_len) unpack8(lds16(slot + 8192 + kl * 128 + dg * 2), f);
#pragma unroll
      for (int q = 0; q < 8; ++q) *reinterpret_cast<bf16_t*>(Vt + vt_off(kl, dg + q)) = f2bf(f[q]);
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < MAXQT; ++u) {
      const int qt = c.wave + NWAVES * u;
      if (qt < NOWN / 16) {
        const bf16x8 qa0 = *reinterpret_cast<const bf16x8*>(Qc + (qt * 2 + 0) * 1024 + c.lane * 16);
        const bf16x8 qa1 = *reinterpret_cast<const bf16x8*>(Qc + (qt * 2 + 1) * 1024 + c.lane * 16);
        f32x4 sb[4];
        float mb[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          f32x4 sc = {0.f, 0.f, 0.f, 0.f};
          sc = mfma16(qa0, *reinterpret_cast<const bf16x8*>(slot + (kt * 2 + 0) * 1024 + c.lane * 16), sc);
          sc = mfma16(qa1, *reinterpret_cast<const bf16x8*>(slot + (kt * 2 + 1) * 1024 + c.lane * 16), sc);
          const bool valid = j * 64 + kt * 16 + (c.lane & 15) < S_len;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            sc[i] = valid ? sc[i] * scale : -INFINITY;
            mb[i] = fmaxf(mb[i], sc[i]);
          }
          sb[kt] = sc;
        }
        float alpha[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int o = 1; o < 16; o <<= 1) mb[i] = fmaxf(mb[i], __shfl_xor(mb[i], o));
          const float mn = fmaxf(mrun[u][i], mb[i]);
          alpha[i] = __expf(mrun[u][i] - mn);
          mrun[u][i] = mn;
        }
        float ps[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float e = __expf(sb[kt][i] - mrun[u][i]);
            sb[kt][i] = e;
            ps[i] += e;
          }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int o = 1; o < 16; o <<= 1) ps[i] += __shfl_xor(ps[i], o);
          den[u][i] = den[u][i] * alpha[i] + ps[i];
        }
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[u][dt][i] *= alpha[i];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              *reinterpret_cast<bf16_t*>(Pst + (4 * (c.lane >> 4) + i) * 64 + (h * 16 + (c.lane & 15)) * 2) = f2bf(sb[2 * kb + h][i]);
          const bf16x8 pa = *reinterpret_cast<const bf16x8*>(Pst + (c.lane & 15) * 64 + (c.lane >> 4) * 16);
#pragma unroll
          for (int dt = 0; dt < 4; ++dt)
            acc[u][dt] = mfma16(pa, *reinterpret_cast<const bf16x8*>(Vt + (kb * 4 + dt) * 1024 + c.lane * 16), acc[u][dt]);
        }
      }
    }
    __syncthreads();
    if (j + 4 < nblk) ca_dma_block(c, l, b, hd, j + 4);
  }
#pragma unroll
  for (int u = 0; u < MAXQT; ++u) {
    const int qt = c.wave + NWAVES * u;
    if (qt < NOWN / 16) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int q = qt * 16 + 4 * (c.lane >> 4) + i;
          if (q < M) {
            const long long off = ((long long)(hd * 4 + dt) * p.NRP + b * p.Mqp + q) * 16 + (c.lane & 15);
            const float o = den[u][i] > 0.f ? acc[u][dt][i] / den[u][i] : 0.f;
            st_sc1_b16(y, (uint32_t)(off * 2), f2bf(o));
          }
        }
    }
  }
}

// ------------------------------------------------------------------------------------------------
// Step tail (src/mk_expert.py:254-299): o = bf16(AdaRMS_final(h_L)); v = o Wout^T + bout (fp32);
// x' = x_pad + dt v; h0' = x'_pad Win + bin (fp32). Tasks [0, H/16): in-projection tiles (they recompute
// the velocity of the real action dims); tasks [H/16, H/16 + A): one output dim each.
template <class S>
__device__ float tail_velocity_row(Ctx<S>& c, const float* hL, int grow, const float* mrow, int a, float* o16, bool have_o) {
  // one wave: lane < H/16 owns 16 columns; returns v_a (all lanes) given o in o16 (computed if !have_o)
  const int lane = c.lane;
  if (!have_o) {
    float x[16];
    float ss = 0.f;
    if (lane < S::HT) {
      const float* p = hL + ((long long)lane * c.p.NRP + grow) * 16;
      load8f(p, x);
      load8f(p + 8, x + 8);
#pragma unroll
      for (int j = 0; j < 16; ++j) ss += x[j] * x[j];
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) ss += __shfl_xor(ss, o);
    const float r = rsqrtf(ss / (float)S::H + c.p.eps);
    if (lane < S::HT) {
      const float* sc = mrow + lane * 16;
      const float* sh = mrow + S::H + lane * 16;
#pragma unroll
      for (int j = 0; j < 16; ++j) o16[j] = rbf(x[j] * r * (1.0f + sc[j]) + sh[j]);
    }
  }
  float d = 0.f;
  if (lane < S::HT) {
    const float* w = c.p.wout + (long long)a * S::H + lane * 16;
#pragma unroll
    for (int j = 0; j < 16; ++j) d += o16[j] * w[j];
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) d += __shfl_xor(d, o);
  return d + c.p.bout[a];
}

template <class S>
__device__ void tail_stage(Ctx<S>& c, int s, bool first, bool last, const float* hL) {
  CP& p = c.p;
  const int nin = last ? 0 : S::HT;
  const int nout = first ? 0 : p.A;
  const int nrows = p.B * p.T;
  const float* xcur = (first || s == 0) ? p.x_in : c.xstep(s);
  float* xp = (float*)(c.smem + S::ABUF);  // [nrows][action_dim] x' of the real dims
  for (int t = c.wg; t < nin + nout; t += c.G) {
    __syncthreads();
    if (t < nin) {
      const int adim = p.action_dim;
      for (int ri = c.wave; ri < nrows; ri += NWAVES) {
        const int b = ri / p.T, i = ri % p.T;
        float o16[16];
        if (first) {
          if (c.lane < adim) xp[ri * adim + c.lane] = xcur[(long long)ri * p.A + c.lane];
        } else {
          const float* mrow = c.modrow(b, s) + 9 * p.L * S::H;
          for (int a = 0; a < adim; ++a) {
            const float v = tail_velocity_row(c, hL, b * p.Mqp + i, mrow, a, o16, a > 0);
            if (c.lane == 0) xp[ri * adim + a] = xcur[(long long)ri * p.A + a] + c.dt * v;
          }
        }
      }
      __syncthreads();
      float* h0n = c.h0(first ? 0 : s + 1);
      for (int it = c.tid; it < p.NRP * 2; it += NTHREADS) {
        const int grow = it >> 1, half = it & 1;
        const int b = grow / p.Mqp, i = grow % p.Mqp;
        const int col = t * 16 + half * 8;
        float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (b < p.B && i < p.T) {
          const float* xr = xp + (b * p.T + i) * adim;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            float acc = 0.f;
            for (int a = 0; a < adim; ++a) acc += xr[a] * p.win[(long long)a * S::H + col + j];
            v[j] = acc + p.bin[col + j];
          }
        } else if (b < p.B && i < p.Mq) {
          unpack8(ld16(p.reg_tok + (long long)(i - p.T) * S::H + col), v);
        }
        st8f_sc1(h0n, ((long long)t * p.NRP + grow) * 16 + half * 8, v);
      }
    } else {
      const int a = t - nin;
      float* xn = last ? p.x_out : c.xstep(s + 1);
      for (int ri = c.wave; ri < nrows; ri += NWAVES) {
        const int b = ri / p.T, i = ri % p.T;
        float o16[16];
        const float* mrow = c.modrow(b, s) + 9 * p.L * S::H;
        const float v = tail_velocity_row(c, hL, b * p.Mqp + i, mrow, a, o16, false);
        if (c.lane == 0) {
          const float xa = a < p.action_dim ? xcur[(long long)ri * p.A + a] : 0.f;
          st_sc1_b32(xn, (uint32_t)(((long long)ri * p.A + a) * 4), __float_as_uint(xa + c.dt * v));
        }
      }
    }
  }
}

template <int H, int I>
__global__ void __launch_bounds__(NTHREADS, 1) mkx_megakernel(Params params) {
  using S = Shape<H, I>;
  __shared__ __attribute__((aligned(1024))) char smem[S::LDS];
  CP& p = *(CP*)(__builtin_amdgcn_kernarg_segment_ptr());
  Ctx<S> c(p, smem);
  c.dt = p.dt[0];
  int* s_ks = (int*)(smem + S::SMALL + 3 * 1024 + 64);  // kv_start[B], ca_len[B]
  if (c.tid < p.B) {
    s_ks[c.tid] = min(max(p.kv_start[c.tid], 0), p.PM);
    s_ks[MAX_BATCH + c.tid] = min(max(p.ca_len[c.tid], 0), p.SP);
  }
  BarCtx bc;
  bc.bs = p.bar;
  bc.x = xcc_id();
  bc.nx = p.nx[bc.x];
  bc.xmask = p.xmask;
  bc.spin_limit = p.spin_limit;
  bc.failed = false;
  bc.base = __hip_atomic_load(&p.bar->gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // one agent-scope acquire per launch: no cache of this XCD holds lines from before the launch
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  if (c.wg == 0 && c.tid < S::HT) __hip_atomic_store(&p.dcnt[c.tid], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  const int NRP = p.NRP;
  const int NBH = p.B * S::NH;
  unsigned long long e = 0;
  auto stamp = [&]() {
    if (p.profile && c.wg == 0 && c.tid == 0) p.prof[e] = clock100() * 10;
  };
  if (p.profile && c.wg == 0 && c.tid == 0) p.prof[0] = clock100() * 10;

  // prefetch of the constant operands of this workgroup's first task in a stage
  auto prefetch = [&](int s, int l, int st) {
    char* wb = smem + S::WBUF;
    const int t = c.wg;
    switch (st) {
      case ST_QKV: if (t < 3 * S::HT) dma_w(c, wb, p.wqkv + l * p.s_qkv + (long long)t * S::NKB * 512, S::NKB); break;
      case ST_SA: if (t < NBH) sa_prefetch(c, l, t / S::NH, t % S::NH); break;
      case ST_O: if (t < S::HT) dma_w(c, wb, p.wo + l * p.s_o + (long long)t * S::NKB * 512, S::NKB); break;
      case ST_CAQ: if (t < S::HT) dma_w(c, wb, p.wqca + l * p.s_o + (long long)t * S::NKB * 512, S::NKB); break;
      case ST_CA: if (t < NBH) ca_prefetch(c, l, t / S::NH, t % S::NH, s_ks[MAX_BATCH + t / S::NH]); break;
      case ST_CAO: if (t < S::HT) dma_w(c, wb, p.woca + l * p.s_o + (long long)t * S::NKB * 512, S::NKB); break;
      case ST_GU: if (t < S::IT) dma_w(c, wb, p.wgu + l * p.s_gu + (long long)t * 2 * S::NKB * 512, 2 * S::NKB); break;
      case ST_DOWN: if (t < S::HT * S::SK) {
          const int tile = t % S::HT, split = t / S::HT;
          dma_w(c, wb, p.wd + l * p.s_d + ((long long)tile * S::SK + split) * S::NKB * 512, S::NKB);
        } break;
      default: break;
    }
  };
  auto sync_next = [&](int s, int l, int st) {
    bar_arrive(bc, ++e);
    if (st >= 0) prefetch(s, l, st);
    bar_wait(bc, e);
    stamp();
  };

  // in-projection of the incoming x (src/mk_expert.py:326-327)
  tail_stage(c, 0, true, false, nullptr);
  sync_next(0, 0, ST_QKV);
  for (int s = 0; s < p.n_steps; ++s) {
    for (int l = 0; l < p.L; ++l) {
      char* fr = c.frame(s, l);
      const float* hin = c.h_in(s, l);
      bf16_t* qkv = (bf16_t*)(fr + S::qkv_off(NRP));
      bf16_t* ysa = (bf16_t*)(fr + S::ysa_off(NRP));
      float* h2 = (float*)(fr + S::h2_off(NRP));
      bf16_t* qca = (bf16_t*)(fr + S::qca_off(NRP));
      bf16_t* yca = (bf16_t*)(fr + S::yca_off(NRP));
      float* h3 = (float*)(fr + S::h3_off(NRP));
      bf16_t* g = (bf16_t*)(fr + S::g_off(NRP));
      float* hl = (float*)(fr + S::hl_off(NRP));
      float* part = (float*)(fr + S::part_off(NRP));
      const int m_sa = 9 * l * H, m_ca = m_sa + 3 * H, m_mlp = m_sa + 6 * H;
      // 1. qkv = bf16(AdaRMS(h) @ Wqkv^T)
      gemm_stage<S, 1, K_PLAIN, true>(c, s, 3 * S::HT, p.wqkv + l * p.s_qkv, S::NKB * 512, hin, m_sa, qkv, nullptr, 0, nullptr, 0);
      sync_next(s, l, ST_SA);
      // 2. self-attention per (sample, head)
      for (int t = c.wg; t < NBH; t += c.G) {
        if (t != c.wg) { __syncthreads(); sa_prefetch(c, l, t / S::NH, t % S::NH); }
        wait_vm0();
        __syncthreads();
        sa_task(c, s, l, t / S::NH, t % S::NH, qkv, ysa, s_ks[t / S::NH]);
        __syncthreads();
      }
      sync_next(s, l, ST_O);
      // 3. h2 = h + (y @ Wo^T) * gate_sa
      gemm_stage<S, 1, K_RES, false>(c, s, S::HT, p.wo + l * p.s_o, S::NKB * 512, ysa, 0, h2, hin, m_sa + 2 * H, nullptr, 0);
      sync_next(s, l, ST_CAQ);
      // 4. qca = bf16(AdaRMS_ca(h2) @ Wqca^T)
      gemm_stage<S, 1, K_PLAIN, true>(c, s, S::HT, p.wqca + l * p.s_o, S::NKB * 512, h2, m_ca, qca, nullptr, 0, nullptr, 0);
      sync_next(s, l, ST_CA);
      // 5. cross-attention per (sample, head)
      for (int t = c.wg; t < NBH; t += c.G) {
        if (t != c.wg) { __syncthreads(); ca_prefetch(c, l, t / S::NH, t % S::NH, s_ks[MAX_BATCH + t / S::NH]); }
        __syncthreads();
        ca_task(c, s, l, t / S::NH, t % S::NH, qca, yca, s_ks[MAX_BATCH + t / S::NH]);
        __syncthreads();
      }
      sync_next(s, l, ST_CAO);
      // 6. h3 = h2 + (y @ Woca^T) * gate_ca
      gemm_stage<S, 1, K_RES, false>(c, s, S::HT, p.woca + l * p.s_o, S::NKB * 512, yca, 0, h3, h2, m_ca + 2 * H, nullptr, 0);
      sync_next(s, l, ST_GU);
      // 7. g = bf16(act(bf16(A Wg^T)) * bf16(A Wu^T)), A = AdaRMS_mlp(h3)
      gemm_stage<S, 2, K_GU, true>(c, s, S::IT, p.wgu + l * p.s_gu, 2 * S::NKB * 512, h3, m_mlp, g, nullptr, 0, nullptr, 0);
      sync_next(s, l, ST_DOWN);
      // 8. h = h3 + (g @ Wd^T) * gate_mlp, K split in I/H parts
      gemm_stage<S, 1, K_SPLIT, false>(c, s, S::HT * S::SK, p.wd + l * p.s_d, 0, g, 0, hl, h3, m_mlp + 2 * H, part, S::HT);
      if (l + 1 < p.L) sync_next(s, l + 1, ST_QKV);
      else sync_next(s, 0, -1);
    }
    // step tail
    const float* hL = (const float*)(c.frame(s, p.L - 1) + S::hl_off(NRP));
    tail_stage(c, s, false, s + 1 == p.n_steps, hL);
    if (s + 1 < p.n_steps) sync_next(s + 1, 0, ST_QKV);
    else sync_next(s, 0, -1);
  }
  if (c.wg == 0 && c.tid == 0) __hip_atomic_store(&p.bar->gen, bc.base + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace mkx
