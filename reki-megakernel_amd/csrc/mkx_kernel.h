// The persistent megakernel: Euler steps of the flow-matching action expert in one launch.
//
// Schedule (mirrors expert_megakernel, src/mk_expert.py:302-426): an in-projection tail, then for each
// step and layer eight stages (QKV, self-attention, out-proj + gated residual, cross-attention query,
// cross-attention, out-proj + gated residual, gate/up, down + gated residual) and a step tail, each
// followed by a grid barrier: 1 + n_steps * (8 L + 1) barriers.
//
// Work decomposition for 256 CUs: every linear layer is cut into 16-column output tiles (one task per
// workgroup, K = H per task; the down projection is split over K into I/H tasks per tile whose fp32
// partials are summed in a fixed order by the last-arriving task). Between arriving at a barrier and
// waiting on it, a workgroup DMAs into LDS everything constant its next task needs: the packed weight tile
// and the per-sample modulation slices (or, for attention, the cached K/V). After the barrier only the
// activations are loaded, straight into VGPRs.
//
// Numerics ("split-bf16"): weights are bf16; every activation operand of an MFMA is split into a bf16 high
// part and a bf16 residual (a = hi + lo, |lo| <= ulp(hi)/2), and both are multiplied, so the products are
// those of the fp32 activation to ~2^-17 relative. Activations, softmax probabilities and the residual
// stream stay fp32 between stages. The kernel therefore reproduces the fp32 eager expert (not the bf16
// rounding points of the reference's Triton kernel, src/mk_expert.py:119, 169-172, 220): a bf16-activation
// kernel sits at the bf16 rounding-noise floor of the model (~1.5e-3 mean |delta| at full depth), which
// is most of the 2e-3 parity budget.
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
  static constexpr int ABUF = WBUF_BYTES, ABUF_BYTES = 88 * 1024;
  static constexpr int RED = ABUF, RED_BYTES = 32 * 1024;              // GEMM cross-wave reduction
  static constexpr int MODS = ABUF + RED_BYTES, MODS_BYTES = 56 * 1024;  // per-sample modulation slices
  static constexpr int SMALL = ABUF + ABUF_BYTES, SMALL_BYTES = 4 * 1024;
  static constexpr int LDS = SMALL + SMALL_BYTES;
  static constexpr int RB_FIT = 144 / (KPW * 8);  // row tiles per GEMM pass held in VGPRs (fp32)
  static constexpr int RBMAX = RB_FIT > 4 ? 4 : RB_FIT;
  static constexpr int MAXKT = (256 + 128) / 16;  // self-attention key tiles (PM <= 256, M_q <= 128)
  static constexpr int MAX_MOD_SAMPLES = MODS_BYTES / (2 * H * 4);
  static_assert(H % 256 == 0 && I % H == 0, "H must be a multiple of 256 and I a multiple of H");
  static_assert(KPW >= 1 && RBMAX >= 1, "tile does not fit registers");
  static_assert(NKB * 1024 * 2 <= WBUF_BYTES, "gate/up weight tile pair must fit the weight buffer");
  static_assert(NWAVES * RBMAX * 2 * 1024 <= RED_BYTES, "cross-wave reduction must fit LDS");
  static_assert(LDS <= 160 * 1024 - 256, "LDS budget");
  // frame layout (bytes), tile-major fp32 buffers [cols/16][NRP][16]
  __host__ __device__ static long long qkv_off(int) { return 0; }
  __host__ __device__ static long long ysa_off(int nrp) { return (long long)nrp * 3 * H * 4; }
  __host__ __device__ static long long h2_off(int nrp) { return ysa_off(nrp) + (long long)nrp * H * 4; }
  __host__ __device__ static long long qca_off(int nrp) { return h2_off(nrp) + (long long)nrp * H * 4; }
  __host__ __device__ static long long yca_off(int nrp) { return qca_off(nrp) + (long long)nrp * H * 4; }
  __host__ __device__ static long long h3_off(int nrp) { return yca_off(nrp) + (long long)nrp * H * 4; }
  __host__ __device__ static long long g_off(int nrp) { return h3_off(nrp) + (long long)nrp * H * 4; }
  __host__ __device__ static long long hl_off(int nrp) { return g_off(nrp) + (long long)nrp * I * 4; }
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

template <class S>
__device__ __forceinline__ void dma_w(Ctx<S>& c, char* dst, const bf16_t* src, int nchunks) {
  for (int k = c.wave; k < nchunks; k += NWAVES) dma16(src + (long long)k * 512 + c.lane * 8, dst + k * 1024);
}
// nfloats (a multiple of 256) contiguous fp32 values into LDS
template <class S>
__device__ __forceinline__ void dma_f32(Ctx<S>& c, char* dst, const float* src, int nfloats) {
  for (int k = c.wave; k < nfloats / 256; k += NWAVES) dma16(src + (long long)k * 256 + c.lane * 4, dst + k * 1024);
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
// split 8 fp32 values into bf16 high parts and bf16 residuals
__device__ __forceinline__ void split8(const float* f, bf16x8& hi, bf16x8& lo) {
  float r[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = f[j] - rbf(f[j]);
  const u32x4 h = pack8(f), l = pack8(r);
  hi = *reinterpret_cast<const bf16x8*>(&h);
  lo = *reinterpret_cast<const bf16x8*>(&l);
}
__device__ __forceinline__ u32x4 lds16(const char* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void sts16(char* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ bf16x8 ldsfrag(const char* p) { return *reinterpret_cast<const bf16x8*>(p); }
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
//   ADARMS: A = h * rstd(h) * (1 + scale) + shift from the fp32 residual stream (src/mk_expert.py:93-122;
//           the per-sample scale/shift slices were staged in LDS by the prefetch); otherwise A is an fp32
//           activation frame.
//   KIND PLAIN: fp32 store (qkv, cross-attention query); RES: h_out = res + acc * gate (:162-172);
//   GU: act(gate) * up (:404-413); SPLIT: K-split partial, the last split of a tile sums the partials in
//   split order and applies RES.
// K (= H per task) is split over the 4 waves; the wave partials are summed through LDS.
enum { K_PLAIN = 0, K_RES = 1, K_GU = 2, K_SPLIT = 3 };

template <class S, int NT>
__device__ __forceinline__ void red_sum8(Ctx<S>& c, int r, int nt, int half, float* out) {
  const float* red = (const float*)(c.smem + S::RED);
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

// staged per-sample modulation slice: ADARMS stages hold [scale | shift] (2H), RES stages hold gate (H)
template <class S>
__device__ __forceinline__ const float* mods_lds(Ctx<S>& c, int b, int width) {
  return (const float*)(c.smem + S::MODS) + (long long)b * width;
}

template <class S, int NT, int KIND, bool ADARMS>
__device__ void gemm_stage(Ctx<S>& c, int s, int ntask, const bf16_t* wbase, long long wtask_stride, const float* asrc,
                           float* out, const float* res, float* part, int split_tiles) {
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
      bf16x8 ahi[RB][KPW], alo[RB][KPW];
      {
        float x[RB][KPW][8];
        // rows beyond the pass are clamped to the pass's last row: every load is unconditional (one batch)
#pragma unroll
        for (int rt = 0; rt < RB; ++rt)
#pragma unroll
          for (int i = 0; i < KPW; ++i) {
            const int row = row0 + min(rt, nrt - 1) * 16 + (c.lane & 15);
            const int col = k0 + (c.wave + NWAVES * i) * 32 + 8 * (c.lane >> 4);
            load8f(asrc + ((long long)(col >> 4) * NRP + row) * 16 + (col & 15), x[rt][i]);
          }
        if (ADARMS) {
          float* ssq = (float*)(c.smem + S::SMALL);  // [4][RB*16]
#pragma unroll
          for (int rt = 0; rt < RB; ++rt) {
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < KPW; ++i)
#pragma unroll
              for (int j = 0; j < 8; ++j) ss += x[rt][i][j] * x[rt][i][j];
            ss += __shfl_xor(ss, 16);
            ss += __shfl_xor(ss, 32);
            if (c.lane < 16) ssq[c.wave * RB * 16 + rt * 16 + c.lane] = ss;
          }
          wait_vm0();  // staged weights and modulation slices have landed
          __syncthreads();
#pragma unroll
          for (int rt = 0; rt < RB; ++rt) {
            const int r = rt * 16 + (c.lane & 15);
            float tot = 0.f;
#pragma unroll
            for (int w = 0; w < NWAVES; ++w) tot += ssq[w * RB * 16 + r];
            const float rs = rsqrtf(tot / (float)S::H + c.p.eps);
            const float* ml = mods_lds(c, c.sample_of(row0 + r), 2 * S::H);
#pragma unroll
            for (int i = 0; i < KPW; ++i) {
              const int col = (c.wave + NWAVES * i) * 32 + 8 * (c.lane >> 4);
              float sc[8], sh[8], v[8];
              load8f(ml + col, sc);
              load8f(ml + S::H + col, sh);
#pragma unroll
              for (int j = 0; j < 8; ++j) v[j] = x[rt][i][j] * rs * (1.0f + sc[j]) + sh[j];
              split8(v, ahi[rt][i], alo[rt][i]);
            }
          }
        } else {
#pragma unroll
          for (int rt = 0; rt < RB; ++rt)
#pragma unroll
            for (int i = 0; i < KPW; ++i) split8(x[rt][i], ahi[rt][i], alo[rt][i]);
          wait_vm0();
          __syncthreads();
        }
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
        for (int nt = 0; nt < NT; ++nt) w[nt] = ldsfrag(c.smem + S::WBUF + (nt * S::NKB + kb) * 1024 + c.lane * 16);
#pragma unroll
        for (int rt = 0; rt < RB; ++rt)
          if (rt < nrt) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
              acc[rt][nt] = mfma16(ahi[rt][i], w[nt], acc[rt][nt]);
              acc[rt][nt] = mfma16(alo[rt][i], w[nt], acc[rt][nt]);
            }
          }
      }
      // cross-wave reduction through LDS: red[w][rt][nt][16 rows][16 cols]
      float* red = (float*)(c.smem + S::RED);
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
        const long long ooff = ((long long)tile * NRP + grow) * 16 + half * 8;  // elements
        float v[8];
        red_sum8<S, NT>(c, r, 0, half, v);
        if (KIND == K_GU) {
          float u[8];
          red_sum8<S, NT>(c, r, NT - 1, half, u);
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = act_fn(v[j], c.p.act) * u[j];
          st8f_sc1(out, ooff, v);
        } else if (KIND == K_PLAIN) {
          st8f_sc1(out, ooff, v);
        } else if (KIND == K_RES) {
          float rv[8], g[8];
          load8f(res + ooff, rv);
          load8f(mods_lds(c, c.sample_of(grow), S::H) + tile * 16 + half * 8, g);
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = rv[j] + v[j] * g[j];
          st8f_sc1(out, ooff, v);
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
          float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
          u32x4 xp[2 * 8];
#pragma unroll
          for (int j = 0; j < 8; ++j) {  // up to 8 splits, loads batched
            if (j < SK) {
              const long long poff = (((long long)j * split_tiles + tile) * NRP + grow) * 16 + half * 8;
              xp[2 * j] = ld_sc1(part, (uint32_t)(poff * 4));
              xp[2 * j + 1] = ld_sc1(part, (uint32_t)(poff * 4 + 16));
            }
          }
          const long long ooff = ((long long)tile * NRP + grow) * 16 + half * 8;
          float rv[8], g[8];
          load8f(res + ooff, rv);
          load8f(mods_lds(c, c.sample_of(grow), S::H) + tile * 16 + half * 8, g);
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (j < SK) {
#pragma unroll
              for (int q = 0; q < 4; ++q) { v[q] += __uint_as_float(xp[2 * j][q]); v[4 + q] += __uint_as_float(xp[2 * j + 1][q]); }
            }
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = rv[j] + v[j] * g[j];
          st8f_sc1(out, ooff, v);
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

// q/k head row, 8 lanes per row (lane j of the group holds d = 8j .. 8j+7 of x): RMSNorm with weight 1 + w,
// then rotate-half RoPE (src/mk_expert.py:175-193), in fp32.
__device__ __forceinline__ void norm_rope8(float* x, const bf16_t* w, const float* cs, const float* sn, float eps, int j) {
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < 8; ++q) ss += x[q] * x[q];
  ss += __shfl_xor(ss, 1);
  ss += __shfl_xor(ss, 2);
  ss += __shfl_xor(ss, 4);
  const float r = rsqrtf(ss / 64.f + eps);
  float wv[8], c8[8], s8[8];
  unpack8(ld16(w + 8 * j), wv);
  load8f(cs + 8 * j, c8);
  load8f(sn + 8 * j, s8);
  float xn[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) xn[q] = x[q] * r * (1.0f + wv[q]);
  const float sgn = j < 4 ? -1.0f : 1.0f;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const float partner = __shfl_xor(xn[q], 4);  // d +- 32
    x[q] = xn[q] * c8[q] + sgn * partner * s8[q];
  }
}

// 8 fp32 values of row `grow`, columns [col, col+8) of a tile-major fp32 buffer
template <class S>
__device__ __forceinline__ void load_frag8(Ctx<S>& c, const float* buf, int grow, int col, float* x) {
  load8f(buf + ((long long)(col >> 4) * c.p.NRP + grow) * 16 + (col & 15), x);
}

template <class S>
__device__ void sa_prefetch(Ctx<S>& c, int l, int b, int hd) {
  const int PM = c.p.PM, PMP = ceil_to(PM, 32);
  char* memK = c.smem + S::WBUF;
  char* memV = memK + PMP * 128;
  const bf16_t* mk = c.p.memk[l] + (long long)b * c.p.mem_sb;
  const bf16_t* mv = c.p.memv[l] + (long long)b * c.p.mem_sb;
  const int nk = (PMP / 16) * 2, nv = PMP / 8;
  for (int k = c.wave; k < nk + nv; k += NWAVES) {
    if (k < nk) {
      const int kt = k >> 1, db = k & 1;
      const int key = min(kt * 16 + (c.lane & 15), PM - 1);
      dma16(mk + ((long long)key * S::NH + hd) * HD + db * 32 + 8 * (c.lane >> 4), memK + k * 1024);
    } else {
      const int i = k - nk;
      const int key = min(i * 8 + (c.lane >> 3), PM - 1);
      dma16(mv + ((long long)key * S::NH + hd) * HD + (c.lane & 7) * 8, memV + i * 1024);
    }
  }
}

// In-place transpose of nkeys raw V rows (key-major [key][64] bf16) into Vt chunks at the same address.
// Keys outside [lo, hi) become zero. nkeys <= 256 (8 pieces of 16 bytes per thread).
__device__ __forceinline__ void transpose_v_inplace(char* buf, int nkeys, int lo, int hi, int tid) {
  u32x4 v[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int it = tid + u * NTHREADS;
    if (it < nkeys * 8) v[u] = lds16(buf + it * 16);
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int it = tid + u * NTHREADS;
    if (it < nkeys * 8) {
      const int key = it >> 3, dg = (it & 7) * 8;
      const bool ok = key >= lo && key < hi;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t w = ok ? v[u][q] : 0u;
        *reinterpret_cast<bf16_t*>(buf + vt_off(key, dg + 2 * q)) = (bf16_t)(w & 0xffffu);
        *reinterpret_cast<bf16_t*>(buf + vt_off(key, dg + 2 * q + 1)) = (bf16_t)(w >> 16);
      }
    }
  }
}

// Self-attention of one (sample, head): queries = own rows; keys = memory rows [kv_start, PM) (bf16 cache,
// pre-normed and rotated) || own rows (normed and rotated here). Two-pass fp32 softmax
// (src/mk_expert.py:196-222). The own-row Q, K and V are split into bf16 hi + lo.
template <class S>
__device__ void sa_task(Ctx<S>& c, int s, int l, int b, int hd, const float* qkv, float* y, int kvs) {
  CP& p = c.p;
  const int M = p.Mq, PM = p.PM, PMP = ceil_to(PM, 32), NOWN = ceil_to(M, 16), NOWN32 = ceil_to(M, 32);
  char* memK = c.smem + S::WBUF;
  char* memVt = memK + PMP * 128;
  char* Qhi = c.smem + S::ABUF;
  char* Qlo = Qhi + NOWN * 128;
  char* Khi = Qlo + NOWN * 128;
  char* Klo = Khi + NOWN * 128;
  char* Vhi = Klo + NOWN * 128;
  char* Vlo = Vhi + NOWN32 * 128;
  char* Pst = Vlo + NOWN32 * 128 + c.wave * 1024;
  const bool want_kv = (s == 0 && p.cur_k != nullptr && p.R > 0);
  // memory V rows -> Vt (rows below kv_start and beyond PM are zero)
  transpose_v_inplace(memVt, PMP, kvs, PM, c.tid);
  // own rows: 8 lanes per (kind, row); kind 0 = q, 1 = k, 2 = v
  const int j = c.tid & 7;
  for (int g0 = 0; g0 < 3 * NOWN32; g0 += NTHREADS / 8) {
    const int g = g0 + (c.tid >> 3);
    if (g < 3 * NOWN32) {
      const int kind = g / NOWN32, i = g % NOWN32;
      const bool valid = i < M;
      const int grow = b * p.Mqp + min(i, M - 1);
      float x[8];
      load_frag8(c, qkv, grow, kind * S::H + hd * HD + 8 * j, x);
      if (kind < 2) {
        norm_rope8(x, (kind == 0 ? p.qn : p.kn) + l * HD, p.sa_cos + min(i, M - 1) * HD, p.sa_sin + min(i, M - 1) * HD, p.qk_eps, j);
        if (i < NOWN) {
          bf16x8 hi, lo;
          split8(x, hi, lo);
          char* dh = kind == 0 ? Qhi : Khi;
          char* dl = kind == 0 ? Qlo : Klo;
          *reinterpret_cast<bf16x8*>(dh + qk_chunk_off(i, 8 * j)) = hi;
          *reinterpret_cast<bf16x8*>(dl + qk_chunk_off(i, 8 * j)) = lo;
        }
        if (kind == 1 && want_kv && valid && i >= p.T) {
          bf16_t* o = p.cur_k + ((((long long)l * p.B + b) * p.R + (i - p.T)) * S::NH + hd) * HD + 8 * j;
          *reinterpret_cast<u32x4*>(o) = pack8(x);
        }
      } else {
        if (want_kv && valid && i >= p.T) {
          bf16_t* o = p.cur_v + ((((long long)l * p.B + b) * p.R + (i - p.T)) * S::NH + hd) * HD + 8 * j;
          *reinterpret_cast<u32x4*>(o) = pack8(x);
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const float v = valid ? x[q] : 0.f;
          const float vh = rbf(v);
          *reinterpret_cast<bf16_t*>(Vhi + vt_off(i, 8 * j + q)) = f2bf(vh);
          *reinterpret_cast<bf16_t*>(Vlo + vt_off(i, 8 * j + q)) = f2bf(v - vh);
        }
      }
    }
  }
  __syncthreads();
  const float scale = p.sm_scale;
  const int mt = PMP / 16, nkt = mt + NOWN / 16, mb = PMP / 32, nkb = mb + NOWN32 / 32;
  for (int qt = c.wave; qt < NOWN / 16; qt += NWAVES) {
    bf16x8 qh[2], ql[2];
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      qh[db] = ldsfrag(Qhi + (qt * 2 + db) * 1024 + c.lane * 16);
      ql[db] = ldsfrag(Qlo + (qt * 2 + db) * 1024 + c.lane * 16);
    }
    f32x4 sreg[S::MAXKT];
    float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
    for (int kt = 0; kt < S::MAXKT; ++kt) {
      if (kt < nkt) {
        f32x4 sc = {0.f, 0.f, 0.f, 0.f};
        if (kt < mt) {
#pragma unroll
          for (int db = 0; db < 2; ++db) {
            const bf16x8 kf = ldsfrag(memK + (kt * 2 + db) * 1024 + c.lane * 16);
            sc = mfma16(qh[db], kf, sc);
            sc = mfma16(ql[db], kf, sc);
          }
        } else {
#pragma unroll
          for (int db = 0; db < 2; ++db) {
            const int off = ((kt - mt) * 2 + db) * 1024 + c.lane * 16;
            const bf16x8 kh = ldsfrag(Khi + off), kl = ldsfrag(Klo + off);
            sc = mfma16(qh[db], kh, sc);
            sc = mfma16(ql[db], kh, sc);
            sc = mfma16(qh[db], kl, sc);
          }
        }
        const int key = kt * 16 + (c.lane & 15);
        const bool valid = kt < mt ? (key >= kvs && key < PM) : (key - PMP < M);
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
    for (int kt = 0; kt < S::MAXKT; ++kt)
      if (kt < nkt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float e = __expf(sreg[kt][i] - mx[i]);
          sreg[kt][i] = e;
          den[i] += e;
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
      if (kb < nkb) {
        // P (fp32) of key tiles 2kb, 2kb+1 -> bf16 hi then lo, through the wave's 1 KB staging tile
        bf16x8 pf[2];
#pragma unroll
        for (int part = 0; part < 2; ++part) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int kt = 2 * kb + h;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float pv = kt < nkt ? sreg[kt][i] : 0.f;
              const float ph = rbf(pv);
              *reinterpret_cast<bf16_t*>(Pst + (4 * (c.lane >> 4) + i) * 64 + (h * 16 + (c.lane & 15)) * 2) =
                  f2bf(part == 0 ? ph : pv - ph);
            }
          }
          pf[part] = ldsfrag(Pst + (c.lane & 15) * 64 + (c.lane >> 4) * 16);
        }
        if (kb < mb) {
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) {
            const bf16x8 vf = ldsfrag(memVt + (kb * 4 + dt) * 1024 + c.lane * 16);
            acc[dt] = mfma16(pf[0], vf, acc[dt]);
            acc[dt] = mfma16(pf[1], vf, acc[dt]);
          }
        } else {
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) {
            const int off = ((kb - mb) * 4 + dt) * 1024 + c.lane * 16;
            const bf16x8 vh = ldsfrag(Vhi + off), vl = ldsfrag(Vlo + off);
            acc[dt] = mfma16(pf[0], vh, acc[dt]);
            acc[dt] = mfma16(pf[1], vh, acc[dt]);
            acc[dt] = mfma16(pf[0], vl, acc[dt]);
          }
        }
      }
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int q = qt * 16 + 4 * (c.lane >> 4) + i;
        if (q < M) {
          const long long off = ((long long)(hd * 4 + dt) * p.NRP + b * p.Mqp + q) * 16 + (c.lane & 15);
          st_sc1_b32(y, (uint32_t)(off * 4), __float_as_uint(acc[dt][i] / den[i]));
        }
      }
  }
}

// Cross-attention: K/V streamed in blocks of 64 source rows through a 4-slot LDS ring (16 KB per slot:
// K chunks, then raw V rows transposed in place), online fp32 softmax (src/mk_expert.py:225-251).
template <class S>
__device__ void ca_dma_block(Ctx<S>& c, int l, int b, int hd, int jb) {
  const int SP = c.p.SP;
  char* slot = c.smem + S::WBUF + (jb & 3) * 16384;
  const bf16_t* kb_ = c.p.kca[l] + (long long)b * c.p.src_sb;
  const bf16_t* vb_ = c.p.vca[l] + (long long)b * c.p.src_sb;
  for (int k = c.wave; k < 16; k += NWAVES) {
    if (k < 8) {
      const int kt = k >> 1, db = k & 1;
      const int key = min(jb * 64 + kt * 16 + (c.lane & 15), SP - 1);
      dma16(kb_ + ((long long)key * S::NH + hd) * HD + db * 32 + 8 * (c.lane >> 4), slot + k * 1024);
    } else {
      const int i = k - 8;
      const int key = min(jb * 64 + i * 8 + (c.lane >> 3), SP - 1);
      dma16(vb_ + ((long long)key * S::NH + hd) * HD + (c.lane & 7) * 8, slot + 8192 + i * 1024);
    }
  }
}

template <class S>
__device__ void ca_prefetch(Ctx<S>& c, int l, int b, int hd, int S_len) {
  const int nblk = (S_len + 63) / 64;
  for (int jb = 0; jb < min(nblk, 4); ++jb) ca_dma_block(c, l, b, hd, jb);
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
__device__ void ca_task(Ctx<S>& c, int s, int l, int b, int hd, const float* qca, float* y, int S_len) {
  CP& p = c.p;
  const int M = p.Mq, NOWN = ceil_to(M, 16);
  char* Qhi = c.smem + S::ABUF;
  char* Qlo = Qhi + NOWN * 128;
  char* Pst = Qlo + NOWN * 128 + c.wave * 1024;
  const int j = c.tid & 7;
  for (int g0 = 0; g0 < NOWN; g0 += NTHREADS / 8) {
    const int i = g0 + (c.tid >> 3);
    if (i < NOWN) {
      const int ic = min(i, M - 1);
      float x[8];
      load_frag8(c, qca, b * p.Mqp + ic, hd * HD + 8 * j, x);
      norm_rope8(x, p.qcan + l * HD, p.ca_cos + ic * HD, p.ca_sin + ic * HD, p.qk_eps, j);
      bf16x8 hi, lo;
      split8(x, hi, lo);
      *reinterpret_cast<bf16x8*>(Qhi + qk_chunk_off(i, 8 * j)) = hi;
      *reinterpret_cast<bf16x8*>(Qlo + qk_chunk_off(i, 8 * j)) = lo;
    }
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
  for (int jb = 0; jb < nblk; ++jb) {
    wait_vm_blocks(min(nblk, jb + 4) - jb - 1);
    __syncthreads();
    char* slot = c.smem + S::WBUF + (jb & 3) * 16384;
    transpose_v_inplace(slot + 8192, 64, 0, S_len - jb * 64, c.tid);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < MAXQT; ++u) {
      const int qt = c.wave + NWAVES * u;
      if (qt < NOWN / 16) {
        bf16x8 qh[2], ql[2];
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          qh[db] = ldsfrag(Qhi + (qt * 2 + db) * 1024 + c.lane * 16);
          ql[db] = ldsfrag(Qlo + (qt * 2 + db) * 1024 + c.lane * 16);
        }
        f32x4 sb[4];
        float mb[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int db = 0; db < 2; ++db) {
            const bf16x8 kf = ldsfrag(slot + (kt * 2 + db) * 1024 + c.lane * 16);
            sc = mfma16(qh[db], kf, sc);
            sc = mfma16(ql[db], kf, sc);
          }
          const bool valid = jb * 64 + kt * 16 + (c.lane & 15) < S_len;
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
          bf16x8 pf[2];
#pragma unroll
          for (int part = 0; part < 2; ++part) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const float pv = sb[2 * kb + h][i];
                const float ph = rbf(pv);
                *reinterpret_cast<bf16_t*>(Pst + (4 * (c.lane >> 4) + i) * 64 + (h * 16 + (c.lane & 15)) * 2) =
                    f2bf(part == 0 ? ph : pv - ph);
              }
            pf[part] = ldsfrag(Pst + (c.lane & 15) * 64 + (c.lane >> 4) * 16);
          }
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) {
            const bf16x8 vf = ldsfrag(slot + 8192 + (kb * 4 + dt) * 1024 + c.lane * 16);
            acc[u][dt] = mfma16(pf[0], vf, acc[u][dt]);
            acc[u][dt] = mfma16(pf[1], vf, acc[u][dt]);
          }
        }
      }
    }
    __syncthreads();
    if (jb + 4 < nblk) ca_dma_block(c, l, b, hd, jb + 4);
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
            st_sc1_b32(y, (uint32_t)(off * 4), __float_as_uint(o));
          }
        }
    }
  }
}

// ------------------------------------------------------------------------------------------------
// Step tail (src/mk_expert.py:254-299): o = AdaRMS_final(h_L); v = o Wout^T + bout; x' = x_pad + dt v;
// h0' = x'_pad Win + bin, all fp32. Tasks [0, H/16): in-projection tiles (they recompute the velocity of
// the real action dims); tasks [H/16, H/16 + A): one output dim each. One wave per action row; lane < H/16
// owns 16 columns; every constant a lane needs is loaded in one batch before use.
constexpr int TAIL_AG = 8;  // output dims per batched group

template <class S>
__device__ void tail_velocity8(Ctx<S>& c, const float* hL, int grow, const float* mrow, int a0, int na, float* v) {
  const int lane = c.lane;
  const int lc = min(lane, S::HT - 1);
  float x[16], sc[16], sh[16], w[TAIL_AG][16];
  load8f(hL + ((long long)lc * c.p.NRP + grow) * 16, x);
  load8f(hL + ((long long)lc * c.p.NRP + grow) * 16 + 8, x + 8);
  load8f(mrow + lc * 16, sc);
  load8f(mrow + lc * 16 + 8, sc + 8);
  load8f(mrow + S::H + lc * 16, sh);
  load8f(mrow + S::H + lc * 16 + 8, sh + 8);
#pragma unroll
  for (int a = 0; a < TAIL_AG; ++a) {
    const float* wr = c.p.wout + (long long)min(a0 + a, c.p.A - 1) * S::H + lc * 16;
    load8f(wr, w[a]);
    load8f(wr + 8, w[a] + 8);
  }
  float ss = 0.f;
  if (lane < S::HT) {
#pragma unroll
    for (int q = 0; q < 16; ++q) ss += x[q] * x[q];
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) ss += __shfl_xor(ss, o);
  const float r = rsqrtf(ss / (float)S::H + c.p.eps);
  float o16[16];
#pragma unroll
  for (int q = 0; q < 16; ++q) o16[q] = lane < S::HT ? x[q] * r * (1.0f + sc[q]) + sh[q] : 0.f;
#pragma unroll
  for (int a = 0; a < TAIL_AG; ++a) {
    float d = 0.f;
#pragma unroll
    for (int q = 0; q < 16; ++q) d += o16[q] * w[a][q];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) d += __shfl_xor(d, o);
    v[a] = d + (a < na ? c.p.bout[a0 + a] : 0.f);
  }
}

template <class S>
__device__ void tail_stage(Ctx<S>& c, int s, bool first, bool last, const float* hL) {
  CP& p = c.p;
  const int nin = last ? 0 : S::HT;
  const int nout = first ? 0 : p.A;
  const int nrows = p.B * p.T;
  const int adim = p.action_dim;
  const float* xcur = (first || s == 0) ? p.x_in : c.xstep(s);
  float* xp = (float*)(c.smem + S::ABUF);  // [nrows][action_dim] x' of the real dims
  for (int t = c.wg; t < nin + nout; t += c.G) {
    __syncthreads();
    if (t < nin) {
      for (int ri = c.wave; ri < nrows; ri += NWAVES) {
        const int b = ri / p.T, i = ri % p.T;
        if (first) {
          if (c.lane < adim) xp[ri * adim + c.lane] = xcur[(long long)ri * p.A + c.lane];
        } else {
          const float* mrow = c.modrow(b, s) + 9 * p.L * S::H;
          for (int a0 = 0; a0 < adim; a0 += TAIL_AG) {
            float v[TAIL_AG];
            tail_velocity8(c, hL, b * p.Mqp + i, mrow, a0, min(TAIL_AG, adim - a0), v);
            if (c.lane < TAIL_AG && a0 + c.lane < adim) {
              float vv = v[0];
#pragma unroll
              for (int a = 1; a < TAIL_AG; ++a) vv = c.lane == a ? v[a] : vv;
              xp[ri * adim + a0 + c.lane] = xcur[(long long)ri * p.A + a0 + c.lane] + c.dt * vv;
            }
          }
        }
      }
      __syncthreads();
      float* h0n = c.h0(first ? 0 : s + 1);
      const int col0 = t * 16;
      for (int it = c.tid; it < p.NRP * 2; it += NTHREADS) {
        const int grow = it >> 1, half = it & 1;
        const int b = grow / p.Mqp, i = grow % p.Mqp;
        const int col = col0 + half * 8;
        float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (b < p.B && i < p.T) {
          load8f(p.bin + col, v);
          const float* xr = xp + (b * p.T + i) * adim;
          for (int a0 = 0; a0 < adim; a0 += TAIL_AG) {
            float w[TAIL_AG][8];
#pragma unroll
            for (int a = 0; a < TAIL_AG; ++a) load8f(p.win + (long long)min(a0 + a, p.A - 1) * S::H + col, w[a]);
#pragma unroll
            for (int a = 0; a < TAIL_AG; ++a)
              if (a0 + a < adim) {
                const float xa = xr[a0 + a];
#pragma unroll
                for (int q = 0; q < 8; ++q) v[q] += xa * w[a][q];
              }
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
        const float* mrow = c.modrow(b, s) + 9 * p.L * S::H;
        float v[TAIL_AG];
        tail_velocity8(c, hL, b * p.Mqp + i, mrow, a, 1, v);
        if (c.lane == 0) {
          const float xa = a < adim ? xcur[(long long)ri * p.A + a] : 0.f;
          st_sc1_b32(xn, (uint32_t)(((long long)ri * p.A + a) * 4), __float_as_uint(xa + c.dt * v[0]));
        }
      }
    }
  }
}

// ------------------------------------------------------------------------------------------------
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
  if (p.profile && c.wg == 0 && c.tid == 0) p.prof[0] = clock100() * 10;

  // DMA of the constant operands of this workgroup's first task in a stage (weight tile or cached K/V)
  // and of the stage's per-sample modulation slices
  auto prefetch = [&](int s, int l, int st) {
    char* wb = smem + S::WBUF;
    char* mb = smem + S::MODS;
    const int t = c.wg;
    const int m_sa = 9 * l * H, m_ca = m_sa + 3 * H, m_mlp = m_sa + 6 * H;
    auto stage_mods = [&](int off, int width) {
      for (int b = 0; b < p.B; ++b) dma_f32(c, mb + b * width * 4, c.modrow(b, s) + off, width);
    };
    switch (st) {
      case ST_QKV:
        if (t < 3 * S::HT) { dma_w(c, wb, p.wqkv + l * p.s_qkv + (long long)t * S::NKB * 512, S::NKB); stage_mods(m_sa, 2 * H); }
        break;
      case ST_SA: if (t < NBH) sa_prefetch(c, l, t / S::NH, t % S::NH); break;
      case ST_O:
        if (t < S::HT) { dma_w(c, wb, p.wo + l * p.s_o + (long long)t * S::NKB * 512, S::NKB); stage_mods(m_sa + 2 * H, H); }
        break;
      case ST_CAQ:
        if (t < S::HT) { dma_w(c, wb, p.wqca + l * p.s_o + (long long)t * S::NKB * 512, S::NKB); stage_mods(m_ca, 2 * H); }
        break;
      case ST_CA: if (t < NBH) ca_prefetch(c, l, t / S::NH, t % S::NH, s_ks[MAX_BATCH + t / S::NH]); break;
      case ST_CAO:
        if (t < S::HT) { dma_w(c, wb, p.woca + l * p.s_o + (long long)t * S::NKB * 512, S::NKB); stage_mods(m_ca + 2 * H, H); }
        break;
      case ST_GU:
        if (t < S::IT) { dma_w(c, wb, p.wgu + l * p.s_gu + (long long)t * 2 * S::NKB * 512, 2 * S::NKB); stage_mods(m_mlp, 2 * H); }
        break;
      case ST_DOWN:
        if (t < S::HT * S::SK) {
          const int tile = t % S::HT, split = t / S::HT;
          dma_w(c, wb, p.wd + l * p.s_d + ((long long)tile * S::SK + split) * S::NKB * 512, S::NKB);
          stage_mods(m_mlp + 2 * H, H);
        }
        break;
      default: break;
    }
  };
  auto sync_next = [&](int s, int l, int st) {
    bar_arrive(bc, ++e);
    if (st >= 0) prefetch(s, l, st);
    bar_wait(bc, e);
    if (p.profile && c.wg == 0 && c.tid == 0) p.prof[e] = clock100() * 10;
  };

  // in-projection of the incoming x (src/mk_expert.py:326-327)
  tail_stage(c, 0, true, false, nullptr);
  sync_next(0, 0, ST_QKV);
  for (int s = 0; s < p.n_steps; ++s) {
    for (int l = 0; l < p.L; ++l) {
      char* fr = c.frame(s, l);
      const float* hin = c.h_in(s, l);
      float* qkv = (float*)(fr + S::qkv_off(NRP));
      float* ysa = (float*)(fr + S::ysa_off(NRP));
      float* h2 = (float*)(fr + S::h2_off(NRP));
      float* qca = (float*)(fr + S::qca_off(NRP));
      float* yca = (float*)(fr + S::yca_off(NRP));
      float* h3 = (float*)(fr + S::h3_off(NRP));
      float* g = (float*)(fr + S::g_off(NRP));
      float* hl = (float*)(fr + S::hl_off(NRP));
      float* part = (float*)(fr + S::part_off(NRP));
      // 1. qkv = AdaRMS(h) @ Wqkv^T
      gemm_stage<S, 1, K_PLAIN, true>(c, s, 3 * S::HT, p.wqkv + l * p.s_qkv, S::NKB * 512, hin, qkv, nullptr, nullptr, 0);
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
      gemm_stage<S, 1, K_RES, false>(c, s, S::HT, p.wo + l * p.s_o, S::NKB * 512, ysa, h2, hin, nullptr, 0);
      sync_next(s, l, ST_CAQ);
      // 4. qca = AdaRMS_ca(h2) @ Wqca^T
      gemm_stage<S, 1, K_PLAIN, true>(c, s, S::HT, p.wqca + l * p.s_o, S::NKB * 512, h2, qca, nullptr, nullptr, 0);
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
      gemm_stage<S, 1, K_RES, false>(c, s, S::HT, p.woca + l * p.s_o, S::NKB * 512, yca, h3, h2, nullptr, 0);
      sync_next(s, l, ST_GU);
      // 7. g = act(A Wg^T) * (A Wu^T), A = AdaRMS_mlp(h3)
      gemm_stage<S, 2, K_GU, true>(c, s, S::IT, p.wgu + l * p.s_gu, 2 * S::NKB * 512, h3, g, nullptr, nullptr, 0);
      sync_next(s, l, ST_DOWN);
      // 8. h = h3 + (g @ Wd^T) * gate_mlp, K split in I/H parts
      gemm_stage<S, 1, K_SPLIT, false>(c, s, S::HT * S::SK, p.wd + l * p.s_d, 0, g, hl, h3, part, S::HT);
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
