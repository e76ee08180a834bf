// mkx C ABI (include/mkx.h): handle creation with weight packing, launch, queries.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <atomic>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "mkx.h"
#include "mkx_kernel.h"
#include "mkx_ring.h"
#include "mkx_prepare.h"
#include "mkx_modproj.h"
#include "mkx_probe.h"

using namespace mkx;

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

#define HIPCHK(x)                                                                              \
  do {                                                                                         \
    hipError_t e_ = (x);                                                                       \
    if (e_ != hipSuccess) return fail(MKX_EHIP, std::string(#x) + ": " + hipGetErrorString(e_)); \
  } while (0)

constexpr unsigned SPIN_LIMIT = 1u << 20;  // default spin bound of a wait (polls), about 0.5 s
constexpr int MAX_ROWS_PADDED = 512;

// W [L][N][K] row-major bf16 -> fp16 chunks (l, t, kb): dst[l*dls + (t'*tstride + toff + kb)*512 + lane*8 + j]
// = W[l][t*16 + lane%16][kb*32 + 8(lane/16) + j] (the MFMA 16x16x32 operand layout). t' = t, or with
// `pairs` the 16-column tiles of each 64-column head reordered 0, 2, 1, 3 (a task's d and d + 32 tiles
// adjacent). bf16 -> fp16 is exact within the fp16 range (8 significant bits of 11; values below 2^-14
// become fp16 subnormals, at most 2^-25 away); a weight beyond it sets *range.
__global__ void pack_tiles(const bf16_t* __restrict__ src, bf16_t* __restrict__ dst, int L, int N, int K,
                           long long dls, int tstride, int toff, int pairs, int* range) {
  const long long total = (long long)L * (N / 16) * (K / 32) * 64;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int lane = (int)(i % 64);
  long long r = i / 64;
  const int kb = (int)(r % (K / 32));
  r /= (K / 32);
  const int t = (int)(r % (N / 16));
  const int l = (int)(r / (N / 16));
  const bf16_t* s = src + ((long long)l * N + t * 16 + lane % 16) * K + kb * 32 + 8 * (lane / 16);
  const int tp = pairs ? ((t & ~3) | ((t & 1) << 1) | ((t >> 1) & 1)) : t;
  bf16_t* d = dst + (long long)l * dls + ((long long)tp * tstride + toff + kb) * 512 + lane * 8;
  const u32x4 w = *reinterpret_cast<const u32x4*>(s);
  u32x4 o;
  bool big = false;
  for (int j = 0; j < 4; ++j) {
    const float a = __uint_as_float(w[j] << 16), b = __uint_as_float(w[j] & 0xffff0000u);
    big = big || fabsf(a) > F16_MAX || fabsf(b) > F16_MAX;
    o[j] = cvt_pk_h(a, b);
  }
  *reinterpret_cast<u32x4*>(d) = o;
  if (big) atomicOr(range, 1);
}

// The same chunk layout for e4m3 bytes: 8 bytes per lane, 512-byte chunks (dls, tstride in chunks).
__global__ void pack_tiles8(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int L, int N, int K,
                            long long dls, int tstride, int toff, int pairs) {
  const long long total = (long long)L * (N / 16) * (K / 32) * 64;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int lane = (int)(i % 64);
  long long r = i / 64;
  const int kb = (int)(r % (K / 32));
  r /= (K / 32);
  const int t = (int)(r % (N / 16));
  const int l = (int)(r / (N / 16));
  const uint8_t* s = src + ((long long)l * N + t * 16 + lane % 16) * K + kb * 32 + 8 * (lane / 16);
  const int tp = pairs ? ((t & ~3) | ((t & 1) << 1) | ((t >> 1) & 1)) : t;
  uint8_t* d = dst + (l * dls + (long long)tp * tstride + toff + kb) * 512 + lane * 8;
  *reinterpret_cast<uint2*>(d) = *reinterpret_cast<const uint2*>(s);
}

__global__ void xcc_probe(unsigned* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}

}  // namespace

// The megakernel's instantiations live in their own translation units (mkx_mk768.hip, mkx_mk1024.hip,
// mkx_mk256.hip with GEMM stages in passes; mkx_mk768r.hip, mkx_mk1024r.hip, mkx_mk256r.hip with row-wise GEMM
// stages), each compiled with its own code-generation options; each has a twin that scales the AdaRMS
// operands (YSHIFT), launched only with an operand shift so that the others compile as without it.
namespace mkx {
#define MKX_EXTERN(H, I)                                                                \
  extern template __global__ void mkx_megakernel<H, I, false, false>(Params);       \
  extern template __global__ void mkx_megakernel<H, I, true, false>(Params);        \
  extern template __global__ void mkx_megakernel<H, I, false, true>(Params);        \
  extern template __global__ void mkx_megakernel<H, I, true, true>(Params);         \
  extern template __global__ void mkx_megakernel<H, I, false, false, true>(Params); \
  extern template __global__ void mkx_megakernel<H, I, true, false, true>(Params);  \
  extern template __global__ void mkx_megakernel<H, I, false, true, true>(Params);  \
  extern template __global__ void mkx_megakernel<H, I, true, true, true>(Params);        \
  extern template __global__ void mkx_megakernel<H, I, true, true, false, true>(Params);  \
  extern template __global__ void mkx_megakernel<H, I, true, true, true, true>(Params);   \
  extern template __global__ void mkx_megakernel<H, I, false, false, false, false, true>(Params); \
  extern template __global__ void mkx_megakernel<H, I, true, false, false, false, true>(Params);  \
  extern template __global__ void mkx_megakernel<H, I, false, false, true, false, true>(Params);  \
  extern template __global__ void mkx_megakernel<H, I, true, false, true, false, true>(Params);
MKX_EXTERN(768, 3072)
MKX_EXTERN(1024, 4096)
MKX_EXTERN(256, 512)
#undef MKX_EXTERN
}  // namespace mkx

namespace {

template <int H, int I, bool ROWWISE, bool YS>
const void* kernel_of(bool w8) {
  return w8 ? reinterpret_cast<const void*>(&mkx_megakernel<H, I, true, ROWWISE, YS>)
            : reinterpret_cast<const void*>(&mkx_megakernel<H, I, false, ROWWISE, YS>);
}
template <int H, int I>
const void* kernel_of(bool w8, bool rowwise, bool ys, bool pairs, bool longsrc) {
  // (two-tile self-attention: fp8-weight row-wise instantiations only)
  if (pairs) return !w8 ? nullptr
                        : ys ? reinterpret_cast<const void*>(&mkx_megakernel<H, I, true, true, true, true>)
                             : reinterpret_cast<const void*>(&mkx_megakernel<H, I, true, true, false, true>);
  if (longsrc && !rowwise)
    return w8 ? (ys ? reinterpret_cast<const void*>(&mkx_megakernel<H, I, true, false, true, false, true>)
                    : reinterpret_cast<const void*>(&mkx_megakernel<H, I, true, false, false, false, true>))
              : (ys ? reinterpret_cast<const void*>(&mkx_megakernel<H, I, false, false, true, false, true>)
                    : reinterpret_cast<const void*>(&mkx_megakernel<H, I, false, false, false, false, true>));
  return rowwise ? (ys ? kernel_of<H, I, true, true>(w8) : kernel_of<H, I, true, false>(w8))
                 : (ys ? kernel_of<H, I, false, true>(w8) : kernel_of<H, I, false, false>(w8));
}

// rowwise: the form whose GEMM stages compute whole-K products per wave (launches with many row tiles); ys: the
// twin with scaled AdaRMS operands (an operand shift); pairs: the row-wise form with two-tile self-attention
// tasks (fp8 weights); longsrc: the form with passes for sources beyond the three-chunk ring
const void* pick_kernel(int H, int I, bool w8, bool rowwise, bool ys = false, bool pairs = false, bool longsrc = false) {
  if (H == 768 && I == 3072) return kernel_of<768, 3072>(w8, rowwise, ys, pairs, longsrc);
  if (H == 1024 && I == 4096) return kernel_of<1024, 4096>(w8, rowwise, ys, pairs, longsrc);
  if (H == 256 && I == 512) return kernel_of<256, 512>(w8, rowwise, ys, pairs, longsrc);
  return nullptr;
}

int lds_of(int H, int I) {
  if (H == 768 && I == 3072) return Shape<768, 3072>::LDS;
  if (H == 1024 && I == 4096) return Shape<1024, 4096>::LDS;
  if (H == 256 && I == 512) return Shape<256, 512>::LDS;
  return 0;
}

// the shape constants the host's task layout depends on
struct ShapeK {
  int HT, IT, SK, NH, NIN, NTW, W_NARROW, RED_NARROW, W_WIDE, RED_WIDE, SMALL, RBMAX;
};
template <class S>
ShapeK shape_k() {
  return {S::HT, S::IT, S::SK, S::NH, S::NIN, S::NTW, S::W_NARROW, S::RED_NARROW, S::W_WIDE, S::RED_WIDE, S::SMALL, S::RBMAX};
}
ShapeK shape_k(int H, int I, bool w8) {
  if (H == 768 && I == 3072) return w8 ? shape_k<Shape<768, 3072, true>>() : shape_k<Shape<768, 3072, false>>();
  if (H == 1024 && I == 4096) return w8 ? shape_k<Shape<1024, 4096, true>>() : shape_k<Shape<1024, 4096, false>>();
  return w8 ? shape_k<Shape<256, 512, true>>() : shape_k<Shape<256, 512, false>>();
}

// Task layout of one launch: row groups, wide tiles, LDS offsets and the workgroup range of every stage's
// tasks (Params::pl). Where the gate/up tasks and the down-projection tasks fit the grid together, each
// stage's range is chosen to share as few workgroups as possible with the stages whose last task directly
// gates it (the out-projections and the down projection then take NTW column tiles per task, so that they
// need few workgroups): a workgroup is then idle in the stage before each of its tasks, so its weight DMA
// and the transition run off the critical path, and its ready-epoch poll is not queued behind its own DMA.
// Cross-attention, whose prefetch is the largest, gets workgroups idle in the two stages before it. The QKV
// tasks may share workgroups with the down projection's split tasks: they wait for the reducers, a stage
// later. Other shapes keep one task per workgroup from the bottom of the grid and the attention, reducer
// and step-tail tasks at the top.
struct Layout {
  int pl[PL_KINDS];
  int rgs_qkv, rgs_o, rgs_cao, nt_o, nt_cao, nt_down, lds_red, lds_mods, tpr, nred;
  int nrg;  // reducer row groups (row-wise form: the QKV row groups)
  bool disjoint;
};
// step-tail output tasks: TAIL_AC dims each, or, in the row-wise form, TAIL_DG dims of TAIL_RCH rows each
int tail_outputs(bool rows, int nrows, int A) {
  return rows ? (nrows + TAIL_RCH - 1) / TAIL_RCH * ((A + TAIL_DG - 1) / TAIL_DG) : (A + TAIL_AC - 1) / TAIL_AC;
}
// nqt: query tiles per sample; rows: the row-wise form (tasks of one column tile)
Layout plan_layout(const ShapeK& k, int G, int RT, int B, int nqt, int H, int A, int nout, bool rows) {
  Layout L{};
  const int nattn = B * k.NH * nqt, mods = B * 2 * H * 4;
  const bool wide = !rows && k.NTW > 1 && k.W_WIDE + std::max(k.RED_WIDE, k.RED_NARROW) + mods <= k.SMALL;
  const int nt = wide ? k.NTW : 1;
  auto clampi = [](int v, int lo, int hi) { return std::max(lo, std::min(hi, v)); };
  const int ndown_d = (k.HT / nt) * k.SK, nred_d = k.HT / nt;
  L.disjoint = k.IT + ndown_d <= G && 6 * k.NH + std::max(nred_d, nattn) <= G;
  // narrow row-wise launches (at most 8 row tiles: each task's row groups fit one per wave): one row group
  // per QKV and out-projection task, which takes no longer, so that QKV, self-attention and the
  // out-projection, then cross-attention and its out-projection, run on disjoint workgroup ranges
  const bool narrow = rows && !L.disjoint && RT <= 8 && 6 * k.NH + k.HT + nattn <= G && nattn <= 6 * k.NH &&
                      6 * k.NH + 2 * k.HT <= G;
  int cnt[PL_KINDS] = {};
  if (narrow) {
    L.nt_o = L.nt_cao = L.nt_down = 1;
    L.rgs_qkv = L.rgs_o = L.rgs_cao = 1;
  } else if (L.disjoint) {
    L.nt_o = L.nt_cao = L.nt_down = nt;
    L.rgs_cao = clampi(ndown_d / (k.HT / nt), 1, RT);
    // QKV leaves room for the self-attention tasks and the reducers; the out-projection sits inside the QKV
    // range and leaves room for both attention stages and the CA out-projection
    L.rgs_qkv = clampi((G - std::max(nred_d, nattn)) / (6 * k.NH), 1, RT);
    const int ncao = (k.HT / nt) * L.rgs_cao;
    L.rgs_o = clampi(std::min(6 * k.NH * L.rgs_qkv, G - 2 * nattn - ncao) / (k.HT / nt), 1, RT);
  } else {
    L.nt_o = L.nt_cao = L.nt_down = 1;
    L.rgs_qkv = clampi(G / (6 * k.NH), 1, RT);
    L.rgs_o = L.rgs_cao = clampi(G / k.HT, 1, RT);
  }
  cnt[PL_QKV] = 6 * k.NH * L.rgs_qkv;
  cnt[PL_SA] = cnt[PL_CA] = nattn;
  cnt[PL_O] = (k.HT / L.nt_o) * L.rgs_o;
  cnt[PL_CAO] = (k.HT / L.nt_cao) * L.rgs_cao;
  cnt[PL_GU] = k.IT;
  cnt[PL_DOWN] = (k.HT / L.nt_down) * k.SK;
  // reducers: with the disjoint layout, one per wide task's tiles (their loads then equal a wide task's
  // operand share, and they fit beside the QKV tasks); otherwise one per 16-column tile, so that batched
  // shapes, whose reductions cover many row tiles, spread them over more workgroups
  L.tpr = L.disjoint ? nt : 1;
  // the row-wise form's reducers also split the rows, in the QKV stage's row groups (each then loads a third or
  // a half of a tile's partials, and a QKV task waits only for its own row group's reducers)
  L.nrg = rows ? L.rgs_qkv : 1;
  L.nred = k.HT / L.tpr * L.nrg;
  cnt[PL_RED] = L.nred;
  cnt[PL_TIN] = k.NIN;
  cnt[PL_TOUT] = nout;
  const bool any_wide = L.nt_o > 1 || L.nt_cao > 1 || L.nt_down > 1;
  L.lds_red = any_wide ? std::max(k.W_WIDE, k.W_NARROW) : k.W_NARROW;
  L.lds_mods = L.lds_red + (any_wide ? std::max(k.RED_WIDE, k.RED_NARROW) : k.RED_NARROW);
  auto md = [&](int v) { return ((v % G) + G) % G; };
  if (L.disjoint) {
    // base of a range that shares the fewest workgroups with the ranges of `avoid` (lowest base on ties)
    auto place = [&](int kind, std::initializer_list<int> avoid) {
      std::vector<char> used(G, 0);
      for (int a : avoid)
        for (int i = 0; i < std::min(cnt[a], G); ++i) used[(L.pl[a] + i) % G] = 1;
      const int n = std::min(cnt[kind], G);
      int best = 0, best_ov = G + 1;
      for (int b = 0; b < G; ++b) {
        int ov = 0;
        for (int i = 0; i < n; ++i) ov += used[(b + i) % G];
        if (ov < best_ov) { best_ov = ov; best = b; }
      }
      L.pl[kind] = best;
    };
    // stage order within a layer: QKV, SA, O, CA, CAO, GU, DOWN (+ reducers); the step tail between the
    // last layer's reducers and the first layer's QKV. The step tail's output tasks (read a step later)
    // share the reducers' workgroups.
    L.pl[PL_GU] = 0;
    place(PL_DOWN, {PL_GU});
    place(PL_CAO, {PL_GU});
    place(PL_RED, {PL_DOWN});
    place(PL_QKV, {PL_RED});
    place(PL_O, {PL_RED});
    place(PL_SA, {PL_QKV, PL_O});
    place(PL_CA, {PL_O, PL_SA, PL_CAO});
    place(PL_TIN, {PL_RED, PL_QKV});
    place(PL_TOUT, {PL_QKV, PL_TIN, PL_DOWN});
  } else if (narrow) {
    // QKV [0, 6 NH), self-attention at the top, the out-projection between them; cross-attention on the QKV
    // tasks' workgroups and its out-projection at the top, above the out-projection's (each range idle in the
    // two stages before); gate/up and down on every workgroup
    L.pl[PL_QKV] = L.pl[PL_CA] = L.pl[PL_GU] = L.pl[PL_DOWN] = 0;
    L.pl[PL_SA] = md(G - nattn);
    L.pl[PL_CAO] = md(G - k.HT);
    L.pl[PL_O] = 6 * k.NH;
    L.pl[PL_TIN] = L.pl[PL_TOUT] = md(G - k.NIN);
    L.pl[PL_RED] = md(G - k.NIN - L.nred);
  } else {
    L.pl[PL_QKV] = L.pl[PL_O] = L.pl[PL_CAO] = L.pl[PL_GU] = L.pl[PL_DOWN] = 0;
    L.pl[PL_SA] = md(G - nattn);
    L.pl[PL_CA] = md(G - 2 * nattn);
    L.pl[PL_TIN] = md(G - k.NIN);
    L.pl[PL_RED] = md(G - k.NIN - L.nred);
    // the step tail's output tasks: with the reducers (passes); on the in-projection tasks' workgroups
    // (row-wise form), which run no reducer, so that the output tasks' prefetch (Wout rows and the final
    // modulation rows) is issued while the reducers still run rather than after one
    L.pl[PL_TOUT] = rows ? L.pl[PL_TIN] : L.pl[PL_RED];
  }
  return L;
}

inline int ceil16(int a) { return (a + 15) / 16 * 16; }
inline int ceil32(int a) { return (a + 31) / 32 * 32; }

long long frame_bytes(int H, int I, int nrp) {
  if (H == 768 && I == 3072) return Shape<768, 3072>::frame_bytes(nrp);
  if (H == 1024 && I == 4096) return Shape<1024, 4096>::frame_bytes(nrp);
  if (H == 256 && I == 512) return Shape<256, 512>::frame_bytes(nrp);
  return 0;
}
long long step_bytes(int H, int I, int nrp, int nxrows, int A) {
  long long x_off = 0;
  if (H == 768 && I == 3072) x_off = Shape<768, 3072>::step_x_off(nrp);
  if (H == 1024 && I == 4096) x_off = Shape<1024, 4096>::step_x_off(nrp);
  if (H == 256 && I == 512) x_off = Shape<256, 512>::step_x_off(nrp);
  return x_off + (long long)((nxrows * A * 4 + 255) / 256 * 256);
}

}  // namespace

struct mkx_handle {
  mkx_dims d;
  int device = 0;
  int G = 0;
  unsigned nx[MAX_XCD] = {};
  unsigned xmask = 0;
  const void* kernel = nullptr;
  char *wqkv = nullptr, *wo = nullptr, *wqca = nullptr, *woca = nullptr, *wgu = nullptr, *wd = nullptr;  // packed chunks
  float* scales = nullptr;  // fp8: [L][3H] qkv | [L][H] o | [L][H] ca q | [L][H] ca o | [L][I] gate | [L][I] up | [L][H] down
  int w8 = 0;
  bf16_t *qn = nullptr, *kn = nullptr, *qcan = nullptr;
  float *win = nullptr, *bin = nullptr, *wout = nullptr, *bout = nullptr;
  char* frames = nullptr;
  size_t frames_cap = 0;
  char* steps = nullptr;
  size_t steps_cap = 0;
  bf16_t* vts = nullptr;  // per-launch V^T copies of the memory and cross-attention V caches
  size_t vts_cap = 0;
  BarState* bar = nullptr;
  unsigned long long* flags = nullptr;  // [FLAG_KINDS][FLAG_MAX][FLAG_STRIDE] ready epochs
  long long* prof = nullptr;
  int prof_len = 0;
  int profile = 0;
  int plain_launch = 0;  // MKX_PLAIN_LAUNCH=1 at creation: hipLaunchKernel instead of the cooperative launch
  const void* kernel_rows = nullptr;  // the instantiation with row-wise GEMM stages
  const void* kernel_ys = nullptr;    // the twins of both with scaled AdaRMS operands (an operand shift)
  const void* kernel_rows_ys = nullptr;
  const void* kernel_pairs = nullptr;  // the row-wise instantiations with two-tile self-attention tasks (fp8)
  const void* kernel_pairs_ys = nullptr;
  const void* kernel_long = nullptr;  // the form with passes for sources beyond the three-chunk ring
  const void* kernel_long_ys = nullptr;
  int gemm_form = -1;    // MKX_GEMM_FORM at creation: 0 passes, 1 row-wise, -1 chosen per launch
  int last_form = -1;    // form of the last launch (0 passes, 1 row-wise; -1 before the first)
  unsigned spin_limit = SPIN_LIMIT;
  int operand_shift = 0;  // AdaRMS operands stored as y 2^-shift (mkx_set_operand_shift)
  int captured = 0;      // a launch of this handle was captured into a graph: its scratch pointers are frozen
  unsigned long long gen_before = 0;
  long long last_nbar = 0;
  long long weight_bytes = 0;
};

static void free_handle(mkx_handle* h) {
  if (!h) return;
  void* ptrs[] = {h->wqkv, h->wo, h->wqca, h->woca, h->wgu, h->wd, h->qn, h->kn, h->qcan, h->win, h->bin,
                  h->wout, h->bout, h->frames, h->steps, h->vts, h->bar, h->flags, h->scales};
  for (void* p : ptrs)
    if (p) (void)hipFree(p);
  delete h;
}

struct mkx_source {
  mkx_source_dims dims{};
  bf16_t* wkp = nullptr;   // [L][NH][C/32][4][64][8] fragment-order K weights
  bf16_t* wvp = nullptr;
  bf16_t* kn = nullptr;    // [L, 64]
  bf16_t* ctxp = nullptr;  // staging: the call's context in fragment order
  int ncu = 256;           // compute units of the handle's device (read once, at creation)
};

static void free_source(mkx_source* h) {
  if (!h) return;
  for (void* p : {(void*)h->wkp, (void*)h->wvp, (void*)h->kn, (void*)h->ctxp})
    if (p) (void)hipFree(p);
  delete h;
}

extern "C" {

int32_t mkx_abi_version(void) { return MKX_ABI_VERSION; }

const char* mkx_last_error(void) { return g_err.c_str(); }

const char* mkx_status_string(int status) {
  switch (status) {
    case MKX_OK: return "ok";
    case MKX_EINVAL: return "invalid argument";
    case MKX_ENORESIDENT: return "persistent grid cannot be co-resident";
    case MKX_EHIP: return "HIP runtime error";
    case MKX_ETIMEOUT: return "grid barrier wait exceeded its spin bound";
    case MKX_ENOMEM: return "out of device memory";
    case MKX_EUNSUPPORTED: return "unsupported shape";
    case MKX_ERANGE: return "value beyond the fp16 range of the GEMM operands";
    default: return "unknown status";
  }
}

int mkx_create(const mkx_dims* dims, const mkx_weights* w, void* stream_, mkx_handle** out) {
  if (!dims || !w || !out) return fail(MKX_EINVAL, "null argument");
  *out = nullptr;
  const mkx_dims d = *dims;
  if (d.L < 1 || d.L > MKX_MAX_LAYERS) return fail(MKX_EINVAL, "L must be in [1, 32]");
  if (d.HD != HD) return fail(MKX_EUNSUPPORTED, "head dim must be 64");
  if (d.NH * d.HD != d.H) return fail(MKX_EINVAL, "H must equal NH * HD");
  if (d.A != 32) return fail(MKX_EUNSUPPORTED, "padded action width A must be 32");
  if (d.weight_dtype != MKX_WEIGHTS_BF16 && d.weight_dtype != MKX_WEIGHTS_FP8_E4M3) return fail(MKX_EUNSUPPORTED, "unknown weight dtype");
  const bool w8 = d.weight_dtype == MKX_WEIGHTS_FP8_E4M3;
  if (d.activation != MKX_ACT_SILU && d.activation != MKX_ACT_GELU_TANH) return fail(MKX_EINVAL, "unknown activation");
  if (d.max_batch < 1 || d.max_batch > MAX_BATCH) return fail(MKX_EINVAL, "max_batch must be in [1, 16]");
  if (d.max_rows < 1 || d.max_rows > 128) return fail(MKX_EINVAL, "max_rows (own rows per sample) must be in [1, 128]");
  if (d.max_mem_rows < 0 || d.max_mem_rows > 256) return fail(MKX_EINVAL, "max_mem_rows must be in [0, 256]");
  const void* kern = pick_kernel(d.H, d.I, w8, false);
  if (!kern) return fail(MKX_EUNSUPPORTED, "no kernel instantiation for (H, I) = (" + std::to_string(d.H) + ", " + std::to_string(d.I) + ")");
  if (!w->wqkv || !w->wo || !w->wqca || !w->woca || !w->wg || !w->wu || !w->wd || !w->qn || !w->kn || !w->qcan ||
      !w->win || !w->bin || !w->wout || !w->bout)
    return fail(MKX_EINVAL, "null weight pointer");
  if (w8 && (!w->wqkv_scale || !w->wo_scale || !w->wqca_scale || !w->woca_scale || !w->wg_scale || !w->wu_scale || !w->wd_scale))
    return fail(MKX_EINVAL, "fp8 weights need every per-output-channel scale pointer");
  hipStream_t stream = (hipStream_t)stream_;
  mkx_handle* h = new mkx_handle();
  h->d = d;
  h->w8 = w8 ? 1 : 0;
  h->kernel = kern;
  h->kernel_rows = pick_kernel(d.H, d.I, w8, true);
  h->kernel_ys = pick_kernel(d.H, d.I, w8, false, true);
  h->kernel_rows_ys = pick_kernel(d.H, d.I, w8, true, true);
  h->kernel_pairs = pick_kernel(d.H, d.I, w8, true, false, true);
  h->kernel_pairs_ys = pick_kernel(d.H, d.I, w8, true, true, true);
  h->kernel_long = pick_kernel(d.H, d.I, w8, false, false, false, true);
  h->kernel_long_ys = pick_kernel(d.H, d.I, w8, false, true, false, true);
  auto bail = [&](int code) { free_handle(h); return code; };
#define HCHK(x)                                                                                       \
  do {                                                                                                \
    hipError_t e_ = (x);                                                                              \
    if (e_ != hipSuccess) return bail(fail(MKX_EHIP, std::string(#x) + ": " + hipGetErrorString(e_))); \
  } while (0)
  HCHK(hipGetDevice(&h->device));
  hipDeviceProp_t prop;
  HCHK(hipGetDeviceProperties(&prop, h->device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return bail(fail(MKX_EUNSUPPORTED, std::string("this library is built for gfx950, device is ") + prop.gcnArchName));
  if (!prop.cooperativeLaunch) return bail(fail(MKX_ENORESIDENT, "device does not support cooperative launch"));
  int per_cu = 0;
  HCHK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, NTHREADS, 0));
  if (per_cu < 1) return bail(fail(MKX_ENORESIDENT, "megakernel does not fit one workgroup per CU"));
  HCHK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, h->kernel_rows, NTHREADS, 0));
  if (per_cu < 1) return bail(fail(MKX_ENORESIDENT, "megakernel (row-wise GEMM form) does not fit one workgroup per CU"));
  for (const void* k : {h->kernel_ys, h->kernel_rows_ys}) {
    HCHK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, NTHREADS, 0));
    if (per_cu < 1) return bail(fail(MKX_ENORESIDENT, "megakernel (scaled AdaRMS operands) does not fit one workgroup per CU"));
  }
  for (const void* k : {h->kernel_pairs, h->kernel_pairs_ys, h->kernel_long, h->kernel_long_ys}) {
    if (!k) continue;
    HCHK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, NTHREADS, 0));
    if (per_cu < 1) return bail(fail(MKX_ENORESIDENT, "megakernel (two-tile attention tasks) does not fit one workgroup per CU"));
  }
  h->G = prop.multiProcessorCount;
  {
    const char* pl = std::getenv("MKX_PLAIN_LAUNCH");
    h->plain_launch = (pl && pl[0] == '1') ? 1 : 0;
    const char* gf = std::getenv("MKX_GEMM_FORM");
    if (gf && std::strcmp(gf, "passes") == 0) h->gemm_form = 0;
    else if (gf && std::strcmp(gf, "rows") == 0) h->gemm_form = 1;
  }
  // XCD of each workgroup of a G-workgroup launch; the barrier's per-XCD counts come from it
  unsigned* dx = nullptr;
  HCHK(hipMalloc(&dx, sizeof(unsigned) * h->G));
  hipLaunchKernelGGL(xcc_probe, dim3(h->G), dim3(NTHREADS), 0, stream, dx);
  std::vector<unsigned> hx(h->G);
  HCHK(hipMemcpyAsync(hx.data(), dx, sizeof(unsigned) * h->G, hipMemcpyDeviceToHost, stream));
  HCHK(hipStreamSynchronize(stream));
  (void)hipFree(dx);
  // One workgroup fits per CU (LDS) and the grid has one workgroup per CU, so every XCD hosts exactly as
  // many workgroups as it has CUs. The probe finds which XCDs exist; the dispatcher's rotation between
  // launches changes which workgroup lands where, not how many land on each XCD.
  if (h->G > 256) return bail(fail(MKX_EUNSUPPORTED, "more than 256 CUs"));
  // the top of the grid holds the step tail's H/32 in-projection tasks and the 16 down-projection reducers
  if (h->G < d.H / 32 + 16) return bail(fail(MKX_ENORESIDENT, "too few CUs for the step tail and the down-projection reducers"));
  int nxcd = 0;
  for (int i = 0; i < h->G; ++i) {
    if (hx[i] >= MAX_XCD) return bail(fail(MKX_EUNSUPPORTED, "unexpected XCC id"));
    if (!((h->xmask >> hx[i]) & 1u)) ++nxcd;
    h->xmask |= 1u << hx[i];
  }
  if (nxcd < 1 || h->G % nxcd != 0) return bail(fail(MKX_EUNSUPPORTED, "CU count not divisible by the XCD count"));
  for (int x = 0; x < MAX_XCD; ++x) h->nx[x] = ((h->xmask >> x) & 1u) ? (unsigned)(h->G / nxcd) : 0u;
  // packed weights
  const int L = d.L, H = d.H, I = d.I;
  auto alloc = [&](void** p, size_t bytes) { return hipMalloc(p, bytes); };
  const size_t sq = (size_t)L * 3 * H * H, so = (size_t)L * H * H, sgu = (size_t)L * 2 * I * H, sd = (size_t)L * H * I;
  const size_t wb = w8 ? 1 : 2;  // bytes per weight
  HCHK(alloc((void**)&h->wqkv, sq * wb));
  HCHK(alloc((void**)&h->wo, so * wb));
  HCHK(alloc((void**)&h->wqca, so * wb));
  HCHK(alloc((void**)&h->woca, so * wb));
  HCHK(alloc((void**)&h->wgu, sgu * wb));
  HCHK(alloc((void**)&h->wd, sd * wb));
  // dls, tstride, toff in chunks (16 x 32 weights)
  // bf16 weights are packed as fp16, the GEMMs' MFMA operand type; a weight beyond the fp16 range is refused
  int* range = nullptr;
  HCHK(hipMalloc(&range, sizeof(int)));
  HCHK(hipMemsetAsync(range, 0, sizeof(int), stream));
  auto pack = [&](const void* src, char* dst, int N, int K, long long dls, int tstride, int toff, int pairs) {
    const long long total = (long long)L * (N / 16) * (K / 32) * 64;
    const dim3 grid((unsigned)((total + 255) / 256));
    if (w8)
      hipLaunchKernelGGL(pack_tiles8, grid, dim3(256), 0, stream, (const uint8_t*)src, (uint8_t*)dst, L, N, K, dls, tstride, toff, pairs);
    else
      hipLaunchKernelGGL(pack_tiles, grid, dim3(256), 0, stream, (const bf16_t*)src, (bf16_t*)dst, L, N, K, dls * 512, tstride, toff, pairs, range);
  };
  const int kbh = H / 32, kbi = I / 32;
  pack(w->wqkv, h->wqkv, 3 * H, H, 3LL * (H / 16) * kbh, kbh, 0, 1);
  pack(w->wo, h->wo, H, H, (long long)(H / 16) * kbh, kbh, 0, 0);
  pack(w->wqca, h->wqca, H, H, (long long)(H / 16) * kbh, kbh, 0, 0);
  pack(w->woca, h->woca, H, H, (long long)(H / 16) * kbh, kbh, 0, 0);
  pack(w->wg, h->wgu, I, H, 2LL * (I / 16) * kbh, 2 * kbh, 0, 0);
  pack(w->wu, h->wgu, I, H, 2LL * (I / 16) * kbh, 2 * kbh, kbh, 0);
  pack(w->wd, h->wd, H, I, (long long)(H / 16) * kbi, kbi, 0, 0);
  HCHK(hipGetLastError());
  {
    int big = 0;
    HCHK(hipMemcpyAsync(&big, range, sizeof(int), hipMemcpyDeviceToHost, stream));
    HCHK(hipStreamSynchronize(stream));
    (void)hipFree(range);
    if (big) return bail(fail(MKX_ERANGE, "a bf16 weight exceeds the fp16 range (65504) of the GEMM operands"));
  }
  if (w8) {
    const size_t n = (size_t)L * (3 * H + 3 * H + 2 * I + H);
    HCHK(alloc((void**)&h->scales, n * 4));
    float* sc = h->scales;
    const float* src[7] = {w->wqkv_scale, w->wo_scale, w->wqca_scale, w->woca_scale, w->wg_scale, w->wu_scale, w->wd_scale};
    const size_t len[7] = {(size_t)3 * H, (size_t)H, (size_t)H, (size_t)H, (size_t)I, (size_t)I, (size_t)H};
    for (int k = 0; k < 7; ++k) {
      HCHK(hipMemcpyAsync(sc, src[k], (size_t)L * len[k] * 4, hipMemcpyDeviceToDevice, stream));
      sc += (size_t)L * len[k];
    }
  }
  h->weight_bytes = (long long)(sq + 3 * so + sgu + sd) * (long long)wb;
  HCHK(alloc((void**)&h->qn, (size_t)L * HD * 2));
  HCHK(alloc((void**)&h->kn, (size_t)L * HD * 2));
  HCHK(alloc((void**)&h->qcan, (size_t)L * HD * 2));
  HCHK(hipMemcpyAsync(h->qn, w->qn, (size_t)L * HD * 2, hipMemcpyDeviceToDevice, stream));
  HCHK(hipMemcpyAsync(h->kn, w->kn, (size_t)L * HD * 2, hipMemcpyDeviceToDevice, stream));
  HCHK(hipMemcpyAsync(h->qcan, w->qcan, (size_t)L * HD * 2, hipMemcpyDeviceToDevice, stream));
  HCHK(alloc((void**)&h->win, (size_t)d.A * H * 4));
  HCHK(alloc((void**)&h->bin, (size_t)H * 4));
  HCHK(alloc((void**)&h->wout, (size_t)d.A * H * 4));
  HCHK(alloc((void**)&h->bout, (size_t)d.A * 4));
  HCHK(hipMemcpyAsync(h->win, w->win, (size_t)d.A * H * 4, hipMemcpyDeviceToDevice, stream));
  HCHK(hipMemcpyAsync(h->bin, w->bin, (size_t)H * 4, hipMemcpyDeviceToDevice, stream));
  HCHK(hipMemcpyAsync(h->wout, w->wout, (size_t)d.A * H * 4, hipMemcpyDeviceToDevice, stream));
  HCHK(hipMemcpyAsync(h->bout, w->bout, (size_t)d.A * 4, hipMemcpyDeviceToDevice, stream));
  HCHK(alloc((void**)&h->bar, sizeof(BarState)));
  HCHK(hipMemsetAsync(h->bar, 0, sizeof(BarState), stream));
  HCHK(alloc((void**)&h->flags, sizeof(unsigned long long) * FLAG_KINDS * FLAG_MAX * FLAG_STRIDE));
  HCHK(hipMemsetAsync(h->flags, 0, sizeof(unsigned long long) * FLAG_KINDS * FLAG_MAX * FLAG_STRIDE, stream));
  HCHK(hipStreamSynchronize(stream));
#undef HCHK
  *out = h;
  return MKX_OK;
}

int mkx_set_spin_limit(mkx_handle* h, uint32_t polls) {
  if (!h) return fail(MKX_EINVAL, "null handle");
  h->spin_limit = polls ? polls : SPIN_LIMIT;
  return MKX_OK;
}

int mkx_set_operand_shift(mkx_handle* h, int32_t shift) {
  if (!h) return fail(MKX_EINVAL, "null handle");
  if (shift < 0 || shift > 30) return fail(MKX_EINVAL, "mkx_set_operand_shift: shift must be in [0, 30]");
  h->operand_shift = shift;
  return MKX_OK;
}

int64_t mkx_barriers(const mkx_handle* h, int32_t n_steps) {
  if (!h || n_steps < 0) return -1;
  return 1 + (int64_t)n_steps * (mkx::STAGES_PER_LAYER * h->d.L + 1);
}

int mkx_set_profile(mkx_handle* h, int64_t* buf, int32_t len) {
  if (!h) return fail(MKX_EINVAL, "null handle");
  if (buf && len < 2) return fail(MKX_EINVAL, "profile buffer too short");
  h->prof = (long long*)buf;
  h->prof_len = buf ? len : 0;
  h->profile = buf ? 1 : 0;
  return MKX_OK;
}

int mkx_run(mkx_handle* h, const mkx_step_args* a, void* stream_) {
  if (!h || !a) return fail(MKX_EINVAL, "null argument");
  const mkx_dims& d = h->d;
  hipStream_t stream = (hipStream_t)stream_;
  const int L = d.L, H = d.H, I = d.I;
  if (a->n_steps < 1) return fail(MKX_EINVAL, "n_steps must be >= 1");
  // step tail: x' of the real action dims (32 KB) and Wout's real-dim rows (64 KB) are staged in LDS
  if ((long long)a->B * a->T_act * a->action_dim * 4 > 32 * 1024) return fail(MKX_EUNSUPPORTED, "B * T_act * action_dim too large for the step tail");
  if ((long long)a->action_dim * H * 4 > 64 * 1024) return fail(MKX_EUNSUPPORTED, "action_dim * H too large for the step tail");
  // the in-projection task's Win columns [action_dim][32] are staged in 3 KB of LDS
  if (a->action_dim > 24) return fail(MKX_EUNSUPPORTED, "action_dim above 24 is not supported by the step tail");
  if (a->B < 1 || a->B > d.max_batch) return fail(MKX_EINVAL, "B out of range");
  if (a->T_act < 1 || a->R_reg < 0) return fail(MKX_EINVAL, "T_act must be >= 1 and R_reg >= 0");
  const int Mq = a->T_act + a->R_reg;
  if (Mq > d.max_rows || Mq > 128) return fail(MKX_EINVAL, "T_act + R_reg exceeds max_rows");
  if (a->action_dim < 1 || a->action_dim > d.A) return fail(MKX_EINVAL, "action_dim must be in [1, A]");
  if (a->PM < 1 || a->PM > 256 || a->PM > d.max_mem_rows) return fail(MKX_EINVAL, "PM must be in [1, min(256, max_mem_rows)]");
  if (a->SP < 1 || a->SP > d.max_src_rows) return fail(MKX_EINVAL, "SP must be in [1, max_src_rows]");
  if (!a->x_in || !a->x_out || !a->mods || !a->dt || !a->kv_start || !a->ca_len || !a->sa_cos || !a->sa_sin ||
      !a->ca_cos || !a->ca_sin)
    return fail(MKX_EINVAL, "null input pointer");
  if (a->R_reg > 0 && !a->reg_tok) return fail(MKX_EINVAL, "reg_tok is required when R_reg > 0");
  if ((a->cur_k != nullptr) != (a->cur_v != nullptr)) return fail(MKX_EINVAL, "cur_k and cur_v must both be set or both NULL");
  for (int l = 0; l < L; ++l)
    if (!a->memk[l] || !a->memv[l] || !a->kca[l] || !a->vca[l]) return fail(MKX_EINVAL, "null per-layer cache pointer");
  if (a->mods_stride_step < 9LL * L * H + 2 * H) return fail(MKX_EINVAL, "mods_stride_step is smaller than MODW = 9 L H + 2 H");
  const int Mqp = ceil16(Mq);  // each sample's rows start on a 16-row tile
  const int NR = a->B * Mqp;
  const int NRP = ceil16(NR);
  if (NRP > MAX_ROWS_PADDED) return fail(MKX_EUNSUPPORTED, "B * (T_act + R_reg) too large for this library");
  if ((long long)a->B * (H / 64) * (Mqp / 16) > FLAG_MAX) return fail(MKX_EUNSUPPORTED, "too many attention tasks for the ready-epoch table");
  // LDS working sets (layout in mkx_kernel.h): self-attention keeps one query tile, the own rows' K and
  // V^T (hi + lo, 32-key blocks, at most 128 rows) and the wave-merge area in the 88 KB activation region;
  // the GEMM stages stage every sample's modulation slices (2 H floats) in 56 KB.
  if ((long long)a->B * 2 * H * 4 > 56 * 1024) return fail(MKX_EUNSUPPORTED, "batch too large to stage its modulation slices in LDS");
  const ShapeK sk = shape_k(H, I, h->w8 != 0);
  Layout lay = plan_layout(sk, h->G, NRP / 16, a->B, Mqp / 16, H, d.A, tail_outputs(false, a->B * a->T_act, d.A), false);
  // Row-wise form where a gate/up task would need more than one pass of row tiles (its layout has tasks of one
  // column tile, and its step tail's output tasks, over row chunks, must number at most 64)
  const bool rows_fit = tail_outputs(true, a->B * a->T_act, d.A) <= 64;
  if (h->gemm_form == 1 && !rows_fit)
    return fail(MKX_EUNSUPPORTED, "MKX_GEMM_FORM=rows: the row-wise form's step tail needs at most 64 output tasks "
                                  "(B * T_act too large for it)");
  const bool rows = rows_fit && (h->gemm_form == 1 || (h->gemm_form < 0 && NRP / 16 > sk.RBMAX));
  if (rows) lay = plan_layout(sk, h->G, NRP / 16, a->B, Mqp / 16, H, d.A, tail_outputs(true, a->B * a->T_act, d.A), true);
  {
    // a task waits on at most 256 ready epochs (one poll of 4 x 64 lanes): gate/up on every CA out-projection
    // task, an out-projection task on every head of its rows; and on at most 64 (one load per poll) where
    // it waits on every out-projection task of a row group (cross-attention) or on the QKV tasks of its
    // head (self-attention)
    const int RTn = NRP / 16, NH = H / 64;
    if ((sk.HT / lay.nt_cao) * lay.rgs_cao > 256 || ((RTn + lay.rgs_o - 1) / lay.rgs_o) * NH > 256 ||
        ((RTn + lay.rgs_cao - 1) / lay.rgs_cao) * NH > 256 || sk.HT > 64 || 6 * lay.rgs_qkv > 64 || lay.nred > 256)
      return fail(MKX_EUNSUPPORTED, "row grouping needs more than 256 ready epochs per wait");
    if (lay.lds_mods + a->B * 2 * H * 4 > sk.SMALL) return fail(MKX_EUNSUPPORTED, "GEMM LDS map does not fit");
  }
  if (h->profile && mkx_barriers(h, a->n_steps) + 1 > h->prof_len) return fail(MKX_EINVAL, "profile buffer shorter than barriers + 1");
#ifdef MKX_TRACE
  if (h->profile && mkx::TRACE_BASE + (1 + mkx_barriers(h, a->n_steps)) * h->G * mkx::TRACE_SLOTS > h->prof_len)
    return fail(MKX_EINVAL, "trace buffer too short");
#endif
  // scratch: one frame per (step, layer), one step area per step; grown on demand
  const long long fb = frame_bytes(H, I, NRP);
  const long long sb = step_bytes(H, I, NRP, a->B * a->T_act, d.A);
  const size_t need_f = (size_t)fb * a->n_steps * L, need_s = (size_t)sb * a->n_steps;
  const int PMP = ceil32(a->PM), SPP = ceil32(a->SP);
  // V^T copies (bf16) and the split AdaRMS shift operands (B * H * 4 bytes per step, layer and AdaRMS)
  const size_t vt_bytes = (size_t)L * a->B * (H / 64) * (PMP + SPP) * 128;
  const size_t need_v = vt_bytes + (size_t)a->n_steps * L * 3 * a->B * H * 4;
  // Capture status first: growing the scratch synchronises the stream and reallocates, which a capturing
  // stream cannot do, and a graph captured earlier keeps the old scratch pointers in its kernel arguments.
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  HIPCHK(hipStreamIsCapturing(stream, &cs));
  const bool capturing = cs == hipStreamCaptureStatusActive;
  const bool grow = need_f > h->frames_cap || need_s > h->steps_cap || need_v > h->vts_cap;
  if (grow && capturing)
    return fail(MKX_EINVAL, "mkx_run under stream capture needs more scratch than the handle holds: run once eagerly "
                            "at this shape (or a larger one) before capturing");
  if (grow && h->captured)
    return fail(MKX_EUNSUPPORTED, "mkx_run: this shape needs more scratch, but a launch of this handle was captured and "
                                  "its graph holds the current scratch; warm up at the largest shape before capturing, or "
                                  "use a second handle");
  if (grow) {
    HIPCHK(hipStreamSynchronize(stream));
    if (need_f > h->frames_cap) {
      if (h->frames) HIPCHK(hipFree(h->frames));
      h->frames = nullptr;
      h->frames_cap = 0;
      if (hipMalloc(&h->frames, need_f) != hipSuccess) return fail(MKX_ENOMEM, "activation frames");
      HIPCHK(hipMemsetAsync(h->frames, 0, need_f, stream));  // operand slots no stage writes stay finite
      h->frames_cap = need_f;
    }
    if (need_s > h->steps_cap) {
      if (h->steps) HIPCHK(hipFree(h->steps));
      h->steps = nullptr;
      h->steps_cap = 0;
      if (hipMalloc(&h->steps, need_s) != hipSuccess) return fail(MKX_ENOMEM, "step areas");
      HIPCHK(hipMemsetAsync(h->steps, 0, need_s, stream));
      h->steps_cap = need_s;
    }
    if (need_v > h->vts_cap) {
      if (h->vts) HIPCHK(hipFree(h->vts));
      h->vts = nullptr;
      h->vts_cap = 0;
      if (hipMalloc(&h->vts, need_v) != hipSuccess) return fail(MKX_ENOMEM, "V^T copies");
      h->vts_cap = need_v;
    }
  }
  Params p;
  std::memset(&p, 0, sizeof(p));
  p.wqkv = h->wqkv; p.wo = h->wo; p.wqca = h->wqca; p.woca = h->woca; p.wgu = h->wgu; p.wd = h->wd;
  const long long wb = h->w8 ? 1 : 2;
  p.s_qkv = 3LL * H * H * wb; p.s_o = (long long)H * H * wb; p.s_gu = 2LL * I * H * wb; p.s_d = (long long)H * I * wb;
  {
    const float* sc = h->scales;  // null for bf16
    auto take = [&](size_t n) { const float* r = sc; if (sc) sc += (size_t)L * n; return r; };
    p.sc_qkv = take(3 * H); p.sc_o = take(H); p.sc_qca = take(H); p.sc_oca = take(H);
    p.sc_g = take(I); p.sc_u = take(I); p.sc_d = take(H);
  }
  p.qn = h->qn; p.kn = h->kn; p.qcan = h->qcan;
  p.win = h->win; p.bin = h->bin; p.wout = h->wout; p.bout = h->bout;
  p.x_in = a->x_in; p.x_out = a->x_out;
  p.mods = a->mods; p.mods_sb = a->mods_stride_b; p.mods_ss = a->mods_stride_step; p.mod_row0 = a->mod_row0;
  p.dt = a->dt;
  for (int l = 0; l < L; ++l) {
    p.memk[l] = (const bf16_t*)a->memk[l]; p.memv[l] = (const bf16_t*)a->memv[l];
    p.kca[l] = (const bf16_t*)a->kca[l]; p.vca[l] = (const bf16_t*)a->vca[l];
  }
  p.mem_sb = a->mem_stride_b; p.src_sb = a->src_stride_b;
  p.kv_start = a->kv_start; p.ca_len = a->ca_len;
  p.sa_cos = a->sa_cos; p.sa_sin = a->sa_sin; p.ca_cos = a->ca_cos; p.ca_sin = a->ca_sin;
  p.reg_tok = (const bf16_t*)a->reg_tok; p.cur_k = (bf16_t*)a->cur_k; p.cur_v = (bf16_t*)a->cur_v;
  p.n_steps = a->n_steps; p.action_dim = a->action_dim; p.T = a->T_act; p.R = a->R_reg; p.B = a->B;
  p.memvt = h->vts; p.cavt = h->vts + (size_t)L * a->B * (H / 64) * PMP * 64; p.SPP = SPP;
  p.shs = (char*)h->vts + vt_bytes;
  p.PM = a->PM; p.SP = a->SP; p.L = L; p.Mq = Mq; p.Mqp = Mqp; p.NR = NR; p.NRP = NRP; p.A = d.A;
  p.act = d.activation == MKX_ACT_GELU_TANH ? 1 : 0;
  p.qk_eps = d.qk_eps; p.sm_scale = 1.0f / 8.0f;
  // AdaRMS operands y 2^-shift: the sums of squares and eps scale by 2^-2 shift (exact), eps_final not
  p.yinv = std::ldexp(1.0f, -h->operand_shift);
  p.eps = std::ldexp(d.eps, -2 * h->operand_shift);
  p.eps_final = d.eps;
  p.frames = h->frames; p.frame_bytes = fb; p.steps = h->steps; p.step_bytes = sb;
  p.bar = h->bar; p.flags = h->flags;
  for (int x = 0; x < MAX_XCD; ++x) p.nx[x] = h->nx[x];
  p.xmask = h->xmask;
  p.prof = h->prof; p.profile = h->profile;
  p.spin_limit = h->spin_limit;
  for (int k = 0; k < PL_KINDS; ++k) p.pl[k] = lay.pl[k];
  p.rgs_qkv = lay.rgs_qkv; p.rgs_o = lay.rgs_o; p.rgs_cao = lay.rgs_cao;
  p.nt_o = lay.nt_o; p.nt_cao = lay.nt_cao; p.nt_down = lay.nt_down;
  p.lds_red = lay.lds_red; p.lds_mods = lay.lds_mods;
  p.tpr = lay.tpr; p.nred = lay.nred; p.nrg = lay.nrg;
  bool pairs;
  {
    // attention tasks of two query tiles (row-wise form): where the one-tile tasks outnumber the workgroups and
    // the two-tile tasks do not (cross-attention: and every source fits the three LDS ring slots)
    const int nhb = a->B * (H / 64), nqt = Mqp / 16;
    pairs = rows && nhb * nqt > h->G && nhb * ((nqt + 1) / 2) <= h->G;
    p.ca_grp = pairs && a->SP <= 384 ? 1 : 0;
    // self-attention: the fp8 kernels; the fp16 ones run a second query tile of a sample-head with its keys and
    // values still in LDS (two-tile tasks measured slower there: workload B 5.84 -> 5.90 ms)
    pairs = pairs && h->w8;
  }
  void* args[] = {&p};
  // the form with passes: sources beyond the three 128-row chunks of the cross-attention ring stream the rest
  const bool longsrc = !rows && a->SP > 384;
  const void* kern = h->operand_shift ? (pairs ? h->kernel_pairs_ys : rows ? h->kernel_rows_ys : longsrc ? h->kernel_long_ys : h->kernel_ys)
                                      : (pairs ? h->kernel_pairs : rows ? h->kernel_rows : longsrc ? h->kernel_long : h->kernel);
  if (capturing) h->captured = 1;
  if (capturing || h->plain_launch) {
    // co-residency was established at creation (one workgroup per CU fits); capture a plain launch
    HIPCHK(hipLaunchKernel(kern, dim3(h->G), dim3(NTHREADS), args, 0, stream));
  } else {
    HIPCHK(hipLaunchCooperativeKernel(kern, dim3(h->G), dim3(NTHREADS), args, 0, stream));
  }
  h->last_nbar = mkx_barriers(h, a->n_steps);
  h->last_form = rows ? 1 : 0;
  return MKX_OK;
}

int mkx_ring_append(const mkx_ring_args* a, void* stream_) {
  if (!a) return fail(MKX_EINVAL, "mkx_ring_append: args is NULL");
  if (a->L < 1 || a->L > MKX_MAX_LAYERS || a->B < 1 || a->NH < 1 || a->HD != 64 || a->PM < 1 || a->R < 1 ||
      a->R > a->PM)
    return fail(MKX_EINVAL, "mkx_ring_append: need 1 <= L <= 32, B >= 1, NH >= 1, HD == 64, 1 <= R <= PM");
  if ((int64_t)a->PM * a->NH * 4 > (int64_t)1 << 30 || a->B > 65535)
    return fail(MKX_EINVAL, "mkx_ring_append: shape too large");
  const int64_t row_elems = (int64_t)a->NH * 64;
  if (a->mem_stride_b < a->PM * row_elems && a->B > 1)
    return fail(MKX_EINVAL, "mkx_ring_append: mem_stride_b smaller than one sample's memory");
  if (!a->cur_k || !a->cur_v || !a->kv_start_in || !a->kv_start_out)
    return fail(MKX_EINVAL, "mkx_ring_append: cur_k, cur_v, kv_start_in and kv_start_out are required");
  if (a->kv_start_in == a->kv_start_out) return fail(MKX_EINVAL, "mkx_ring_append: kv_start_out aliases kv_start_in");
  if ((a->shift_cos == nullptr) != (a->shift_sin == nullptr) || (a->new_cos == nullptr) != (a->new_sin == nullptr))
    return fail(MKX_EINVAL, "mkx_ring_append: pass both or neither of each cos/sin pair");
  auto misaligned = [](const void* p) { return ((uintptr_t)p & 15u) != 0; };
  if (misaligned(a->cur_k) || misaligned(a->cur_v) || (a->mem_stride_b & 7))
    return fail(MKX_EINVAL, "mkx_ring_append: caches must be 16-byte aligned (mem_stride_b a multiple of 8)");
  // one sample's memory spans [p, p + (B - 1) stride + PM row) elements; out must not overlap any input
  const uint64_t span = (uint64_t)(((int64_t)a->B - 1) * a->mem_stride_b + a->PM * row_elems) * 2;
  for (int l = 0; l < a->L; ++l) {
    const void* ins[2] = {a->memk_in[l], a->memv_in[l]};
    const void* outs[2] = {a->memk_out[l], a->memv_out[l]};
    for (const void* p : ins)
      if (!p || misaligned(p)) return fail(MKX_EINVAL, "mkx_ring_append: memory input NULL or misaligned");
    for (const void* p : outs)
      if (!p || misaligned(p)) return fail(MKX_EINVAL, "mkx_ring_append: memory output NULL or misaligned");
    for (int l2 = 0; l2 < a->L; ++l2)
      for (const void* o : outs)
        for (const void* i : {a->memk_in[l2], a->memv_in[l2], a->cur_k, a->cur_v}) {
          const uint64_t po = (uint64_t)(uintptr_t)o, pi = (uint64_t)(uintptr_t)i;
          const uint64_t ispan = (i == a->cur_k || i == a->cur_v)
                                     ? (uint64_t)a->L * a->B * a->R * row_elems * 2 : span;
          if (po < pi + ispan && pi < po + span)
            return fail(MKX_EINVAL, "mkx_ring_append: an output buffer overlaps an input (use two buffer sets)");
        }
  }
  hipStream_t stream = (hipStream_t)stream_;
  const int lanes = a->PM * a->NH * 4;
  dim3 grid((lanes + RING_BLOCK - 1) / RING_BLOCK, 2 * a->L, a->B);
  hipLaunchKernelGGL(ring_append_kernel, grid, dim3(RING_BLOCK), 0, stream, *a);
  HIPCHK(hipGetLastError());
  return MKX_OK;
}

}  // extern "C"

// Static staging for mkx_source_run_noalloc: the call's context in fragment order (ceil32(B * SP) + PREP_ROW_PAD
// rows of C bf16 values, prep_ctx_bytes) lives in this file-scope device array instead of the handle's allocation. Each GPU holds its own copy until the
// process ends; calls on one GPU share it (the last call's contents stay, and calls that overlap race).
constexpr long long SOURCE_SCRATCH_BYTES = 16LL << 20;
static __device__ __align__(256) char scratch[SOURCE_SCRATCH_BYTES];

namespace {
constexpr int SCRATCH_MAX_DEVICES = 64;
std::atomic<void*> g_scratch_ptr[SCRATCH_MAX_DEVICES];
std::mutex g_scratch_mu;

// The device address of `scratch` on the current device (the host-side name is only a stand-in): looked up
// once per device with that device current, then cached.
int source_scratch(void** out) {
  int dev = 0;
  HIPCHK(hipGetDevice(&dev));
  if (dev < 0 || dev >= SCRATCH_MAX_DEVICES) return fail(MKX_EUNSUPPORTED, "device index beyond the static scratch table");
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      HIPCHK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
      if (!p) return fail(MKX_EHIP, "hipGetSymbolAddress(scratch) returned NULL");
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return MKX_OK;
}

// Validation shared by mkx_source_run and mkx_source_run_noalloc.
int source_args_check(const mkx_source* h, const mkx_source_args* a, const char* who) {
  const std::string w(who);
  if (!h || !a) return fail(MKX_EINVAL, w + ": handle or args is NULL");
  const mkx_source_dims& d = h->dims;
  if (a->B < 1 || a->SP < 1 || (int64_t)a->B * a->SP > d.max_rows)
    return fail(MKX_EINVAL, w + ": need B, SP >= 1 and B * SP <= max_rows");
  const int64_t row_elems = (int64_t)d.NH * 64;
  if (a->B > 1 && a->src_stride_b < a->SP * row_elems)
    return fail(MKX_EINVAL, w + ": src_stride_b smaller than one sample's cache");
  if (a->src_stride_b & 3) return fail(MKX_EINVAL, w + ": src_stride_b must be a multiple of 4");
  auto bad = [](const void* p, uintptr_t align) { return p == nullptr || ((uintptr_t)p & (align - 1)) != 0; };
  if (bad(a->ctx, 16) || bad(a->ca_len, 4) || bad(a->cos, 4) || bad(a->sin, 4))
    return fail(MKX_EINVAL, w + ": ctx, ca_len, cos, sin: NULL or misaligned");
  for (int l = 0; l < d.L; ++l)
    if (bad(a->kca[l], 8) || bad(a->vca[l], 8)) return fail(MKX_EINVAL, w + ": kca / vca NULL or not 8-byte aligned");
  return MKX_OK;
}

// Row tiles per wave of prepare_source_kernel for nrows source rows on ncu compute units: the one whose
// busiest CU has the least work, counting a workgroup's fixed cost (its first k-blocks in flight, the
// epilogue) as one row tile.
int prep_rtw(int nrows, int ncol_groups, int ncu) {
  const int nrt = (nrows + 15) / 16;
  int best = 2;
  long long best_cost = -1;
  for (int rtw = 2; rtw <= 5; ++rtw) {
    const long long nwg = (long long)((nrt + 2 * rtw - 1) / (2 * rtw)) * ncol_groups;
    const long long cost = (nwg + ncu - 1) / ncu * (rtw + 1);
    if (best_cost < 0 || cost < best_cost) { best_cost = cost; best = rtw; }
  }
  return best;
}
// Packed context bytes of a preparation of nrows rows (padded to a whole workgroup of the largest kind)
long long prep_ctx_bytes(int nrows, int C) { return (long long)((nrows + 31) / 32 * 32 + PREP_ROW_PAD) * C * 2; }

// The two launches of a source preparation, the packed context staged at ctxp.
int source_launch(const mkx_source* h, const mkx_source_args* a, bf16_t* ctxp, hipStream_t stream) {
  const mkx_source_dims& d = h->dims;
  const int nrows = a->B * a->SP;
  const int np = (d.NH + 1) / 2, ncg = d.L * 2 * np;
  const int rtw = prep_rtw(nrows, ncg, h->ncu), wg_rows = 32 * rtw;
  const int ngroups = (nrows + wg_rows - 1) / wg_rows;
  // packed pieces: rows padded with zeros to whole workgroups
  const long long n_x = (long long)ngroups * wg_rows * d.C / 8;
  // packed in groups of a workgroup's 2 rtw row tiles, so that one k-block of a workgroup's rows is contiguous
  hipLaunchKernelGGL(pack_rows_kernel, dim3((unsigned)((n_x + 255) / 256)), dim3(256), 0, stream, (const bf16_t*)a->ctx,
                     ctxp, nrows, d.C, 2 * rtw, n_x);
  SourceParams p{};
  p.L = d.L; p.NH = d.NH; p.C = d.C; p.B = a->B; p.SP = a->SP;
  p.ctxp = ctxp; p.wkp = h->wkp; p.wvp = h->wvp; p.k_norm = h->kn;
  p.ca_len = a->ca_len; p.cos = a->cos; p.sin = a->sin;
  for (int l = 0; l < d.L; ++l) { p.kca[l] = a->kca[l]; p.vca[l] = a->vca[l]; }
  p.src_sb = a->src_stride_b;
  p.eps = d.eps;
  const dim3 grid((unsigned)ngroups, (unsigned)ncg);
  // the production context width (2048) runs the fully unrolled k-loop
  const bool c2048 = d.C == 2048;
  switch (rtw) {
    case 2: if (c2048) hipLaunchKernelGGL((prepare_source_kernel<2, 64>), grid, dim3(PREP_BLOCK), 0, stream, p);
            else hipLaunchKernelGGL((prepare_source_kernel<2, 0>), grid, dim3(PREP_BLOCK), 0, stream, p); break;
    case 3: if (c2048) hipLaunchKernelGGL((prepare_source_kernel<3, 64>), grid, dim3(PREP_BLOCK), 0, stream, p);
            else hipLaunchKernelGGL((prepare_source_kernel<3, 0>), grid, dim3(PREP_BLOCK), 0, stream, p); break;
    case 4: if (c2048) hipLaunchKernelGGL((prepare_source_kernel<4, 64>), grid, dim3(PREP_BLOCK), 0, stream, p);
            else hipLaunchKernelGGL((prepare_source_kernel<4, 0>), grid, dim3(PREP_BLOCK), 0, stream, p); break;
    default: if (c2048) hipLaunchKernelGGL((prepare_source_kernel<5, 64>), grid, dim3(PREP_BLOCK), 0, stream, p);
             else hipLaunchKernelGGL((prepare_source_kernel<5, 0>), grid, dim3(PREP_BLOCK), 0, stream, p); break;
  }
  HIPCHK(hipGetLastError());
  return MKX_OK;
}
}  // namespace

extern "C" {

int mkx_source_create(const mkx_source_dims* d, const void* wk, const void* wv, const void* k_norm, void* stream_,
                      mkx_source** out) {
  if (!out) return fail(MKX_EINVAL, "mkx_source_create: out is NULL");
  *out = nullptr;
  if (!d) return fail(MKX_EINVAL, "mkx_source_create: dims is NULL");
  if (d->L < 1 || d->L > MKX_MAX_LAYERS || d->NH < 1 || d->HD != 64 || d->C < 32 || (d->C & 31) || d->max_rows < 1)
    return fail(MKX_EINVAL, "mkx_source_create: need 1 <= L <= 32, NH >= 1, HD == 64, C a multiple of 32, max_rows >= 1");
  if ((int64_t)d->L * 2 * d->NH > 65535 || (int64_t)d->max_rows * d->C > ((int64_t)1 << 34) ||
      (int64_t)d->L * d->NH * 64 * d->C > ((int64_t)1 << 34))
    return fail(MKX_EINVAL, "mkx_source_create: shape too large");
  if (!(d->eps >= 0.f)) return fail(MKX_EINVAL, "mkx_source_create: eps must be >= 0");
  auto bad16 = [](const void* p) { return p == nullptr || ((uintptr_t)p & 15u) != 0; };
  if (bad16(wk) || bad16(wv) || k_norm == nullptr || ((uintptr_t)k_norm & 1u))
    return fail(MKX_EINVAL, "mkx_source_create: wk / wv NULL or not 16-byte aligned, or k_norm NULL / misaligned");
  hipStream_t stream = (hipStream_t)stream_;
  mkx_source* h = new mkx_source();
  h->dims = *d;
  {
    // the device's CU count, which sizes every call's launch (read here so that calls query nothing)
    int dev = 0;
    hipDeviceProp_t pr;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&pr, dev) == hipSuccess && pr.multiProcessorCount > 0)
      h->ncu = pr.multiProcessorCount;
  }
  const int64_t wel = (int64_t)d->L * d->NH * 64 * d->C;
  auto cleanup = [&](int code, const std::string& msg) {
    free_source(h);
    return fail(code, msg);
  };
  if (hipMalloc(&h->wkp, wel * 2) != hipSuccess || hipMalloc(&h->wvp, wel * 2) != hipSuccess ||
      hipMalloc(&h->kn, (size_t)d->L * 64 * 2) != hipSuccess || hipMalloc(&h->ctxp, (size_t)prep_ctx_bytes(d->max_rows, d->C)) != hipSuccess)
    return cleanup(MKX_ENOMEM, "mkx_source_create: device allocation failed");
  // weights in fragment order: 16-row groups of one head (S = 4) per head of every layer
  const long long n_w = wel / 8;
  const int S = 4, rows_w = d->L * d->NH * 64;
  hipLaunchKernelGGL(pack_rows_kernel, dim3((unsigned)((n_w + 255) / 256)), dim3(256), 0, stream, (const bf16_t*)wk,
                     h->wkp, rows_w, d->C, S, n_w);
  hipLaunchKernelGGL(pack_rows_kernel, dim3((unsigned)((n_w + 255) / 256)), dim3(256), 0, stream, (const bf16_t*)wv,
                     h->wvp, rows_w, d->C, S, n_w);
  if (hipGetLastError() != hipSuccess ||
      hipMemcpyAsync(h->kn, k_norm, (size_t)d->L * 64 * 2, hipMemcpyDeviceToDevice, stream) != hipSuccess ||
      hipStreamSynchronize(stream) != hipSuccess)
    return cleanup(MKX_EHIP, "mkx_source_create: weight packing failed");
  {
    // the static scratch of mkx_source_run_noalloc on this device, looked up now (set-up time)
    void* sp = nullptr;
    const int rs = source_scratch(&sp);
    if (rs != MKX_OK) {
      const std::string msg = g_err;
      return cleanup(rs, msg);
    }
  }
  *out = h;
  return MKX_OK;
}

int mkx_source_run(mkx_source* h, const mkx_source_args* a, void* stream_) {
  const int rc = source_args_check(h, a, "mkx_source_run");
  if (rc != MKX_OK) return rc;
  return source_launch(h, a, h->ctxp, (hipStream_t)stream_);
}

int mkx_source_run_noalloc(mkx_source* h, const mkx_source_args* a, void* stream_) {
  const int rc = source_args_check(h, a, "mkx_source_run_noalloc");
  if (rc != MKX_OK) return rc;
  const long long need = prep_ctx_bytes(a->B * a->SP, h->dims.C);
  if (need > SOURCE_SCRATCH_BYTES)
    return fail(MKX_EINVAL, "mkx_source_run_noalloc: the packed context (" + std::to_string(need) +
                                " bytes) exceeds the static scratch of " + std::to_string(SOURCE_SCRATCH_BYTES) + " bytes");
  void* sp = nullptr;
  const int rs = source_scratch(&sp);
  if (rs != MKX_OK) return rs;
  return source_launch(h, a, (bf16_t*)sp, (hipStream_t)stream_);
}

int mkx_source_destroy(mkx_source* h) {
  free_source(h);
  return MKX_OK;
}

int mkx_modulations(const mkx_modproj_args* a, void* stream_) {
  if (!a) return fail(MKX_EINVAL, "mkx_modulations: args is NULL");
  if (a->R < 1 || a->N < 16 || (a->N & 15) || a->R > (1 << 20))
    return fail(MKX_EINVAL, "mkx_modulations: need R >= 1 and N a positive multiple of 16");
  if (a->K != 256 && a->K != 512 && a->K != 768 && a->K != 1024)
    return fail(MKX_EUNSUPPORTED, "mkx_modulations: K must be 256, 512, 768 or 1024");
  if (a->c_stride < a->K || (a->c_stride & 3) || a->out_stride < a->N || (a->out_stride & 3))
    return fail(MKX_EINVAL, "mkx_modulations: strides must cover a row and be multiples of 4");
  auto bad16 = [](const void* p) { return p == nullptr || ((uintptr_t)p & 15u) != 0; };
  if (bad16(a->c) || bad16(a->w) || bad16(a->bias) || bad16(a->out))
    return fail(MKX_EINVAL, "mkx_modulations: c, w, bias, out: NULL or not 16-byte aligned");
  hipStream_t stream = (hipStream_t)stream_;
  const dim3 grid((unsigned)((a->N / 16 + 3) / 4)), block(MODP_BLOCK * MODP_KSPLIT);
  switch (a->K / 32) {
    case 8: hipLaunchKernelGGL(modproj_kernel<8>, grid, block, modproj_lds_bytes<8>(), stream, *a); break;
    case 16: hipLaunchKernelGGL(modproj_kernel<16>, grid, block, modproj_lds_bytes<16>(), stream, *a); break;
    case 24: hipLaunchKernelGGL(modproj_kernel<24>, grid, block, modproj_lds_bytes<24>(), stream, *a); break;
    default: hipLaunchKernelGGL(modproj_kernel<32>, grid, block, modproj_lds_bytes<32>(), stream, *a); break;
  }
  HIPCHK(hipGetLastError());
  return MKX_OK;
}

int mkx_modulation_input(const mkx_modin_args* a, void* stream_) {
  if (!a) return fail(MKX_EINVAL, "mkx_modulation_input: args is NULL");
  if (a->N < 1 || a->N > 4096 || a->B < 1 || a->B > (1 << 20))
    return fail(MKX_EINVAL, "mkx_modulation_input: need 1 <= N <= 4096 and B >= 1");
  if (a->H != 256 && a->H != 512 && a->H != 768 && a->H != 1024)
    return fail(MKX_EUNSUPPORTED, "mkx_modulation_input: H must be 256, 512, 768 or 1024");
  if (a->tdim < 32 || a->tdim > 32 * MODIN_MAX_TKB || (a->tdim & 31))
    return fail(MKX_EUNSUPPORTED, "mkx_modulation_input: tdim must be a multiple of 32 in [32, 512]");
  if (a->sc_stride < a->H || (a->sc_stride & 3) || (a->out_stride_k & 3) || (a->out_stride_b & 3) ||
      a->out_stride_k < a->H || (a->B > 1 && a->out_stride_b < (int64_t)a->N * a->out_stride_k))
    return fail(MKX_EINVAL, "mkx_modulation_input: strides must cover a row (and a sample) and be multiples of 4");
  auto bad16 = [](const void* p) { return p == nullptr || ((uintptr_t)p & 15u) != 0; };
  if (bad16(a->t1_w) || bad16(a->t1_b) || bad16(a->t2_w) || bad16(a->t2_b) || bad16(a->state_cond) || bad16(a->out))
    return fail(MKX_EINVAL, "mkx_modulation_input: a pointer is NULL or not 16-byte aligned");
  hipLaunchKernelGGL(modin_kernel, dim3((unsigned)(a->H / 64)), dim3(MODP_BLOCK), 0, (hipStream_t)stream_, *a);
  HIPCHK(hipGetLastError());
  return MKX_OK;
}

int mkx_check(mkx_handle* h, void* stream_) {
  if (!h) return fail(MKX_EINVAL, "null handle");
  HIPCHK(hipStreamSynchronize((hipStream_t)stream_));
  int err = 0;
  HIPCHK(hipMemcpy(&err, &h->bar->err, sizeof(int), hipMemcpyDeviceToHost));
  if (err) {
    HIPCHK(hipMemset(h->bar, 0, sizeof(BarState)));
    HIPCHK(hipMemset(h->flags, 0, sizeof(unsigned long long) * FLAG_KINDS * FLAG_MAX * FLAG_STRIDE));
    h->gen_before = 0;
    if (err & 1) return fail(MKX_ETIMEOUT, "a stage wait exceeded its spin bound; the synchronisation state was reset");
    return fail(MKX_ERANGE, "a GEMM operand exceeded the fp16 range (65504); the launch returned NaN");
  }
  return MKX_OK;
}

int mkx_probe(mkx_probe_args* a, void* stream_) {
  if (!a) return fail(MKX_EINVAL, "mkx_probe: args is NULL");
  a->us_median = a->us_min = 0.0;
  a->timed_out = 0;
  a->xcd_first[0] = a->xcd_first[1] = -1;
  if (a->kind != MKX_PROBE_BARRIER && a->kind != MKX_PROBE_HANDOFF) return fail(MKX_EINVAL, "mkx_probe: unknown kind");
  if (a->n < 2 || a->n > FLAG_MAX || (a->n & 1)) return fail(MKX_EINVAL, "mkx_probe: n must be even and in [2, 2048]");
  if (a->reps < 1 || a->reps > 100) return fail(MKX_EINVAL, "mkx_probe: reps must be in [1, 100]");
  const void* kern = nullptr;
  if (a->kind == MKX_PROBE_BARRIER) {
    kern = reinterpret_cast<const void*>(&barrier_probe_kernel);
  } else if (a->bytes == 4096) {
    kern = reinterpret_cast<const void*>(&handoff_probe_kernel<1>);
  } else if (a->bytes == 24576) {
    kern = reinterpret_cast<const void*>(&handoff_probe_kernel<6>);
  } else if (a->bytes == 73728) {
    kern = reinterpret_cast<const void*>(&handoff_probe_kernel<18>);
  } else {
    return fail(MKX_EINVAL, "mkx_probe: bytes must be 4096, 24576 or 73728");
  }
  hipStream_t stream = (hipStream_t)stream_;
  int dev = 0;
  HIPCHK(hipGetDevice(&dev));
  hipDeviceProp_t prop;
  HIPCHK(hipGetDeviceProperties(&prop, dev));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return fail(MKX_EUNSUPPORTED, "mkx_probe: built for gfx950");
  const int G = prop.multiProcessorCount;
  if (G < 2 || G > 256) return fail(MKX_EUNSUPPORTED, "mkx_probe: 2 to 256 CUs");
  if (a->kind == MKX_PROBE_HANDOFF && (a->fan < 1 || 2 * a->fan > G)) return fail(MKX_EINVAL, "mkx_probe: fan must be in [1, CUs / 2]");
  int per_cu = 0;
  HIPCHK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, NTHREADS, 0));
  if (per_cu < 1) return fail(MKX_ENORESIDENT, "mkx_probe: kernel does not fit one workgroup per CU");
  ProbeParams p{};
  // every allocation is released on every path below
  unsigned* dx = nullptr;
  char* data = nullptr;
  void* sync = nullptr;  // BarState, then the flag table, then out[4]
  const size_t flag_bytes = sizeof(unsigned long long) * FLAG_MAX * FLAG_STRIDE;
  const size_t sync_bytes = sizeof(BarState) + flag_bytes + 4 * sizeof(long long);
  const size_t data_bytes = a->kind == MKX_PROBE_HANDOFF ? (size_t)a->n * a->bytes : 256;
  std::vector<double> us;
  int status = MKX_OK;
  auto run = [&]() -> int {
    HIPCHK(hipMalloc(&dx, sizeof(unsigned) * G));
    HIPCHK(hipMalloc(&data, data_bytes));
    HIPCHK(hipMalloc(&sync, sync_bytes));
    // workgroups per XCD of a G-workgroup grid (the barrier's arrival targets)
    hipLaunchKernelGGL(xcc_probe, dim3(G), dim3(NTHREADS), 0, stream, dx);
    std::vector<unsigned> hx(G);
    HIPCHK(hipMemcpyAsync(hx.data(), dx, sizeof(unsigned) * G, hipMemcpyDeviceToHost, stream));
    HIPCHK(hipStreamSynchronize(stream));
    unsigned cnt[MAX_XCD] = {};
    for (int i = 0; i < G; ++i) {
      if (hx[i] >= MAX_XCD) return fail(MKX_EUNSUPPORTED, "mkx_probe: unexpected XCC id");
      ++cnt[hx[i]];
      p.xmask |= 1u << hx[i];
    }
    for (int x = 0; x < MAX_XCD; ++x) p.nx[x] = cnt[x];
    p.bar = (BarState*)sync;
    p.flags = (unsigned long long*)((char*)sync + sizeof(BarState));
    p.out = (long long*)((char*)sync + sizeof(BarState) + flag_bytes);
    p.data = data;
    p.n = a->n;
    p.fan = a->kind == MKX_PROBE_HANDOFF ? a->fan : 0;
    p.spin_limit = SPIN_LIMIT;
    HIPCHK(hipMemsetAsync(data, 0, data_bytes, stream));
    for (int r = 0; r < a->reps; ++r) {
      HIPCHK(hipMemsetAsync(sync, 0, sync_bytes, stream));
      void* args[] = {&p};
      HIPCHK(hipLaunchCooperativeKernel(kern, dim3(G), dim3(NTHREADS), args, 0, stream));
      long long out[4] = {0, 0, -1, -1};
      int err = 0;
      HIPCHK(hipMemcpyAsync(out, p.out, sizeof(out), hipMemcpyDeviceToHost, stream));
      HIPCHK(hipMemcpyAsync(&err, &p.bar->err, sizeof(int), hipMemcpyDeviceToHost, stream));
      HIPCHK(hipStreamSynchronize(stream));
      if (err) a->timed_out = 1;
      a->xcd_first[0] = (int32_t)out[2];
      a->xcd_first[1] = (int32_t)out[3];
      us.push_back(out[0] * 0.01 / a->n);  // 100 MHz clock
    }
    return MKX_OK;
  };
  status = run();
  if (dx) (void)hipFree(dx);
  if (data) (void)hipFree(data);
  if (sync) (void)hipFree(sync);
  if (status != MKX_OK) return status;
  std::sort(us.begin(), us.end());
  a->us_median = us[us.size() / 2];
  a->us_min = us[0];
  return MKX_OK;
}

int64_t mkx_query(const mkx_handle* h, int32_t key) {
  if (!h) return -1;
  switch (key) {
    case MKX_Q_GRID: return h->G;
    case MKX_Q_BLOCK: return NTHREADS;
    case MKX_Q_BARRIER_COUNT: {
      // workgroup arrivals recorded by the per-XCD counters since the previous query (synchronises)
      if (hipDeviceSynchronize() != hipSuccess) return -1;
      std::vector<unsigned long long> arr(MAX_XCD * 32);
      if (hipMemcpy(arr.data(), h->bar->arrive, sizeof(unsigned long long) * MAX_XCD * 32, hipMemcpyDeviceToHost) != hipSuccess) return -1;
      unsigned long long gen = 0;
      if (hipMemcpy(&gen, &h->bar->gen, sizeof(gen), hipMemcpyDeviceToHost) != hipSuccess) return -1;
      long long total = 0;
      mkx_handle* hm = const_cast<mkx_handle*>(h);
      for (int x = 0; x < MAX_XCD; ++x) total += (long long)(arr[x * 32] - hm->gen_before * h->nx[x]);
      hm->gen_before = gen;
      return total;
    }
    case MKX_Q_ERROR_FLAG: {
      int err = 0;
      if (hipMemcpy(&err, &h->bar->err, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess) return -1;
      return err;
    }
    case MKX_Q_PROFILE_LEN: return h->prof_len;
    case MKX_Q_WEIGHT_BYTES: return h->weight_bytes;
    case MKX_Q_LDS_BYTES: return lds_of(h->d.H, h->d.I);
    case MKX_Q_GEMM_FORM: return h->last_form;
    case MKX_Q_OPERAND_SHIFT: return h->operand_shift;
    default: return -1;
  }
}

int mkx_destroy(mkx_handle* h) {
  if (!h) return MKX_OK;
  (void)hipDeviceSynchronize();
  free_handle(h);
  return MKX_OK;
}

}  // extern "C"
