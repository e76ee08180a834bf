// The persistent megakernel: Euler steps of the flow-matching action expert in one launch.
//
// Schedule (the stage math of expert_megakernel, src/mk_expert.py:302-426): an in-projection tail, then for
// each step and layer seven stages (QKV, self-attention, out-proj + gated residual, cross-attention with its
// own query projection, out-proj + gated residual, gate/up, down + gated residual) and a step tail:
// 1 + n_steps * (7 L + 1) stage boundaries (the reference runs the cross-attention query projection as a
// stage of its own and a grid barrier after every stage: 8 L + 1). Only the first boundary is a grid
// barrier; afterwards every task publishes a ready epoch and every task waits for exactly the producer
// tasks whose output it reads.
//
// Code layout: the kernel is one flat loop over stages, and each kind of stage (GEMM, self-attention,
// cross-attention, tail) is a single inlined body driven by a runtime descriptor. The whole loop stays
// resident in the instruction cache; a stage never waits on instruction fetch. A workgroup passes over the
// stages in which it has no task.
//
// Work decomposition for 256 CUs: every linear layer is cut into tasks of 16-column output tiles (or NTW of
// them, for the out-projections and the down projection) over a group of row tiles, K = H per task (the down
// projection is split over K into I/H tasks per tile group whose fp32 partials are summed in a fixed order
// by reducer tasks). The host places each stage's tasks on a range of workgroups (Params::pl), where the
// grid allows on workgroups idle in the stage before. Between finishing its
// work in one stage and waiting for the producers of its next task, a workgroup DMAs into LDS everything
// constant that task needs: the packed weight tile (or, for attention, the cached K/V). After the wait only
// the activations are loaded, straight into VGPRs.
//
// Activation frames are fragment-major: a buffer of C columns and NRP rows is cut into 2 KB blocks
// (32-column block kb, 16-row tile rt) at ((kb * RT + rt) * 2) KB, lane-major inside (lane = row % 16 +
// 16 * (8-column group)). "fp32" buffers hold columns 0-3 of each 8-column group in the first 1 KB and 4-7
// in the second; GEMM operand buffers hold an MFMA operand fragment directly, 8 fp16 values per lane in the
// first 1 KB, so that a wave loads one fragment (16 rows x 32 columns) with one contiguous 1 KB load and
// feeds it to the MFMA unchanged; the attention operands (q, k, V^T) are split: 8 bf16 high parts per lane
// in the first 1 KB and the 8 bf16 residuals in the second.
//
// Numerics: the linear layers run on fp16 MFMAs with fp32 accumulation. Weights are fp16 (bf16 weights are
// packed as fp16 at handle creation, exactly within the fp16 range; fp8 e4m3 weights are decoded to fp16, also
// exactly). Every GEMM operand is stored once, by its producer, as fp16 (round to nearest even): attention
// writes its output in fp16; the residual stages write h (fp32, for the next residual add), y = h * (1 + scale)
// of the next AdaRMS (fp16) and per-tile partial sums of squares of h; the AdaRMS GEMM then computes
// rstd(h) * (y W^T) + shift W^T (src/mk_expert.py:93-122 rearranged), with shift W^T taken by the MFMA as
// one extra row tile of per-sample fp16 shift rows. The residual stream, softmax and everything between
// stages stay fp32, and attention multiplies its operands as split bf16 (hi + lo, ~2^-17 relative). The QKV
// projection is computed per (head, d-quarter pair) so its epilogue holds d and d + 32 of a row: it applies
// the q/k norm weight and RoPE and writes the attention operands split (V directly in the transposed P V
// layout), leaving only the per-row RMS factor, which attention folds into the scores. The cross-attention
// query is projected inside the cross-attention stage, where a workgroup holds whole head rows. fp16 carries
// 3 more significant bits than bf16: the kernel tracks the fp32 eager expert about ten times closer than a
// bf16-activation kernel (which sits at ~1.5e-3 mean |delta| at full depth, most of the 2e-3 parity budget),
// and loads half the operand bytes of the split-bf16 operands it replaces. An operand beyond the fp16 range
// (65504) sets the launch's range error: the launch returns NaN and mkx_check reports it.
#pragma once
#include "mkx_device.h"

namespace mkx {

struct Params {
  // packed weights; per-layer strides in elements
  const char* wqkv; const char* wo; const char* wqca; const char* woca; const char* wgu; const char* wd;
  long long s_qkv, s_o, s_gu, s_d;  // bytes per layer
  // fp8 weights: per-output-channel scales, [L][3H] (q;k;v), [L][H], [L][H], [L][H], [L][I] (gate), [L][I]
  // (up), [L][H] (down); null for bf16 weights
  const float* sc_qkv; const float* sc_o; const float* sc_qca; const float* sc_oca; const float* sc_g; const float* sc_u; const float* sc_d;
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
  // V^T copies of the memory / cross-attention V caches, made once per launch:
  // [L][B][NH][PMP/32 or SPP/32 key blocks][4 d-slices][512 bf16]
  bf16_t* memvt; bf16_t* cavt; int SPP;
  // AdaRMS shift slices as fp16, made once per launch: [n_steps][L][3: self-attn, cross-attn, MLP] blocks
  // of B * H * 4 bytes; sample b's 8-column group (k-block kb, group j) is 16 bytes of fp16 at
  // ((b * H/32 + kb) * 4 + j) * 32 (the next 16 bytes are unused)
  char* shs;
  int n_steps, action_dim, T, R, B, PM, SP, L, Mq, Mqp, NR, NRP, A, act;
  float eps, qk_eps, sm_scale;
  // scratch
  char* frames; long long frame_bytes;   // [n_steps * L] layer frames
  char* steps; long long step_bytes;     // [n_steps] step areas: h0 (fp32, fragment-major) + x (fp32)
  BarState* bar; unsigned nx[MAX_XCD]; unsigned xmask;
  unsigned long long* flags;             // [FLAG_KINDS][FLAG_MAX][FLAG_STRIDE] ready epochs
  long long* prof; int profile;
  unsigned spin_limit;
  // Task placement (computed on the host for the launch's shape): task t of placement kind k runs on
  // workgroup (pl[k] + t) % G, then t + G, ...; the host places consecutive stages on disjoint workgroups
  // where the grid allows, so a workgroup is idle in the stage before each of its tasks.
  int pl[10];
  int rgs_qkv, rgs_o, rgs_cao;  // row groups of the QKV, out-projection and CA out-projection stages
  int nt_o, nt_cao, nt_down;    // 16-column tiles per out-projection / CA out-projection / down task (1 or NTW)
  int lds_red, lds_mods;        // GEMM stages' LDS map: cross-wave reduction buffer, staged modulation slices
  int tpr, nred;                // down-projection reducers: 16-column tiles per reducer, reducers (HT / tpr)
  // AdaRMS operand scaling by yinv = 2^-E (the instantiations with Shape::YS; E = 0 otherwise), so that a
  // residual stream beyond the fp16 range of y can be run: the producers of h store y = h (1 + scale) yinv and
  // the sums of squares of h yinv, and eps is eps_final yinv^2, so the AdaRMS consumers' rsqrt(ss / H + eps)
  // is exactly 2^E rstd(h) (powers of two scale exactly) and rstd (y W^T) comes out unchanged; eps_final, the
  // model's eps, serves the step tail's AdaRMS, which sums the squares of h itself
  float yinv, eps_final;
  // down-projection reducers of the row-wise form: row groups per tile (the QKV stage's row groups, so that a
  // QKV task waits for its own row group's reducers); reducer r = tile r % HT of row group r / HT; 1 in the
  // form with passes
  int nrg;
  // row-wise form: cross-attention tasks of two query tiles (ca_stage_pairs; the self-attention ones are the
  // Shape::PAIRS instantiations')
  int ca_grp;
};

// placement kinds (Params::pl)
enum { PL_QKV = 0, PL_SA, PL_O, PL_CA, PL_CAO, PL_GU, PL_DOWN, PL_RED, PL_TIN, PL_TOUT, PL_KINDS };

// the kernel reads its parameters in place from the kernarg segment (constant address space), so the
// per-layer pointer tables are indexed with scalar loads and never copied to scratch
typedef const __attribute__((address_space(4))) Params CP;

__host__ __device__ constexpr int ceil_to(int a, int m) { return (a + m - 1) / m * m; }

template <int H_, int I_, bool W8_ = false, bool RW_ = false, bool YS_ = false, bool PR_ = false, bool LS_ = false>
struct Shape {
  // YS: AdaRMS operands scaled by Params::yinv (the launches with an operand shift)
  static constexpr bool YS = YS_;
  static constexpr int H = H_, I = I_, NH = H / HD, NKB = H / 32, HT = H / 16, IT = I / 16, SK = I / H;
  // RW: the launch form for many row tiles (row-wise GEMM stages, step-tail output tasks over row chunks)
  static constexpr bool RW = RW_;
  // Row-wise attention variants (RW_ATTN): attention tasks beyond the grid run as second query tiles of a
  // sample-head (attn_task), and cross-attention DMAs its source K/V after its ready-epoch poll instead of
  // before it. Compiled into the row-wise form with fp16-packed weights only: the fp8 row-wise instantiation
  // measured slower with them, also for launches that never run the pairs (workload D 7.65 -> 7.86 ms and
  // D-b4 12.79 -> 13.00 ms with the pairs; 7.65 -> 7.69 and 12.77 -> 12.86 ms with the late K/V DMA).
  static constexpr bool RW_ATTN = RW_ && !W8_;
  // CA_LATE: cross-attention DMAs its source K/V after its ready-epoch poll and query rows: the fp16 row-wise
  // instantiations and the two-tile ones (not the other fp8 row-wise ones, whose launches, workload D, measured
  // 7.59 -> 7.74 ms with it)
  static constexpr bool CA_LATE = RW_ && (!W8_ || PR_);
  // CA_REG: the other fp8 row-wise instantiations: one-tile cross-attention over at most three 128-row chunks
  // loads each wave's source K/V blocks into registers after its poll (ca_stage) instead of the LDS ring DMA'd
  // ahead of it
  static constexpr bool CA_REG = RW_ && !CA_LATE;
  // PAIRS: the fp8-weight row-wise instantiations for launches whose attention tasks run two query tiles each
  // (chosen by the host where the one-tile tasks outnumber the workgroups and the two-tile tasks do not):
  // self-attention by sa_stage_pairs only. Separate instantiations, so that the others keep their code (and
  // register allocation) unchanged: compiled into them, the two-tile path made the kernels slower for every
  // launch (workload D 7.59 -> 7.90 ms without taking it).
  static constexpr bool PAIRS = RW_ && PR_;
  // SA_REG: the same instantiations', the two-tile ones' and the long-source ones' self-attention loads each
  // wave's own-key block (K, V^T, hi and lo parts) and its keys' RMS factors into registers (sa_stage,
  // sa_stage_pairs) instead of DMAing every own key into LDS after the poll, except in launches that also
  // store the register rows' K/V (they read them from LDS)
  static constexpr bool SA_REG = CA_REG || PAIRS || (LS_ && !RW_);
  // LONG: the instantiations of the form with passes for sources longer than the three-chunk LDS ring (the
  // host picks them for launches whose source exceeds 384 rows): cross-attention streams the chunks beyond
  // the third into registers (ca_stage). Separate instantiations, so that the others keep their code.
  static constexpr bool LONG = LS_ && !RW_;
  // packed weight chunks (16 output columns x 32 K values, one MFMA operand fragment per lane): fp16 (packed
  // from bf16), or fp8 e4m3 decoded to fp16 fragments when read (weight-only quantisation)
  static constexpr bool W8 = W8_;
  static constexpr int CH = W8 ? 512 : 1024;  // bytes per chunk
  static constexpr int KPW = NKB / NWAVES;  // 32-wide k-blocks per wave
  static constexpr int WBUF = 0, WBUF_BYTES = 64 * 1024;
  static constexpr int ABUF = WBUF_BYTES, ABUF_BYTES = 88 * 1024;
  static constexpr int RED = ABUF, RED_BYTES = 32 * 1024;              // GEMM cross-wave reduction
  static constexpr int MODS = ABUF + RED_BYTES, MODS_BYTES = 56 * 1024;  // per-sample modulation slices
  static constexpr int SMALL = ABUF + ABUF_BYTES, SMALL_BYTES = 4 * 1024;
  static constexpr int LDS = SMALL + SMALL_BYTES;
  static constexpr int RB_FIT = 144 / (KPW * 8);  // row tiles per GEMM pass held in VGPRs (hi + lo)
  // Fixed-role tasks at the end of a layer and of a step: NIN step-tail in-projection tasks (two 16-column
  // tiles each) and Params::nred reducers, each of which sums the down projection's split-K partials of
  // Params::tpr output tiles (at most NTW; a reducer's loads, 5 KB per tile and row tile, are its critical
  // path). The host places them (Params::pl).
  static constexpr int NIN = HT / 2;
  static constexpr int RBMAX = RB_FIT > 3 ? 3 : RB_FIT;
  // Wide tasks of the gated-residual and down-projection GEMMs: NTW = HT / 16 16-column tiles per task where
  // their weights fit 72 KB of LDS, else single tiles. A wide pass holds one row tile (residual stages) or up
  // to RBMAX (down-projection splits); its accumulators are not split into hi / lo products (NTW x row tiles
  // independent accumulators already keep consecutive MFMAs apart).
  static constexpr int WT = HT / 16;
  static constexpr int NTW = (WT > 1 && WT <= 4 && WT * NKB * CH <= 72 * 1024) ? WT : 1;
  // GEMM-stage LDS map, narrow (nt <= 2) and wide tasks: weight tiles from 0, then the cross-wave reduction
  // buffer ([wave][row tile][tile][64 lanes] x 16 bytes), then the staged modulation slices
  static constexpr int W_NARROW = 2 * NKB * CH, RED_NARROW = NWAVES * (RBMAX + 1) * 2 * 1024;
  static constexpr int W_WIDE = NTW * NKB * CH, RED_WIDE = NWAVES * RBMAX * NTW * 1024;
  static_assert(H % 256 == 0 && I % H == 0, "H must be a multiple of 256 and I a multiple of H");
  // waits on at most 64 ready epochs poll with one load (flag_wait<1>): the QKV, down-split, reducer,
  // self-attention, cross-attention and step-tail waits
  static_assert(HT <= 64 && 5 * SK <= 64, "waits polled with one load cover at most 64 flags");
  static_assert(KPW >= 1 && RBMAX >= 1, "tile does not fit registers");
  static_assert(NKB * CH * 2 <= WBUF_BYTES, "gate/up weight tile pair must fit the weight buffer");
  static_assert(NWAVES * (RBMAX + 1) * 2 * 1024 <= RED_BYTES, "cross-wave reduction must fit LDS");
  static_assert(LDS <= 160 * 1024 - 256, "LDS budget");
  // frame layout (bytes), buffers of NRP rows; HB = NRP * H * 4:
  //   qs, ks: split q / k (roped, not normed) | vt: split V^T blocks per (sample, head) (2 HB) | ysa f16 |
  //   h2 fp32 | y2 f16 | yca f16 | h3 fp32 | y3 f16 | g f16 (I columns) | hl fp32 | yl f16 |
  //   (f16: fp16 GEMM operands in the first 1 KB of each 2 KB block)
  //   part fp32 [SK][H] | ssqk [2][NH][2][NRP] | ss2, ss3, ssl [RT][HT / 2][16][2]
  // (sums of squares of h per 16-column tile t and row: one 128-byte line per (16-row tile, tile pair), so
  // that a line has at most two writers: many producers writing 4-byte pieces of one line at once take
  // twice as long to be acknowledged)
  __host__ __device__ static long long hb(int nrp) { return (long long)nrp * H * 4; }
  __host__ __device__ static long long qs_off(int) { return 0; }
  __host__ __device__ static long long ks_off(int nrp) { return hb(nrp); }
  __host__ __device__ static long long vtb_off(int nrp) { return 2 * hb(nrp); }
  __host__ __device__ static long long ysa_off(int nrp) { return 4 * hb(nrp); }
  __host__ __device__ static long long h2_off(int nrp) { return 5 * hb(nrp); }
  __host__ __device__ static long long y2_off(int nrp) { return 6 * hb(nrp); }
  __host__ __device__ static long long yca_off(int nrp) { return 7 * hb(nrp); }
  __host__ __device__ static long long h3_off(int nrp) { return 8 * hb(nrp); }
  __host__ __device__ static long long y3_off(int nrp) { return 9 * hb(nrp); }
  __host__ __device__ static long long g_off(int nrp) { return 10 * hb(nrp); }
  __host__ __device__ static long long hl_off(int nrp) { return (10 + SK) * hb(nrp); }
  __host__ __device__ static long long yl_off(int nrp) { return (11 + SK) * hb(nrp); }
  __host__ __device__ static long long part_off(int nrp) { return (12 + SK) * hb(nrp); }
  __host__ __device__ static long long ssqk_off(int nrp) { return (12 + 2 * SK) * hb(nrp); }
  __host__ __device__ static long long ss2_off(int nrp) { return ssqk_off(nrp) + 4LL * NH * nrp * 4; }
  __host__ __device__ static long long ss_bytes(int nrp) { return (long long)HT * nrp * 4; }
  __host__ __device__ static long long ss3_off(int nrp) { return ss2_off(nrp) + ss_bytes(nrp); }
  __host__ __device__ static long long ssl_off(int nrp) { return ss3_off(nrp) + ss_bytes(nrp); }
  __host__ __device__ static long long frame_bytes(int nrp) { return ssl_off(nrp) + ss_bytes(nrp); }
  // step area: h0 fp32 | y0 f16 | ss0 [RT][HT / 2][16][2] | x [B*T][A] fp32
  __host__ __device__ static long long step_x_off(int nrp) { return 2 * hb(nrp) + ss_bytes(nrp); }
};

// byte offset of the 4-float piece (row r, columns c .. c+3; c % 4 == 0) of a fragment-major fp32 buffer
__host__ __device__ __forceinline__ uint32_t fpiece(int r, int c, int RT) {
  return (uint32_t)((((c >> 5) * RT + (r >> 4)) * 2 + ((c >> 2) & 1)) * 1024 + ((r & 15) + 16 * ((c & 31) >> 3)) * 16);
}
// byte offset of the 4 fp16 values (row r, columns c .. c+3) of a GEMM operand buffer, or of the 4 high parts
// of a split buffer (the residuals are 1 KB later)
__host__ __device__ __forceinline__ uint32_t spiece(int r, int c, int RT) {
  return (uint32_t)(((c >> 5) * RT + (r >> 4)) * 2048 + ((r & 15) + 16 * ((c & 31) >> 3)) * 16 + (c & 4) * 2);
}

enum Stage { ST_QKV = 0, ST_SA, ST_O, ST_CA, ST_CAO, ST_GU, ST_DOWN, ST_TAIL };
constexpr int STAGES_PER_LAYER = 7;
enum { K_QKV = 0, K_RES = 1, K_GU = 2, K_SPLIT = 3 };

// Optional per-workgroup phase trace (diagnostic builds with MKX_TRACE): clock of phase `slot` of the
// interval after barrier ep, at prof[TRACE_BASE + (ep * G + wg) * TRACE_SLOTS + slot].
constexpr long long TRACE_BASE = 8192, TRACE_SLOTS = 16;
#ifdef MKX_TRACE
#define MKX_TR(c, slot)                                                                                          \
  do {                                                                                                           \
    if ((c).tid == 0 && (c).p.profile) (c).p.prof[TRACE_BASE + ((long long)(c).ep * (c).G + (c).wg) * TRACE_SLOTS + (slot)] = clock100(); \
  } while (0)
#define MKX_TRW(c, slot)                                                                                         \
  do {                                                                                                           \
    if ((c).tid == 64 && (c).p.profile) (c).p.prof[TRACE_BASE + ((long long)(c).ep * (c).G + (c).wg) * TRACE_SLOTS + (slot)] = clock100(); \
  } while (0)
#else
#define MKX_TR(c, slot) \
  do {                  \
  } while (0)
#define MKX_TRW(c, slot) \
  do {                   \
  } while (0)
#endif

template <class S>
struct Ctx {
  CP& p;
  char* smem;
  int wg, G, wave, lane, tid, RT;
  int dw, dn;  // DMA issue: this wave's index among the dn issuing waves (all 4, or waves 1-3 in a barrier)
  unsigned ep = 0;  // barriers passed so far in this launch
  float dt;
  __device__ Ctx(CP& p_, char* smem_) : p(p_), smem(smem_) {
    wg = blockIdx.x; G = gridDim.x; tid = threadIdx.x; lane = tid & 63;
    wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, so offsets built from it stay scalar
    RT = p.NRP >> 4;
    dw = wave;
    dn = NWAVES;
  }
  __device__ char* frame(int s, int l) const { return p.frames + (long long)(s * p.L + l) * p.frame_bytes; }
  __device__ char* step(int s) const { return p.steps + (long long)s * p.step_bytes; }
  __device__ float* h0(int s) const { return (float*)step(s); }
  __device__ float* y0(int s) const { return (float*)(step(s) + S::hb(p.NRP)); }
  __device__ float* ss0(int s) const { return (float*)(step(s) + 2 * S::hb(p.NRP)); }
  __device__ float* xstep(int s) const { return (float*)(step(s) + S::step_x_off(p.NRP)); }
  // layer inputs: the residual stream h (fp32), its AdaRMS operand y (split) and sums of squares
  __device__ const float* h_in(int s, int l) const {
    return l == 0 ? h0(s) : (const float*)(frame(s, l - 1) + S::hl_off(p.NRP));
  }
  __device__ const float* y_in(int s, int l) const {
    return l == 0 ? y0(s) : (const float*)(frame(s, l - 1) + S::yl_off(p.NRP));
  }
  __device__ const float* ss_in(int s, int l) const {
    return l == 0 ? ss0(s) : (const float*)(frame(s, l - 1) + S::ssl_off(p.NRP));
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

__device__ __forceinline__ u32x4 bload(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u32x2 bload8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
}
// sum of N pairs of floats, pairwise
template <int N>
__device__ __forceinline__ float ss_pairs_sum(const u32x2 (&v)[N]) {
  float p[N];
#pragma unroll
  for (int i = 0; i < N; ++i) p[i] = __uint_as_float(v[i][0]) + __uint_as_float(v[i][1]);
#pragma unroll
  for (int w = 1; w < N; w *= 2)
#pragma unroll
    for (int i = 0; i + w < N; i += 2 * w) p[i] += p[i + w];
  return p[0];
}
__device__ __forceinline__ f32x4 as_f4(u32x4 v) { return __builtin_bit_cast(f32x4, v); }
__device__ __forceinline__ u32x4 as_u4(f32x4 v) { return __builtin_bit_cast(u32x4, v); }

// nbytes (a multiple of 1 KB) of packed weight chunks into LDS
template <class S>
__device__ __forceinline__ void dma_w(Ctx<S>& c, char* dst, const char* src, int nbytes) {
  for (int k = c.dw; k < nbytes / 1024; k += c.dn) dma16(src + (long long)k * 1024 + c.lane * 16, dst + k * 1024);
}
// nfloats (a multiple of 256) contiguous fp32 values into LDS
template <class S>
__device__ __forceinline__ void dma_f32(Ctx<S>& c, char* dst, const float* src, int nfloats) {
  for (int k = c.dw; k < nfloats / 256; k += c.dn) dma16(src + (long long)k * 256 + c.lane * 4, dst + k * 1024);
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
// two fp32 -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t cvt_pk(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}
// split 8 fp32 values into bf16 high parts and bf16 residuals
__device__ __forceinline__ void split8(const float* f, bf16x8& hi, bf16x8& lo) {
  u32x4 h, l;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h[j] = cvt_pk(f[2 * j], f[2 * j + 1]);
    l[j] = cvt_pk(f[2 * j] - __uint_as_float(h[j] << 16), f[2 * j + 1] - __uint_as_float(h[j] & 0xffff0000u));
  }
  hi = __builtin_bit_cast(bf16x8, h);
  lo = __builtin_bit_cast(bf16x8, l);
}
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
// two fp32 -> packed fp16 pair, round to nearest even (v_cvt_pk_f16_f32)
__device__ __forceinline__ uint32_t cvt_pk_h(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, f16x2_t));
}
// 8 e4m3 values (OCP fp8, as the weights are quantised) -> 8 fp16, exactly (v_cvt_scalef32_pk_f16_fp8 with
// scale 1 decodes OCP e4m3 on gfx950; every e4m3 value is an fp16 value)
__device__ __forceinline__ f16x8 fp8x8_to_f16(uint2 v) {
  u32x4 r;
  r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)v.x, 1.0f, false));
  r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)v.x, 1.0f, true));
  r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)v.y, 1.0f, false));
  r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)v.y, 1.0f, true));
  return __builtin_bit_cast(f16x8, r);
}
// this lane's fp16 weight operand fragment of a packed chunk in LDS (chunk = its first byte): bf16 weights are
// packed as fp16 at handle creation, fp8 weights are decoded here
template <class S>
__device__ __forceinline__ f16x8 wfrag_lds(const char* chunk, int lane) {
  if constexpr (S::W8) return fp8x8_to_f16(*reinterpret_cast<const uint2*>(chunk + lane * 8));
  else return *reinterpret_cast<const f16x8*>(chunk + lane * 16);
}
// the same from global memory
template <class S>
__device__ __forceinline__ f16x8 wfrag_glb(const char* chunk, int lane) {
  if constexpr (S::W8) return fp8x8_to_f16(*reinterpret_cast<const uint2*>(chunk + lane * 8));
  else return __builtin_bit_cast(f16x8, ld16(chunk + lane * 16));
}
__device__ __forceinline__ void unpack8(u32x4 v, float* f) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f[2 * j] = __uint_as_float(v[j] << 16);
    f[2 * j + 1] = __uint_as_float(v[j] & 0xffff0000u);
  }
}
// 4 fp32 values -> hi and lo bf16 pairs at off and off + 1024 of a split buffer, written through
__device__ __forceinline__ void st_split4(void* base, uint32_t off, f32x4 v) {
  u32x2 h, l;
  h[0] = cvt_pk(v[0], v[1]);
  h[1] = cvt_pk(v[2], v[3]);
  l[0] = cvt_pk(v[0] - __uint_as_float(h[0] << 16), v[1] - __uint_as_float(h[0] & 0xffff0000u));
  l[1] = cvt_pk(v[2] - __uint_as_float(h[1] << 16), v[3] - __uint_as_float(h[1] & 0xffff0000u));
  st_sc1_b64(base, off, h);
  st_sc1_b64(base, off + 1024, l);
}
// Largest finite fp16 value. GEMM operands are stored as fp16; a value beyond it cannot be represented.
constexpr float F16_MAX = 65504.0f;
// 4 fp32 values -> 4 fp16 (round to nearest even) at off of a GEMM operand buffer (the first 1 KB of each
// 2 KB block holds an MFMA fragment), written through; returns whether a value exceeds the fp16 range
__device__ __forceinline__ bool st_h4(void* base, uint32_t off, f32x4 v) {
  u32x2 h;
  h[0] = cvt_pk_h(v[0], v[1]);
  h[1] = cvt_pk_h(v[2], v[3]);
  st_sc1_b64(base, off, h);
  return fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))) > F16_MAX;
}
// records that a GEMM operand of this launch exceeded the fp16 range (error bit 2): the launch returns NaN and
// mkx_check reports MKX_ERANGE
__device__ __forceinline__ void range_error(BarState* bs) {
  __hip_atomic_fetch_or(&bs->err, ERR_RANGE, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u32x4 lds16(const char* p) { return *reinterpret_cast<const u32x4*>(p); }
// Marks LDS values as needed together: the reads that produced them are issued back to back and waited for
// once, instead of the compiler reusing one register and waiting after every read.
template <class T, int N>
__device__ __forceinline__ void lds_batch(T (&v)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(v[i]));
}
__device__ __forceinline__ void sts16(char* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ bf16x8 ldsfrag(const char* p) { return *reinterpret_cast<const bf16x8*>(p); }
__device__ __forceinline__ f16x8 ldsfrag_h(const char* p) { return *reinterpret_cast<const f16x8*>(p); }
__device__ __forceinline__ f32x4 ldf4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }

// SiLU, or GELU with the tanh approximation (tanh u = 1 - 2 / (exp(2u) + 1)); hardware exp and reciprocal
__device__ __forceinline__ float act_fn(float x, int gelu) {
  if (gelu) {
    const float k0 = 0.7978845608028654f, k1 = 0.044715f;
    const float u = k0 * (x + k1 * x * x * x);
    const float th = 1.0f - 2.0f * __builtin_amdgcn_rcpf(__expf(2.0f * u) + 1.0f);
    return 0.5f * x * (1.0f + th);
  }
  return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

// staged per-sample modulation slices: gated-residual tasks hold [gate | next AdaRMS scale] (2H) at the GEMM
// map's offset, the step tail the final [scale | shift] (2H) at its own
template <class S>
__device__ __forceinline__ const float* mods_lds(Ctx<S>& c, int b, int width) {
  return (const float*)(c.smem + c.p.lds_mods) + (long long)b * width;
}
template <class S>
__device__ __forceinline__ const float* tail_mods_lds(Ctx<S>& c, int b) {
  return (const float*)(c.smem + S::MODS) + (long long)b * 2 * S::H;
}

// this workgroup's first task (then every G-th) of placement kind k
template <class S>
__device__ __forceinline__ int task_first(Ctx<S>& c, int k) {
  const int t = c.wg - c.p.pl[k];
  return t < 0 ? t + c.G : t;
}

// row group (of rgs over RT row tiles, group g covering [g RT / rgs, (g + 1) RT / rgs)) holding row tile rt
__device__ __forceinline__ int row_group_of(int rt, int RT, int rgs) { return ((rt + 1) * rgs - 1) / RT; }

// ------------------------------------------------------------------------------------------------
// Stage descriptor: what one stage computes, where its operands live, and what to prefetch for it.

struct Desc {
  int st, s, l;
  bool first, last;
  // GEMM stages
  const char* w; long long wstride;    // packed weight chunks; tile t at w + t * wstride bytes (not split)
  const float* sc; const float* sc2;   // fp8 weights: the layer's output-channel scales (gate/up: sc2 = up)
  const float* a;                      // fp16 operand frame
  float* out; const float* res; float* part;
  float* yout; float* ssout;           // residual stages: y = h * (1 + next scale) (split), sums of squares
  const float* ssin;                   // AdaRMS stages: the operand's sums of squares [RT][HT / 2][16][2]
  int ntask, tiles, kind, nt;          // nt: 16-column tiles per task (QKV, gate/up: a pair; wide tasks: NTW)
  int rgs;                             // row groups: task t = tile t % tiles over row-tile group t / tiles
  int pk;                              // placement kind (Params::pl)
  const char* shs;                     // AdaRMS stages: the fp16 shift fragments of this step and layer
  // staged modulation slices (H floats each, per sample): AdaRMS stages: shift; residual stages: gate, then
  // the scale of the next AdaRMS
  int mod_off, mod_off2;
};

// Position of stage g of a launch: step s, layer l and kind k (ST_QKV .. ST_DOWN), or l == L for the step
// tail; the launch's first stage (g = 0) is the tail of step -1. Stepped forward by increments only.
struct StagePos {
  int g, s, l, k;
};
__device__ __forceinline__ void advance(StagePos& q, int L) {
  ++q.g;
  if (q.l == L) {
    q.l = 0;
    q.k = 0;
    ++q.s;
  } else if (++q.k == STAGES_PER_LAYER) {
    q.k = 0;
    ++q.l;
  }
}

template <class S>
__device__ __forceinline__ Desc describe(Ctx<S>& c, const StagePos& q) {
  CP& p = c.p;
  Desc d;
  d.first = q.g == 0;
  d.last = false;
  d.w = nullptr; d.wstride = 0; d.a = nullptr; d.out = nullptr; d.res = nullptr; d.part = nullptr;
  d.sc = nullptr; d.sc2 = nullptr;
  d.yout = nullptr; d.ssout = nullptr; d.ssin = nullptr; d.shs = nullptr;
  d.ntask = 0; d.tiles = 1; d.kind = K_QKV; d.nt = 1; d.mod_off = 0; d.mod_off2 = 0; d.rgs = 1; d.pk = PL_TIN;
  if (q.g == 0) { d.st = ST_TAIL; d.s = 0; d.l = 0; return d; }
  d.s = q.s;
  if (q.l == p.L) {
    d.st = ST_TAIL; d.l = p.L - 1; d.last = d.s + 1 == p.n_steps;
    return d;
  }
  d.l = q.l;
  d.st = q.k;
  const int NRP = p.NRP, l = d.l;
  char* fr = c.frame(d.s, l);
  // AdaRMS slices of a layer's mods row (src/mk_expert.py:302-426): [scale | shift | gate] for self-attention,
  // cross-attention and the MLP; the next layer's (or the final) AdaRMS scale follows at 9 (l + 1) H
  const int m_sa = 9 * l * S::H, m_ca = m_sa + 3 * S::H, m_mlp = m_sa + 6 * S::H, m_next = m_sa + 9 * S::H;
  d.wstride = (long long)S::NKB * S::CH;
  const char* shs = p.shs + (long long)(d.s * p.L + l) * 3 * p.B * S::H * 4;
  switch (d.st) {
    case ST_QKV:  // task ((kind * NH + head) * 2 + j): columns 16 j + [0, 16) and 16 j + 32 + [0, 16) of the head
      d.w = p.wqkv + l * p.s_qkv; d.wstride = 2LL * S::NKB * S::CH; d.a = c.y_in(d.s, l); d.ssin = c.ss_in(d.s, l);
      if (S::W8) d.sc = p.sc_qkv + (long long)l * 3 * S::H;
      d.out = (float*)(fr + S::qs_off(NRP)); d.yout = (float*)(fr + S::ks_off(NRP)); d.part = (float*)(fr + S::vtb_off(NRP));
      d.ssout = (float*)(fr + S::ssqk_off(NRP)); d.tiles = 6 * S::NH; d.nt = 2; d.shs = shs;
      d.rgs = p.rgs_qkv; d.pk = PL_QKV;
      break;
    case ST_O:
      d.w = p.wo + l * p.s_o; d.a = (const float*)(fr + S::ysa_off(NRP)); d.out = (float*)(fr + S::h2_off(NRP));
      if (S::W8) d.sc = p.sc_o + (long long)l * S::H;
      d.yout = (float*)(fr + S::y2_off(NRP)); d.ssout = (float*)(fr + S::ss2_off(NRP));
      d.res = c.h_in(d.s, l); d.kind = K_RES; d.mod_off = m_sa + 2 * S::H; d.mod_off2 = m_ca;
      d.nt = p.nt_o; d.tiles = S::HT / d.nt; d.wstride = (long long)d.nt * S::NKB * S::CH; d.rgs = p.rgs_o; d.pk = PL_O;
      break;
    case ST_CAO:
      d.w = p.woca + l * p.s_o; d.a = (const float*)(fr + S::yca_off(NRP)); d.out = (float*)(fr + S::h3_off(NRP));
      if (S::W8) d.sc = p.sc_oca + (long long)l * S::H;
      d.yout = (float*)(fr + S::y3_off(NRP)); d.ssout = (float*)(fr + S::ss3_off(NRP));
      d.res = (const float*)(fr + S::h2_off(NRP)); d.kind = K_RES;
      d.mod_off = m_ca + 2 * S::H; d.mod_off2 = m_mlp;
      d.nt = p.nt_cao; d.tiles = S::HT / d.nt; d.wstride = (long long)d.nt * S::NKB * S::CH; d.rgs = p.rgs_cao; d.pk = PL_CAO;
      break;
    case ST_GU:
      d.w = p.wgu + l * p.s_gu; d.wstride = 2LL * S::NKB * S::CH; d.a = (const float*)(fr + S::y3_off(NRP));
      if (S::W8) { d.sc = p.sc_g + (long long)l * S::I; d.sc2 = p.sc_u + (long long)l * S::I; }
      d.ssin = (const float*)(fr + S::ss3_off(NRP)); d.out = (float*)(fr + S::g_off(NRP));
      d.tiles = S::IT; d.kind = K_GU; d.nt = 2; d.shs = shs + 2 * p.B * S::H * 4; d.pk = PL_GU;
      break;
    case ST_DOWN:
      d.w = p.wd + l * p.s_d; d.a = (const float*)(fr + S::g_off(NRP)); d.out = (float*)(fr + S::hl_off(NRP));
      if (S::W8) d.sc = p.sc_d + (long long)l * S::H;
      d.yout = (float*)(fr + S::yl_off(NRP)); d.ssout = (float*)(fr + S::ssl_off(NRP));
      d.res = (const float*)(fr + S::h3_off(NRP)); d.part = (float*)(fr + S::part_off(NRP));
      d.nt = p.nt_down; d.tiles = S::HT / d.nt; d.rgs = S::SK; d.kind = K_SPLIT; d.pk = PL_DOWN;
      d.mod_off = m_mlp + 2 * S::H; d.mod_off2 = m_next;
      break;
    case ST_SA:
      d.pk = PL_SA;
      break;
    case ST_CA:
      d.pk = PL_CA;
      break;
    default:
      break;
  }
  d.ntask = d.tiles * d.rgs;  // K_SPLIT: the K splits take the place of row groups
  return d;
}

// DMA of task t's weight tiles into LDS at dst: nt consecutive 16-column tiles ([tile][k-block] chunks; the
// down projection's splits are packed [tile][split][k-block], so its tiles are nt runs)
template <class S>
__device__ __forceinline__ void dma_task_w(Ctx<S>& c, const Desc& d, int t, char* dst) {
  const int tile = t % d.tiles, split = t / d.tiles;
  if (d.kind == K_SPLIT) {
    for (int j = 0; j < d.nt; ++j)
      dma_w(c, dst + j * S::NKB * S::CH, d.w + ((long long)(tile * d.nt + j) * S::SK + split) * S::NKB * S::CH,
            S::NKB * S::CH);
  } else {
    dma_w(c, dst, d.w + (long long)tile * d.wstride, d.nt * S::NKB * S::CH);
  }
}

// The row-wise form's gated-residual tasks and reducers cover one 16-column tile: they stage only that tile's
// gate and next scale, [sample][gate 16 | scale 16] floats (128 bytes per sample), instead of B x 2H floats
// (48 KB for 8 samples of width 768, all DMA'd ahead of the task's ready-epoch poll, which returns after them).
// One 1 KB DMA per 8 samples: lane l copies piece l % 4 of vector (l / 4) % 2 of sample l / 8.
template <class S>
__device__ __forceinline__ void dma_mods_tile(Ctx<S>& c, const Desc& d, int tile) {
  const int nb = (c.p.B + 7) >> 3;
  for (int k = c.dw; k < nb; k += c.dn) {
    const int b = min(k * 8 + (c.lane >> 3), c.p.B - 1), v = (c.lane >> 2) & 1, q = c.lane & 3;
    dma16(c.modrow(b, d.s) + (v ? d.mod_off2 : d.mod_off) + tile * 16 + 4 * q, c.smem + c.p.lds_mods + k * 1024);
  }
}

// ------------------------------------------------------------------------------------------------
// GEMM stage: out tile (16 columns, all rows) of A @ W^T for each task of this workgroup, computed
// transposed (D^T = W_tile A^T) so that each lane's accumulator is 4 consecutive output columns of one row:
// one 16-byte piece of the fragment-major output. A is an fp16 operand frame.
//   AdaRMS stages (K_QKV: q/k/v; K_GU): A = y = h * (1 + scale) was written by the
//     producer of h, so out = rstd(h) * (y W^T) + shift W^T (src/mk_expert.py:93-122); rstd comes from the
//     producer's per-tile sums of squares, shift W^T from an extra MFMA row tile whose rows are the
//     samples' shift slices. K_QKV: see qk_piece / the V^T epilogue; K_GU stores act(gate) * up in fp16
//     (:404-413).
//   K_RES: h_out = res + acc * gate (:162-172), stored fp32, plus y = h_out * (1 + next scale) in fp16 and
//     the tile's sums of squares of h_out; K_SPLIT: K-split partial; the tile's reducer sums the partials
//     in split order and applies K_RES (down_reduce).
// K (= H per task) is split over the 4 waves; the wave partials are summed through LDS.

// byte offset of the sum of squares of (row, 16-column tile t) in a [RT][HT / 2][16][2] array: one 128-byte
// line per (row tile, tile pair), written by the tasks that compute those two tiles of those rows; a row's
// two tiles of a pair are one 8-byte piece
template <int HT>
__device__ __forceinline__ uint32_t ss_slot(int row, int t) {
  return (uint32_t)(((((row >> 4) * (HT / 2) + (t >> 1)) * 16 + (row & 15)) * 2 + (t & 1)) * 4);
}

// residual epilogue of one 4-column piece: h = res + v * gate; stores h, y = h (1 + next scale) and the
// piece's share of the row's sum of squares (lanes L, L^16, L^32, L^48 hold one row's 16 columns)
template <class S>
__device__ __forceinline__ void res_piece(Ctx<S>& c, const Desc& d, int tile, int row, int col, int L, f32x4 v, f32x4 res) {
  const uint32_t off = fpiece(row, col, c.RT);
  // [gate | next scale] of the row's sample: full rows of H, or (row-wise form) the tile's 16 columns
  const float* ml = S::RW ? mods_lds(c, c.sample_of(row), 32) + (col & 15) : mods_lds(c, c.sample_of(row), 2 * S::H) + col;
  const int so = S::RW ? 16 : S::H;
  const f32x4 h = res + v * ldf4(ml);
  st_sc1(d.out, off, as_u4(h));
  const f32x4 hs = S::YS ? h * c.p.yinv : h;  // (the AdaRMS operand scaling)
  if (st_h4(d.yout, spiece(row, col, c.RT), hs * (1.0f + ldf4(ml + so)))) range_error(c.p.bar);
  float ss = hs[0] * hs[0] + hs[1] * hs[1] + hs[2] * hs[2] + hs[3] * hs[3];
  ss = xor32_sum(xor16_sum(ss));
  if (L < 16) st_sc1_b32(d.ssout, ss_slot<S::HT>(row, tile), __float_as_uint(ss));
}

// q/k epilogue of one row: xa, xb = columns d0 .. d0+3 and d0+32 .. d0+35 of head hd (kind 0 = q, 1 = k).
// Stores the row's share of the head's sum of squares (lanes L, L^16,
// L^32, L^48 hold the task's 32 columns) and u = rope(x (1 + w)) split (src/mk_expert.py:175-193; the RMS
// factor is applied to the scores).
// The epilogue's constant operands of one (row, 4-column) item, loaded with the activations: RoPE cos/sin of
// columns d0 and d0 + 32 and the norm weights (q/k tasks), or the residual piece (residual stages).
struct EpiPre {
  f32x4 c0, s0, c1, s1;
  uint2 w0, w1;
  f32x4 sa, sb;  // fp8 weights: output-channel scales of the item's columns (V tasks: one per 16-column tile)
};

// The constant part (RoPE tables, q/k norm weights, fp8 output-channel scales), loaded in each pass right
// after the operand loads: issued before the ready-epoch poll, these loads would delay the poll, since loads
// return in issue order per CU (3.33 to 3.28 ms for workload A).
template <class S>
__device__ __forceinline__ EpiPre epi_const(Ctx<S>& c, const Desc& d, int kind, int j, int tile, int row, int L) {
  CP& p = c.p;
  EpiPre e;
  if (d.kind == K_QKV && kind < 2) {
    const int d0 = 16 * j + 4 * (L >> 4);
    const bf16_t* nw = (kind == 0 ? p.qn : p.kn) + d.l * HD;
    e.w0 = *reinterpret_cast<const uint2*>(nw + d0);
    e.w1 = *reinterpret_cast<const uint2*>(nw + d0 + 32);
    const int pos = min(row - c.sample_of(row) * p.Mqp, p.Mq - 1);
    const float* cs = p.sa_cos + pos * HD + d0;
    const float* sn = p.sa_sin + pos * HD + d0;
    e.c0 = ldf4(cs);
    e.s0 = ldf4(sn);
    e.c1 = ldf4(cs + 32);
    e.s1 = ldf4(sn + 32);
  }
  if constexpr (S::W8) {
    // K_RES / K_GU: columns tile * 16 + 4 (L / 16) + 0..3 (gate/up: sa gate, sb up); q, k: d0 and d0 + 32 of
    // the head; v: column 16 j + L % 16 (+ 32 for the second tile) of the head
    if (d.kind == K_RES) {
      e.sa = ldf4(d.sc + tile * 16 + 4 * (L >> 4));
    } else if (d.kind == K_GU) {
      e.sa = ldf4(d.sc + tile * 16 + 4 * (L >> 4));
      e.sb = ldf4(d.sc2 + tile * 16 + 4 * (L >> 4));
    } else if (d.kind == K_QKV) {
      const float* sq = d.sc + kind * S::H + ((tile >> 1) % S::NH) * HD;
      if (kind < 2) {
        e.sa = ldf4(sq + 16 * j + 4 * (L >> 4));
        e.sb = ldf4(sq + 16 * j + 4 * (L >> 4) + 32);
      } else {
        e.sa[0] = sq[16 * j + (L & 15)];
        e.sa[1] = sq[16 * j + (L & 15) + 32];
      }
    }
  }
  return e;
}

// row of the epilogue item of thread tid in a pass over nrt row tiles from rt0
__device__ __forceinline__ int epi_row(int rt0, int nrt, int tid) { return (rt0 + min(tid >> 6, nrt - 1)) * 16 + (tid & 15); }

template <class S>
__device__ __forceinline__ void qk_piece(Ctx<S>& c, const Desc& d, int kind, int hd, int j, int row, int L, f32x4 xa, f32x4 xb,
                                         const EpiPre& e) {
  CP& p = c.p;
  float ss = xa[0] * xa[0] + xa[1] * xa[1] + xa[2] * xa[2] + xa[3] * xa[3] + xb[0] * xb[0] + xb[1] * xb[1] + xb[2] * xb[2] + xb[3] * xb[3];
  ss = xor32_sum(xor16_sum(ss));
  if (L < 16) st_sc1_b32(d.ssout, (uint32_t)((((long long)(kind * S::NH + hd) * 2 + j) * p.NRP + row) * 4), __float_as_uint(ss));
  const int d0 = 16 * j + 4 * (L >> 4);
  const uint2 wa = e.w0, wb = e.w1;
  const f32x4 ga = {1.0f + __uint_as_float(wa.x << 16), 1.0f + __uint_as_float(wa.x & 0xffff0000u),
                    1.0f + __uint_as_float(wa.y << 16), 1.0f + __uint_as_float(wa.y & 0xffff0000u)};
  const f32x4 gb = {1.0f + __uint_as_float(wb.x << 16), 1.0f + __uint_as_float(wb.x & 0xffff0000u),
                    1.0f + __uint_as_float(wb.y << 16), 1.0f + __uint_as_float(wb.y & 0xffff0000u)};
  const f32x4 za = xa * ga, zb = xb * gb;
  const f32x4 ua = za * e.c0 - zb * e.s0;
  const f32x4 ub = zb * e.c1 + za * e.s1;
  float* buf = kind == 0 ? d.out : d.yout;
  st_split4(buf, spiece(row, hd * HD + d0, c.RT), ua);
  st_split4(buf, spiece(row, hd * HD + d0 + 32, c.RT), ub);
}

// MFMAs of one pass (fp16 operands, fp16 weight fragments, fp32 accumulation) over this wave's k-blocks:
// acc[rt][nt][i % NA] (NA = 2: consecutive k-blocks alternate between two accumulators of each tile, so that no
// MFMA waits for its predecessor where the tiles alone are too few). SWAP (V tasks): D = A W^T; otherwise
// D^T = W A^T. ADA adds the shift row tile (always D^T) into accs[nt][i % 2].
template <class S, int NRT, int NT, int NTA, int NA, bool SWAP, bool ADA>
__device__ __forceinline__ void gemm_mma(f32x4 (&acc)[NRT][NTA][NA], f32x4 (&accs)[NTA][2], const f16x8 (&a)[NRT][S::KPW],
                                         const f16x8 (&sh)[S::KPW], const char* wl, int wave, int lane) {
#pragma unroll
  for (int i = 0; i < S::KPW; ++i) {
    const int kb = wave + NWAVES * i;
    f16x8 wf[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) wf[nt] = wfrag_lds<S>(wl + (nt * S::NKB + kb) * S::CH, lane);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt) {
        f32x4& r = acc[rt][nt][i % NA];
        r = SWAP ? mfma16h(a[rt][i], wf[nt], r) : mfma16h(wf[nt], a[rt][i], r);
      }
    if (ADA) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) accs[nt][i & 1] = mfma16h(wf[nt], sh[i], accs[nt][i & 1]);
    }
  }
}

// One pass of a GEMM task over row tiles rt0 .. rt0 + NRT - 1: operand loads (and, for AdaRMS stages, the
// shift fragments and sums of squares), the epilogue's preloaded constants, the MFMAs, and the per-wave
// partial tiles written to the cross-wave reduction buffer.
template <class S, int NRT>
__device__ __forceinline__ void gemm_pass(Ctx<S>& c, const Desc& d, int rt0, int kb0, bool vtask, int qkind, int qj,
                                          int tile, EpiPre& epre) {
  constexpr int KPW = S::KPW, RB = S::RBMAX;
  CP& p = c.p;
  const int RT = c.RT, NRP = p.NRP;
  const bool ada = d.kind == K_QKV || d.kind == K_GU;
  const __amdgpu_buffer_rsrc_t ra = rsrc(d.a);
  const uint32_t vlane = (uint32_t)c.lane * 16;
  float* ssw = (float*)(c.smem + S::SMALL);  // [4 waves][64 pass rows] partial sums of squares
  char* red = c.smem + p.lds_red;             // [wave][RB + 1][2][64 lanes] x 16 bytes
  // this wave's share (tiles wave HT / 4 .. + HT / 4 - 1, as HT / 8 pairs) of the sums of squares of pass row
  // `lane` (the lanes past the pass rows repeat its first row tile): loaded first, so that waiting for them
  // never waits for the operand loads
  u32x2 ssv[S::HT / 8];
  if (ada) {
    const __amdgpu_buffer_rsrc_t rs_ = rsrc(d.ssin);
    const int prow = c.lane < NRT * 16 ? c.lane : (c.lane & 15);
    const uint32_t so = ss_slot<S::HT>(min(rt0 * 16 + prow, NRP - 1), c.wave * (S::HT / 4));
#pragma unroll
    for (int i = 0; i < S::HT / 8; ++i) ssv[i] = bload8(rs_, so, (uint32_t)i * 128);
  }
  // fp16 operand fragments (the first 1 KB of each 2 KB block), k-block major, in the order the MFMAs use
  // them: the MFMAs of the first k-blocks start while the later blocks are still arriving
  f16x8 a[NRT][KPW];
#pragma unroll
  for (int i = 0; i < KPW; ++i)
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
      a[rt][i] = __builtin_bit_cast(f16x8, bload(ra, vlane, (uint32_t)(((kb0 + c.wave + NWAVES * i) * RT + rt0 + rt) * 2048)));
  f16x8 sh[KPW];  // the fp16 shift fragments of this wave's k-blocks (rows = samples)
  if (!ada) {
#pragma unroll
    for (int i = 0; i < KPW; ++i) sh[i] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
  }
  const int erow = epi_row(rt0, NRT, c.tid), eL = c.tid & 63;
  epre = epi_const(c, d, qkind, qj, tile, erow, eL);
  if (d.kind == K_RES) epre.c0 = as_f4(ld16((const char*)d.res + fpiece(erow, tile * 16 + 4 * (eL >> 4), c.RT)));
  // The staged weights and modulation slices (the prefetch's LDS DMAs, issued before every load above) and
  // the sums of squares have landed once no more than the activation loads are outstanding; the activations
  // are waited for where the MFMAs use them.
  wait_vm_le<NRT * KPW>();
  exec_barrier();
  if (ada) {
    // the shift fragments, staged in LDS by the prefetch: lane l reads sample l % 16 (zeros for the samples
    // >= B)
    const char* shl = c.smem + p.lds_mods;
    const bool has = (c.lane & 15) < p.B;
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      const int o = (((c.lane & 15) * S::NKB + c.wave + NWAVES * i) * 4 + (c.lane >> 4)) * 32;
      sh[i] = has ? ldsfrag_h(shl + o) : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
  }
  MKX_TR(c, 1);
  f32x4 acc[NRT][2][2], accs[2][2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) acc[rt][nt][0] = acc[rt][nt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    accs[nt][0] = accs[nt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const char* wl = c.smem + S::WBUF;
  if (vtask) gemm_mma<S, NRT, 2, 2, 2, true, true>(acc, accs, a, sh, wl, c.wave, c.lane);
  else if (d.nt == 2) gemm_mma<S, NRT, 2, 2, 2, false, true>(acc, accs, a, sh, wl, c.wave, c.lane);
  else gemm_mma<S, NRT, 1, 2, 2, false, false>(acc, accs, a, sh, wl, c.wave, c.lane);
  if (ada) ssw[c.wave * 64 + c.lane] = ss_pairs_sum<S::HT / 8>(ssv);
  // cross-wave reduction through LDS (the shift tile at slot RB)
#pragma unroll
  for (int rt = 0; rt <= NRT; ++rt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
      if (nt < d.nt && (rt < NRT || ada))
        sts16(red + (((c.wave * (RB + 1) + (rt < NRT ? rt : RB)) * 2 + nt) * 64 + c.lane) * 16,
              as_u4(rt < NRT ? acc[rt][nt][0] + acc[rt][nt][1] : accs[nt][0] + accs[nt][1]));
}

// One pass of a wide task (NTW column tiles; gated-residual stages over one row tile, down-projection splits
// over up to RBMAX): operand loads, the residual piece (and fp8 scales) of this thread's epilogue item
// (row tile rt0, column tile etile), the MFMAs, and the per-wave partial tiles at [wave][rt][nt] of the
// reduction buffer.
template <class S, int NRT>
__device__ __forceinline__ void gemm_pass_wide(Ctx<S>& c, const Desc& d, int rt0, int kb0, int etile, EpiPre& epre) {
  constexpr int KPW = S::KPW, NT = S::NTW, NA = NRT == 1 ? 2 : 1;
  CP& p = c.p;
  const int RT = c.RT;
  const __amdgpu_buffer_rsrc_t ra = rsrc(d.a);
  const uint32_t vlane = (uint32_t)c.lane * 16;
  char* red = c.smem + p.lds_red;
  f16x8 a[NRT][KPW];
#pragma unroll
  for (int i = 0; i < KPW; ++i)
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
      a[rt][i] = __builtin_bit_cast(f16x8, bload(ra, vlane, (uint32_t)(((kb0 + c.wave + NWAVES * i) * RT + rt0 + rt) * 2048)));
  f16x8 sh0[KPW];
#pragma unroll
  for (int i = 0; i < KPW; ++i) sh0[i] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
  if (d.kind == K_RES) {
    const int erow = rt0 * 16 + (c.tid & 15), eL = c.tid & 63;
    epre = epi_const(c, d, 0, 0, etile, erow, eL);
    epre.c0 = as_f4(ld16((const char*)d.res + fpiece(erow, etile * 16 + 4 * (eL >> 4), RT)));
  }
  // the staged weight tiles (issued before every load above) have landed
  wait_vm_le<NRT * KPW>();
  exec_barrier();
  MKX_TR(c, 1);
  f32x4 acc[NRT][NT][NA], accs[NT][2];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
      for (int h = 0; h < NA; ++h) acc[rt][nt][h] = f32x4{0.f, 0.f, 0.f, 0.f};
    accs[nt][0] = accs[nt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  gemm_mma<S, NRT, NT, NT, NA, false, false>(acc, accs, a, sh0, c.smem + S::WBUF, c.wave, c.lane);
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      f32x4 v = acc[rt][nt][0];
      if (NA == 2) v += acc[rt][nt][NA - 1];
      sts16(red + (((c.wave * NRT + rt) * NT + nt) * 64 + c.lane) * 16, as_u4(v));
    }
}

// Waits until the producer tasks of stage g - 1 whose output lines this task reads have published: QKV reads
// every column of its rows (the down projection's reducers or the step tail's in-projection tasks), the
// out-projections read every head of their row tiles (attention tasks), gate/up every row of every column
// (all out-projection tasks), a down split its quarter of the gate/up tiles.
template <class S>
__device__ __forceinline__ void gemm_wait(Ctx<S>& c, const Desc& d, BarCtx& bc, int g, int split, int rt_lo, int rt_hi) {
  const int NQT = c.p.Mqp / 16;
  if (d.st == ST_QKV) {
    // every column of its rows: the step tail's in-projection tasks, or the down projection's reducers
    if constexpr (S::RW) {
      // (row-wise form: the reducers of this task's row group; the row groups are the same)
      const int rg = split;
      if (d.l == 0) flag_wait<1>(bc, F_TAIL_IN, S::NIN, [](int i) { return i; }, (unsigned long long)g);
      else flag_wait<1>(bc, F_DOWN, S::HT, [&](int i) { return rg * S::HT + i; }, (unsigned long long)g);
    } else {
      flag_wait<1>(bc, d.l == 0 ? F_TAIL_IN : F_DOWN, d.l == 0 ? S::NIN : c.p.nred, [](int i) { return i; }, (unsigned long long)g);
    }
  } else if (d.st == ST_O || d.st == ST_CAO) {
    flag_wait(bc, d.st == ST_O ? F_SA : F_CA, (rt_hi - rt_lo) * S::NH, [&](int i) {
      const int rt = rt_lo + i / S::NH, hd = i % S::NH;
      return ((rt / NQT) * S::NH + hd) * NQT + rt % NQT;
    }, (unsigned long long)g);
  } else if (d.st == ST_GU) {
    flag_wait(bc, F_CAO, (S::HT / c.p.nt_cao) * c.p.rgs_cao, [](int i) { return i; }, (unsigned long long)g);
  } else {
    flag_wait<1>(bc, F_GU, S::HT, [&](int i) { return split * S::HT + i; }, (unsigned long long)g);
  }
}

// Down-projection reducer r: once the split tasks of its output tiles t0 .. t0 + TPR - 1 have published
// their partial sums (SK per tile group of nt tiles: split task (split, group) is task split * tiles + group),
// it adds them in split order and applies the gated residual (hl = h3 + gate * sum, with yl and the sums of
// squares for the next AdaRMS), then publishes one ready epoch for the TPR tiles. Instantiated for the two
// reducer widths the host uses (Params::tpr: the wide tasks' NTW tiles, or one).
template <class S, int TPR>
__device__ __forceinline__ void down_reduce(Ctx<S>& c, const Desc& d, BarCtx& bc, int g, int r) {
  constexpr int tpr = TPR;
  const int RT = c.RT;
  // (row-wise form: reducer r covers tile r % HT over the row tiles of row group r / HT; the form with
  // passes: tiles r tpr .. of every row tile)
  int t0, rlo, nrt;
  if constexpr (S::RW) {
    const int rgr = r / S::HT;
    t0 = (r % S::HT) * tpr;
    rlo = rgr * RT / c.p.nrg;
    nrt = (rgr + 1) * RT / c.p.nrg - rlo;
  } else {
    t0 = r * tpr;
    rlo = 0;
    nrt = RT;
  }
  // the tile groups (split tasks per split) holding tiles t0 .. t0 + tpr - 1
  const int g0 = t0 / d.nt, ng = (t0 + tpr - 1) / d.nt - g0 + 1;
  flag_wait<1>(bc, F_DPART, S::SK * ng, [&](int i) { return (i % S::SK) * d.tiles + g0 + i / S::SK; }, (unsigned long long)g);
  wait_vm0();  // the staged gate and next AdaRMS scale (the prefetch's DMA) have landed
  __syncthreads();
  // one (tile, row tile) block of 64 items per wave and round (lanes L, L^16, L^32, L^48 hold one row);
  // the loads of RR rounds are issued together, so their latencies overlap
  constexpr int RR = 3;
  const int nblk = tpr * nrt;
  for (int b0 = c.wave; b0 < nblk; b0 += NWAVES * RR) {
    u32x4 xp[RR][S::SK];
    f32x4 res[RR];
#pragma unroll
    for (int k = 0; k < RR; ++k) {
      const int blk = min(b0 + NWAVES * k, nblk - 1);
      const int tile = t0 + blk / nrt, rtg = rlo + blk % nrt, L = c.lane;
#pragma unroll
      for (int j = 0; j < S::SK; ++j) xp[k][j] = ld16((const char*)d.part + ((((j * S::HT + tile) * RT + rtg) * 64 + L) * 16));
      res[k] = as_f4(ld16((const char*)d.res + fpiece(rtg * 16 + (L & 15), tile * 16 + 4 * (L >> 4), RT)));
    }
#pragma unroll
    for (int k = 0; k < RR; ++k) {
      const int blk = b0 + NWAVES * k;
      if (blk >= nblk) break;
      const int tile = t0 + blk / nrt, rtg = rlo + blk % nrt, L = c.lane;
      const int row = rtg * 16 + (L & 15), col = tile * 16 + 4 * (L >> 4);
      f32x4 v = as_f4(xp[k][0]);
#pragma unroll
      for (int j = 1; j < S::SK; ++j) v += as_f4(xp[k][j]);
      if (S::W8) v *= ldf4(d.sc + col);  // the output channel's scale
      res_piece(c, d, tile, row, col, L, v, res[k]);
    }
  }
  MKX_TR(c, 7);
  flag_publish(bc, F_DOWN, r, (unsigned long long)g + 1);
}

template <class S>
__device__ __forceinline__ void gemm_stage(Ctx<S>& c, const Desc& d, BarCtx& bc, int g) {
  constexpr int KPW = S::KPW, RB = S::RBMAX;
  CP& p = c.p;
  const int RT = c.RT, NRP = p.NRP;
  const bool ada = d.kind == K_QKV || d.kind == K_GU;
  const __amdgpu_buffer_rsrc_t ra = rsrc(d.a);
  const uint32_t vlane = (uint32_t)c.lane * 16;
  float* ssw = (float*)(c.smem + S::SMALL);  // [4 waves][64 pass rows] partial sums of squares
  char* red = c.smem + p.lds_red;             // [wave][RB + 1][2][64 lanes] x 16 bytes (wide: [wave][rt][nt])
  // wide tasks (gated-residual or down-projection tasks of NTW column tiles); a wide gated-residual pass
  // covers one row tile, so that each wave's epilogue item is one column tile of it
  const bool wide = (d.kind == K_RES || d.kind == K_SPLIT) && d.nt > 1;
  const int RBS = wide && d.kind == K_RES ? 1 : RB;
  const int t0 = task_first(c, d.pk);
  for (int t = t0; t < d.ntask; t += c.G) {
    const int tile = t % d.tiles, split = t / d.tiles;  // split: K quarter (K_SPLIT) or row group
    // QKV tiles: kind (q, k, v), head, quarter pair j; v is computed untransposed (D = A W^T) so that each
    // lane holds 4 consecutive keys of one d: 8 bytes of the V^T layout
    const int qkind = d.kind == K_QKV ? tile / (2 * S::NH) : 0, qhd = (tile >> 1) % S::NH, qj = tile & 1;
    const bool vtask = qkind == 2;
    if (t != t0) {  // later tasks of this workgroup: load their weights now (the first was prefetched)
      wait_vm0();
      __syncthreads();
      dma_task_w(c, d, t, c.smem + S::WBUF);
    }
    const int kb0 = d.kind == K_SPLIT ? split * S::NKB : 0;
    const int rt_lo = d.kind == K_SPLIT ? 0 : split * RT / d.rgs;
    const int rt_hi = d.kind == K_SPLIT ? RT : (split + 1) * RT / d.rgs;
    // The epilogue's constant operands are loaded in each pass after its operand loads, not before the
    // wait: loads return in issue order per CU, so a load issued before the ready-epoch poll delays the poll.
    EpiPre epre;
    MKX_TR(c, 14);
    gemm_wait(c, d, bc, g, split, rt_lo, rt_hi);
    MKX_TR(c, 0);
    for (int rt0 = rt_lo; rt0 < rt_hi; rt0 += RBS) {
      const int nrt = min(RBS, rt_hi - rt0);
      if (wide) {
        const int etile = tile * d.nt + min(c.wave, d.nt - 1);
        if (nrt == 1) gemm_pass_wide<S, 1>(c, d, rt0, kb0, etile, epre);
        else if (nrt == 2 || RB == 2) gemm_pass_wide<S, (RB < 2 ? 1 : 2)>(c, d, rt0, kb0, etile, epre);
        else gemm_pass_wide<S, RB>(c, d, rt0, kb0, etile, epre);
      } else {
        if (nrt == 1) gemm_pass<S, 1>(c, d, rt0, kb0, vtask, qkind, qj, tile, epre);
        else if (nrt == 2 || RB == 2) gemm_pass<S, (RB < 2 ? 1 : 2)>(c, d, rt0, kb0, vtask, qkind, qj, tile, epre);
        else gemm_pass<S, RB>(c, d, rt0, kb0, vtask, qkind, qj, tile, epre);
      }
      __syncthreads();
      MKX_TR(c, 2);
      if (wide) {
        // one (row tile, column tile) block of 64 items per wave and round: row (rt0 + rt) * 16 + L % 16,
        // columns of 16-column tile tile * nt + j, 4 (L / 16) + 0..3; gated-residual passes have one row
        // tile, so wave j's block is the one its preloaded residual piece belongs to
        for (int blk = c.wave; blk < nrt * d.nt; blk += NWAVES) {
          const int rt = blk / d.nt, j = blk - rt * d.nt, L = c.lane;
          f32x4 pw[NWAVES];
#pragma unroll
          for (int w = 0; w < NWAVES; ++w) pw[w] = ldf4((const float*)(red + (((w * nrt + rt) * d.nt + j) * 64 + L) * 16));
          lds_batch(pw);
          const f32x4 v = ((pw[0] + pw[1]) + pw[2]) + pw[3];
          const int t16 = tile * d.nt + j;
          if (d.kind == K_SPLIT) {
            st_sc1(d.part, (uint32_t)((((split * S::HT + t16) * RT + rt0 + rt) * 64 + L) * 16), as_u4(v));
          } else {
            const int row = (rt0 + rt) * 16 + (L & 15), col = t16 * 16 + 4 * (L >> 4);
            res_piece(c, d, t16, row, col, L, S::W8 ? v * epre.sa : v, epre.c0);
          }
        }
      } else
      // epilogue: one (row tile, lane) item per thread: row (rt0 + rt) * 16 + L % 16, columns tile*16 + 4 (L / 16) + 0..3
      {
        const int rt = c.tid >> 6, L = c.tid & 63;
        if (rt < nrt) {
          // every LDS operand of the item is read as one batch (the 4 waves' partial tiles, the shift tile's
          // rows, the partial sums of squares), then summed in wave order
          auto sum4 = [](const f32x4 (&pw)[NWAVES]) { return ((pw[0] + pw[1]) + pw[2]) + pw[3]; };
          constexpr int WS = (RB + 1) * 2 * 64 * 16;  // bytes per wave's partial tiles
          const int row = (rt0 + rt) * 16 + (L & 15);
          const int col = tile * 16 + 4 * (L >> 4);
          if (vtask) {
            // lane L: d = 16 j + 32 nt + L % 16, rows (keys) 4 (L / 16) + e of a 16-row tile of one sample
            const int row0 = (rt0 + rt) * 16, b = c.sample_of(row0);
            const int ib = row0 - b * p.Mqp + 4 * (L >> 4);
            const int KBO = ceil_to(p.Mq, 32) / 32;
            const int cl = L & 15, bl = b + 16 * (cl >> 2);
            // the 4 rows' sums of squares (rows rt * 16 + 4 (L / 16) + 0..3), both column tiles' partials and
            // the shift tile's entries of this lane's column
            f32x4 sw[NWAVES], a0[NWAVES], a1[NWAVES];
            float b0[NWAVES], b1[NWAVES];
#pragma unroll
            for (int w = 0; w < NWAVES; ++w) {
              const char* rw = red + w * WS;
              sw[w] = ldf4(ssw + 64 * w + rt * 16 + 4 * (L >> 4));
              a0[w] = ldf4((const float*)(rw + ((rt * 2 + 0) * 64 + L) * 16));
              a1[w] = ldf4((const float*)(rw + ((rt * 2 + 1) * 64 + L) * 16));
              b0[w] = ((const float*)(rw + ((RB * 2 + 0) * 64 + bl) * 16))[cl & 3];
              b1[w] = ((const float*)(rw + ((RB * 2 + 1) * 64 + bl) * 16))[cl & 3];
            }
            lds_batch(sw);
            lds_batch(a0);
            lds_batch(a1);
            lds_batch(b0);
            lds_batch(b1);
            const f32x4 tot = sum4(sw);
            float rs[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) rs[e] = rsqrtf(tot[e] * (1.0f / (float)S::H) + p.eps);
            const uint32_t vo = (uint32_t)(((b * S::NH + qhd) * KBO + (ib >> 5)) * 8192 + L * 16 + ((ib >> 4) & 1) * 8);
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
              const f32x4 a = sum4(nt ? a1 : a0);
              const float* bb = nt ? b1 : b0;
              const float bias = ((bb[0] + bb[1]) + bb[2]) + bb[3];
              const float sv = S::W8 ? epre.sa[nt] : 1.0f;  // fp8: the output channel's scale
              f32x4 x;
#pragma unroll
              for (int e = 0; e < 4; ++e) x[e] = ib + e < p.Mq ? (a[e] * rs[e] + bias) * sv : 0.f;
              st_split4(d.part, vo + (uint32_t)((qj + 2 * nt) * 2048), x);
            }
          } else if (d.kind == K_SPLIT || d.kind == K_RES) {
            f32x4 pw[NWAVES];
#pragma unroll
            for (int w = 0; w < NWAVES; ++w) pw[w] = ldf4((const float*)(red + w * WS + ((rt * 2) * 64 + L) * 16));
            lds_batch(pw);
            const f32x4 v = sum4(pw);
            if (d.kind == K_SPLIT) st_sc1(d.part, (uint32_t)((((split * d.tiles + tile) * RT + rt0 + rt) * 64 + L) * 16), as_u4(v));
            else res_piece(c, d, tile, row, col, L, S::W8 ? v * epre.sa : v, epre.c0);
          } else {
            // the two column tiles' partials, the shift tile's rows of this lane's sample and the row's partial
            // sums of squares
            const int r = rt * 16 + (L & 15);
            const int bl = c.sample_of(row) + 16 * (L >> 4);
            f32x4 pv[NWAVES], pu[NWAVES], pb0[NWAVES], pb1[NWAVES];
            float sw[NWAVES];
#pragma unroll
            for (int w = 0; w < NWAVES; ++w) {
              const char* rw = red + w * WS;
              pv[w] = ldf4((const float*)(rw + ((rt * 2 + 0) * 64 + L) * 16));
              pu[w] = ldf4((const float*)(rw + ((rt * 2 + 1) * 64 + L) * 16));
              pb0[w] = ldf4((const float*)(rw + ((RB * 2 + 0) * 64 + bl) * 16));
              pb1[w] = ldf4((const float*)(rw + ((RB * 2 + 1) * 64 + bl) * 16));
              sw[w] = ssw[64 * w + r];
            }
            lds_batch(pv);
            lds_batch(pu);
            lds_batch(pb0);
            lds_batch(pb1);
            lds_batch(sw);
            const float rs = rsqrtf((((sw[0] + sw[1]) + sw[2]) + sw[3]) * (1.0f / (float)S::H) + p.eps);
            f32x4 v = sum4(pv) * rs + sum4(pb0);
            f32x4 u = sum4(pu) * rs + sum4(pb1);
            if (S::W8) {  // output-channel scales (the shift row tile used the same weights)
              v *= epre.sa;
              u *= epre.sb;
            }
            if (d.kind == K_GU) {
#pragma unroll
              for (int j = 0; j < 4; ++j) v[j] = act_fn(v[j], p.act) * u[j];
              if (st_h4(d.out, spiece(row, col, RT), v)) range_error(p.bar);
            } else {
              qk_piece(c, d, qkind, qhd, qj, row, L, v, u, epre);
            }
          }
        }
      }
      if (rt0 + RBS < rt_hi) __syncthreads();  // red and ssw are reused by the next pass
      MKX_TR(c, 3);
    }
    flag_publish(bc, d.st == ST_QKV ? F_QKV : d.st == ST_O ? F_O : d.st == ST_CAO ? F_CAO : d.st == ST_GU ? F_GU : F_DPART, t,
                 (unsigned long long)g + 1);
  }
  if (d.kind == K_SPLIT) {
    const int r = task_first(c, PL_RED);
    if (r < p.nred) {
      if (p.tpr == S::NTW) down_reduce<S, S::NTW>(c, d, bc, g, r);
      else down_reduce<S, 1>(c, d, bc, g, r);
    }
  }
}

// ------------------------------------------------------------------------------------------------
// Row-wise GEMM stages, for launches whose tasks cover more row tiles than one pass of gemm_stage holds
// (batched samples, long chunks): gemm_stage runs such a task as passes that each wait for their operands,
// sum the four waves' K quarters through LDS and run the epilogue, one after the other. Here each wave
// computes whole-K products of its own rows instead: groups of ROWS_NR consecutive row tiles of the task,
// round-robin over the waves, with the operand fragments streamed by loads issued ROWS_PF k-blocks ahead of
// the MFMAs (the first group's first loads are issued before the shift tile), and the epilogue of a group run from the wave's own accumulators. No
// cross-wave reduction and no barrier between groups; every wave reads all k-blocks of the task's weight tiles
// from LDS. AdaRMS tasks compute the shift row tile once per task (a quarter of K per wave, summed through
// LDS), and each lane loads the sums of squares of its row's quarter of the tiles (summed across the four
// lanes holding the row).
// The host uses this form only where every task has at most two column tiles (the layout with one task per
// workgroup and stage).
constexpr int ROWS_NR = 2;  // row tiles per group
constexpr int ROWS_PF = 8;  // k-blocks of operand loads in flight ahead of the MFMAs
template <class S>
constexpr int rows_pf() { return ROWS_PF < S::NKB ? ROWS_PF : S::NKB; }

// soffsets of the operand blocks (k-block 0) of the group at row tile rt0: row tiles from rt_hi on repeat the
// last valid one
__device__ __forceinline__ void rows_roff(uint32_t (&roff)[ROWS_NR], int rt0, int rt_hi) {
#pragma unroll
  for (int r = 0; r < ROWS_NR; ++r) roff[r] = (uint32_t)min(rt0 + r, rt_hi - 1) * 2048;
}
// the operand loads of a group's first rows_pf() k-blocks
template <class S>
__device__ __forceinline__ void rows_head(f16x8 (&pre)[rows_pf<S>()][ROWS_NR], __amdgpu_buffer_rsrc_t ra, const uint32_t (&roff)[ROWS_NR],
                                          int kb0, int RT, int lane) {
#pragma unroll
  for (int i = 0; i < rows_pf<S>(); ++i)
#pragma unroll
    for (int r = 0; r < ROWS_NR; ++r)
      pre[i][r] = __builtin_bit_cast(f16x8, bload(ra, (uint32_t)lane * 16, (uint32_t)((kb0 + i) * RT) * 2048 + roff[r]));
}

// D^T = W A^T (SWAP: D = A W^T) of NT weight tiles (LDS, [tile][k-block] chunks) over ROWS_NR row tiles
// (operand blocks at soffset roff[r] of k-block 0) and every k-block of the task from kb0; consecutive
// k-blocks alternate between two accumulators per product. pre holds the loads of the first rows_pf()
// k-blocks (issued by rows_head). Each k-block's step issues the operand loads of
// k-block i + ROWS_PF and the LDS reads of the weight fragments of k-block i + 1 before its MFMAs, and ends in
// a scheduling barrier: left to itself, the scheduler moves every load down to its use (fewer live
// registers), which leaves one memory round trip per k-block.
template <class S, int NT, bool SWAP>
__device__ __forceinline__ void rows_mma(f32x4 (&acc)[ROWS_NR][NT][2], __amdgpu_buffer_rsrc_t ra, const uint32_t (&roff)[ROWS_NR],
                                         int kb0, int RT, const char* wl, int lane, const f16x8 (&pre)[rows_pf<S>()][ROWS_NR]) {
  constexpr int NKB = S::NKB, PF = rows_pf<S>();
  const uint32_t vl = (uint32_t)lane * 16;
  f16x8 a[NKB][ROWS_NR];
#pragma unroll
  for (int i = 0; i < PF; ++i)
#pragma unroll
    for (int r = 0; r < ROWS_NR; ++r) a[i][r] = pre[i][r];
  // the weight fragments are read WA k-blocks ahead (two in the fp16-weight kernels: B 5.680 -> 5.656 ms; the
  // fp8 kernels, which decode their fragments, measured slower with two: D +12 us, D-b4 +23 us)
  constexpr int WA = S::W8 ? 1 : 2;
  f16x8 wn[WA][NT];
#pragma unroll
  for (int j = 0; j < WA; ++j)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) wn[j][nt] = wfrag_lds<S>(wl + (nt * NKB + j) * S::CH, lane);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < NKB; ++i) {
    if (i + PF < NKB) {
#pragma unroll
      for (int r = 0; r < ROWS_NR; ++r)
        a[i + PF][r] = __builtin_bit_cast(f16x8, bload(ra, vl, (uint32_t)((kb0 + i + PF) * RT) * 2048 + roff[r]));
    }
    f16x8 wf[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) wf[nt] = wn[i % WA][nt];
    if (i + WA < NKB) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) wn[i % WA][nt] = wfrag_lds<S>(wl + (nt * NKB + i + WA) * S::CH, lane);
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int r = 0; r < ROWS_NR; ++r) {
        f32x4& x = acc[r][nt][i & 1];
        x = SWAP ? mfma16h(a[i][r], wf[nt], x) : mfma16h(wf[nt], a[i][r], x);
      }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// One group of a wave: row tiles rt0 .. rt0 + ROWS_NR - 1 (those from rt_hi on repeat the last valid one and
// store nothing), whose first loads (pre) rows_head has issued. NT = 2: AdaRMS tasks (QKV, gate/up; SWAP: V), whose shift-tile partials the waves left in LDS; NT = 1:
// gated-residual (K_RES) or down-projection split (K_SPLIT) tasks.
template <class S, int NT, bool SWAP>
__device__ __forceinline__ void rows_group(Ctx<S>& c, const Desc& d, int rt0, int rt_hi, int kb0, int tile, int split, int qkind,
                                           int qhd, int qj, const f16x8 (&pre)[rows_pf<S>()][ROWS_NR]) {
  constexpr int NR = ROWS_NR, HT = S::HT;
  CP& p = c.p;
  const int RT = c.RT, L = c.lane;
  const char* red = c.smem + p.lds_red;  // [wave][2 tiles][64 lanes] x 16 bytes: shift-tile partials
  int rts[NR];
  uint32_t roff[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) rts[r] = min(rt0 + r, rt_hi - 1);
  rows_roff(roff, rt0, rt_hi);
  // the epilogue's operands, issued before the operand stream: sums of squares (this lane's quarter of its
  // row's tile pairs), constants (RoPE tables, norm weights, fp8 scales) and residual pieces
  u32x2 ssv[NR][HT / 8];
  EpiPre ep[NR];
  f32x4 res[NR];
  const int col = tile * 16 + 4 * (L >> 4);
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int row = rts[r] * 16 + (L & 15);
    if constexpr (NT == 2) {
      const __amdgpu_buffer_rsrc_t rs_ = rsrc(d.ssin);
      const uint32_t so = ss_slot<HT>(row, (L >> 4) * (HT / 4));
#pragma unroll
      for (int i = 0; i < HT / 8; ++i) ssv[r][i] = bload8(rs_, so, (uint32_t)i * 128);
    }
    ep[r] = epi_const(c, d, qkind, qj, tile, row, L);
    if constexpr (NT == 1) {
      if (d.kind == K_RES) res[r] = as_f4(ld16((const char*)d.res + fpiece(row, col, RT)));
    }
  }
  f32x4 acc[NR][NT][2];
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[r][nt][0] = acc[r][nt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  rows_mma<S, NT, SWAP>(acc, rsrc(d.a), roff, kb0, RT, c.smem + S::WBUF, L, pre);
  auto sum4 = [](const f32x4 (&pw)[NWAVES]) { return ((pw[0] + pw[1]) + pw[2]) + pw[3]; };
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    if (rt0 + r >= rt_hi) break;
    const int row = rts[r] * 16 + (L & 15);
    if constexpr (NT == 1) {
      const f32x4 v = acc[r][0][0] + acc[r][0][1];
      if (d.kind == K_SPLIT) st_sc1(d.part, (uint32_t)((((split * d.tiles + tile) * RT + rts[r]) * 64 + L) * 16), as_u4(v));
      else res_piece(c, d, tile, row, col, L, S::W8 ? v * ep[r].sa : v, res[r]);
    } else {
      // the row's sum of squares: this lane's quarter, then the four lanes holding the row
      const float ss = xor32_sum(xor16_sum(ss_pairs_sum<HT / 8>(ssv[r])));
      if constexpr (SWAP) {
        // V: lane L holds column 16 j + 32 nt + L % 16 of the head for rows (keys) 4 (L / 16) + e of a
        // 16-row tile of one sample; their RMS factors come from the lanes holding those rows
        const int row0 = rts[r] * 16, b = c.sample_of(row0);
        const int ib = row0 - b * p.Mqp + 4 * (L >> 4);
        const int KBO = ceil_to(p.Mq, 32) / 32;
        const int cl = L & 15, bl = b + 16 * (cl >> 2);
        float rsv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) rsv[e] = rsqrtf(__shfl(ss, 4 * (L >> 4) + e) * (1.0f / (float)S::H) + p.eps);
        float b0[NWAVES], b1[NWAVES];
#pragma unroll
        for (int w = 0; w < NWAVES; ++w) {
          b0[w] = ((const float*)(red + ((w * 2 + 0) * 64 + bl) * 16))[cl & 3];
          b1[w] = ((const float*)(red + ((w * 2 + 1) * 64 + bl) * 16))[cl & 3];
        }
        lds_batch(b0);
        lds_batch(b1);
        const uint32_t vo = (uint32_t)(((b * S::NH + qhd) * KBO + (ib >> 5)) * 8192 + L * 16 + ((ib >> 4) & 1) * 8);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          const f32x4 a = acc[r][nt][0] + acc[r][nt][1];
          const float* bb = nt ? b1 : b0;
          const float bias = ((bb[0] + bb[1]) + bb[2]) + bb[3];
          const float sv = S::W8 ? ep[r].sa[nt] : 1.0f;
          f32x4 x;
#pragma unroll
          for (int e = 0; e < 4; ++e) x[e] = ib + e < p.Mq ? (a[e] * rsv[e] + bias) * sv : 0.f;
          st_split4(d.part, vo + (uint32_t)((qj + 2 * nt) * 2048), x);
        }
      } else {
        const float rsr = rsqrtf(ss * (1.0f / (float)S::H) + p.eps);
        const int bl = c.sample_of(row) + 16 * (L >> 4);
        f32x4 pb0[NWAVES], pb1[NWAVES];
#pragma unroll
        for (int w = 0; w < NWAVES; ++w) {
          pb0[w] = ldf4((const float*)(red + ((w * 2 + 0) * 64 + bl) * 16));
          pb1[w] = ldf4((const float*)(red + ((w * 2 + 1) * 64 + bl) * 16));
        }
        lds_batch(pb0);
        lds_batch(pb1);
        f32x4 v = (acc[r][0][0] + acc[r][0][1]) * rsr + sum4(pb0);
        f32x4 u = (acc[r][1][0] + acc[r][1][1]) * rsr + sum4(pb1);
        if (S::W8) {
          v *= ep[r].sa;
          u *= ep[r].sb;
        }
        if (d.kind == K_GU) {
#pragma unroll
          for (int j = 0; j < 4; ++j) v[j] = act_fn(v[j], p.act) * u[j];
          if (st_h4(d.out, spiece(row, col, RT), v)) range_error(p.bar);
        } else {
          qk_piece(c, d, qkind, qhd, qj, row, L, v, u, ep[r]);
        }
      }
    }
  }
}

template <class S>
__device__ __forceinline__ void gemm_stage_rows(Ctx<S>& c, const Desc& d, BarCtx& bc, int g) {
  constexpr int KPW = S::KPW, NKB = S::NKB, NR = ROWS_NR;
  CP& p = c.p;
  const int RT = c.RT, L = c.lane;
  const bool ada = d.kind == K_QKV || d.kind == K_GU;
  const int t0 = task_first(c, d.pk);
  for (int t = t0; t < d.ntask; t += c.G) {
    const int tile = t % d.tiles, split = t / d.tiles;
    const int qkind = d.kind == K_QKV ? tile / (2 * S::NH) : 0, qhd = (tile >> 1) % S::NH, qj = tile & 1;
    if (t != t0) {
      wait_vm0();
      __syncthreads();
      dma_task_w(c, d, t, c.smem + S::WBUF);
      if (d.kind == K_RES) dma_mods_tile(c, d, tile);
    }
    const int kb0 = d.kind == K_SPLIT ? split * NKB : 0;
    const int rt_lo = d.kind == K_SPLIT ? 0 : split * RT / d.rgs;
    const int rt_hi = d.kind == K_SPLIT ? RT : (split + 1) * RT / d.rgs;
    MKX_TR(c, 14);
    gemm_wait(c, d, bc, g, split, rt_lo, rt_hi);
    MKX_TR(c, 0);
    // the task's weight tiles (and a gated-residual task's modulation slices: the prefetch's DMA) have landed
    wait_vm0();
    __syncthreads();
    MKX_TR(c, 1);
    // AdaRMS tasks: the fp16 shift fragments of this wave's k-blocks (lane l: sample l % 16, zeros for the
    // samples >= B), loaded from the launch's copy after the poll rather than staged in LDS ahead of it (the
    // poll returns only after every load issued before it), and before the operand loads, so they land first
    f16x8 shv[KPW];
    if (ada) {
      const bool has = (L & 15) < p.B;
      const int sb = min(L & 15, p.B - 1);
#pragma unroll
      for (int i = 0; i < KPW; ++i) {
        const f16x8 v = __builtin_bit_cast(f16x8, ld16(d.shs + ((sb * NKB + c.wave + NWAVES * i) * 4 + (L >> 4)) * 32));
        shv[i] = has ? v : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
    // the operand loads of this wave's first group go out before the shift tile
    const int ng = (rt_hi - rt_lo + NR - 1) / NR;
    const __amdgpu_buffer_rsrc_t ra = rsrc(d.a);
    f16x8 pre[rows_pf<S>()][NR];
    if (c.wave < ng) {
      uint32_t roff0[NR];
      rows_roff(roff0, rt_lo + c.wave * NR, rt_hi);
      rows_head<S>(pre, ra, roff0, kb0, RT, L);
    }
    if (ada) {
      // shift row tile (rows = samples) over this wave's k-blocks, into LDS
      const char* wl = c.smem + S::WBUF;
      f32x4 accs[2][2];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) accs[nt][0] = accs[nt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < KPW; ++i) {
        const int kb = c.wave + NWAVES * i;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) accs[nt][i & 1] = mfma16h(wfrag_lds<S>(wl + (nt * NKB + kb) * S::CH, L), shv[i], accs[nt][i & 1]);
      }
      char* red = c.smem + p.lds_red;
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) sts16(red + ((c.wave * 2 + nt) * 64 + L) * 16, as_u4(accs[nt][0] + accs[nt][1]));
      __syncthreads();
    }
    MKX_TR(c, 2);
    for (int gi = c.wave; gi < ng; gi += NWAVES) {
      const int rt0 = rt_lo + gi * NR;
      if (gi != c.wave) {  // the wave's later groups: their first loads now
        uint32_t roffg[NR];
        rows_roff(roffg, rt0, rt_hi);
        rows_head<S>(pre, ra, roffg, kb0, RT, L);
      }
      if (d.kind == K_QKV && qkind == 2) rows_group<S, 2, true>(c, d, rt0, rt_hi, kb0, tile, split, qkind, qhd, qj, pre);
      else if (ada) rows_group<S, 2, false>(c, d, rt0, rt_hi, kb0, tile, split, qkind, qhd, qj, pre);
      else rows_group<S, 1, false>(c, d, rt0, rt_hi, kb0, tile, split, qkind, qhd, qj, pre);
      MKX_TR(c, gi < 4 ? 3 : gi < 8 ? 5 : gi < 12 ? 11 : 12);  // wave 0's groups
    }
    flag_publish(bc, d.st == ST_QKV ? F_QKV : d.st == ST_O ? F_O : d.st == ST_CAO ? F_CAO : d.st == ST_GU ? F_GU : F_DPART, t,
                 (unsigned long long)g + 1);
  }
  if (d.kind == K_SPLIT) {
    const int r = task_first(c, PL_RED);
    if (r < p.nred) {
      if (p.tpr == S::NTW) down_reduce<S, S::NTW>(c, d, bc, g, r);
      else down_reduce<S, 1>(c, d, bc, g, r);
    }
  }
}

// ------------------------------------------------------------------------------------------------
// Attention. One task per (sample, head, 16-query tile); its 4 waves take the 32-key blocks round-robin
// and merge their online-softmax states through LDS at the end.
// K chunk (key tile kt, d-block db), 1 KB: lane l holds K[kt*16 + l%16][db*32 + 8(l/16) + j] (the split
// frame's hi or lo half, so own-row Q/K chunks are DMA'd straight from the projection's output). Vt chunk
// (32-key block kb, 16-d slice dt), 1 KB: lane l = d%16 + 16 g holds V[kb*32 + key_j][dt*16 + d%16] for
// key_j = (j/4)*16 + 4g + j%4, j < 8. Scores are computed transposed (S^T = K Q^T), so a lane holds, for
// its query l%16, exactly the 8 keys its P operand of P V needs in that order: the probabilities never
// leave registers. The own-row q and k arrive un-normalised (u = rope(x (1 + w))); their RMS factors
// multiply the scores (src/mk_expert.py:175-222 rearranged: rms(x) is a per-row scalar and RoPE is linear).

__device__ __forceinline__ int kchunk_off(int row, int d) {  // byte offset of 8 d-values (d % 8 == 0)
  return ((row >> 4) * 2 + (d >> 5)) * 1024 + ((row & 15) + 16 * ((d & 31) >> 3)) * 16;
}
__device__ __forceinline__ int vt_off(int key, int d) {  // byte offset of one bf16
  const int kk = key & 31, g = (kk & 15) >> 2, j = (kk >> 4) * 4 + (kk & 3);
  return ((key >> 5) * 4 + (d >> 4)) * 1024 + ((d & 15) + 16 * g) * 16 + j * 2;
}

struct AttnState {
  f32x4 acc[4];
  float m, den;
  bf16x8 qh[2], ql[2];
};

// One block of 32 keys (K: 4 chunks, Vt: 4 chunks; Kl/Vl: bf16 residual parts or null) for the wave's
// query tile; keys [klo, khi) of the block are valid (invalid keys hold finite values). Scores are scaled
// by qs (softmax scale x query RMS factor) and, when rk is set, by the key RMS factors rk[key]. Online
// fp32 softmax (src/mk_expert.py:196-251).
__device__ __forceinline__ void attn_block(AttnState& A, int lane, const char* K, const char* Kl, const char* V, const char* Vl,
                                           int klo, int khi, float qs, const float* rk) {
  // every LDS operand of the block is read up front (distinct registers), so the reads overlap each other
  // instead of each waiting for the MFMA before it
  bf16x8 kf[4], kl[4], vf[4], vl[4];
  f32x4 rkv[2] = {f32x4{1.f, 1.f, 1.f, 1.f}, f32x4{1.f, 1.f, 1.f, 1.f}};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    kf[i] = ldsfrag(K + i * 1024 + lane * 16);
    if (Kl) kl[i] = ldsfrag(Kl + i * 1024 + lane * 16);
  }
  // key RMS factors of the lane's 8 keys: 4 (lane / 16) + 0..3 and 16 + the same
  if (rk) {
    rkv[0] = *reinterpret_cast<const f32x4*>(rk + 4 * (lane >> 4));
    rkv[1] = *reinterpret_cast<const f32x4*>(rk + 16 + 4 * (lane >> 4));
  }
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    vf[dt] = ldsfrag(V + dt * 1024 + lane * 16);
    if (Vl) vl[dt] = ldsfrag(Vl + dt * 1024 + lane * 16);
  }
  f32x4 s[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    s[h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      s[h] = mfma16(kf[h * 2 + db], A.qh[db], s[h]);
      s[h] = mfma16(kf[h * 2 + db], A.ql[db], s[h]);
      if (Kl) s[h] = mfma16(kl[h * 2 + db], A.qh[db], s[h]);
    }
  }
  float pv[8];
  float mb = -INFINITY;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int key = (j >> 2) * 16 + 4 * (lane >> 4) + (j & 3);
    const float sc = qs * rkv[j >> 2][j & 3];
    pv[j] = s[j >> 2][j & 3] * sc + ((key >= klo && key < khi) ? 0.f : -INFINITY);
    mb = fmaxf(mb, pv[j]);
  }
  mb = xor32_max(xor16_max(mb));
  const float mn = fmaxf(A.m, mb);
  const float mu = mn == -INFINITY ? 0.f : mn;
  const float alpha = __expf(A.m - mu);
  A.m = mn;
  float ps = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    pv[j] = __expf(pv[j] - mu);
    ps += pv[j];
  }
  A.den = A.den * alpha + ps;
  bf16x8 ph, pl;
  split8(pv, ph, pl);
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    f32x4 a = A.acc[dt] * alpha;
    a = mfma16(vf[dt], ph, a);
    a = mfma16(vf[dt], pl, a);
    if (Vl) a = mfma16(vl[dt], ph, a);
    A.acc[dt] = a;
  }
}

// Two blocks of 32 bf16 keys (K0/V0 with keys [0, khi0) valid, K1/V1 with [0, khi1)) as one 64-key step of the
// online softmax: the two blocks' MFMA chains and softmax arithmetic are independent until the shared
// maximum, so their latencies overlap (the same result as two attn_block calls up to rounding).
__device__ __forceinline__ void attn_block2(AttnState& A, int lane, const char* K0, const char* V0, int khi0, const char* K1,
                                            const char* V1, int khi1, float qs) {
  bf16x8 kf[2][4], vf[2][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    kf[0][i] = ldsfrag(K0 + i * 1024 + lane * 16);
    kf[1][i] = ldsfrag(K1 + i * 1024 + lane * 16);
  }
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    vf[0][dt] = ldsfrag(V0 + dt * 1024 + lane * 16);
    vf[1][dt] = ldsfrag(V1 + dt * 1024 + lane * 16);
  }
  f32x4 s[2][2];
#pragma unroll
  for (int bk = 0; bk < 2; ++bk)
#pragma unroll
    for (int h = 0; h < 2; ++h) s[bk][h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int hl = 0; hl < 2; ++hl)
#pragma unroll
      for (int bk = 0; bk < 2; ++bk)
#pragma unroll
        for (int h = 0; h < 2; ++h) s[bk][h] = mfma16(kf[bk][h * 2 + db], hl ? A.ql[db] : A.qh[db], s[bk][h]);
  float pv[2][8];
  float mb = -INFINITY;
#pragma unroll
  for (int bk = 0; bk < 2; ++bk) {
    const int khi = bk ? khi1 : khi0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int key = (j >> 2) * 16 + 4 * (lane >> 4) + (j & 3);
      pv[bk][j] = s[bk][j >> 2][j & 3] * qs + (key < khi ? 0.f : -INFINITY);
      mb = fmaxf(mb, pv[bk][j]);
    }
  }
  mb = xor32_max(xor16_max(mb));
  const float mn = fmaxf(A.m, mb);
  const float mu = mn == -INFINITY ? 0.f : mn;
  const float alpha = __expf(A.m - mu);
  A.m = mn;
  float ps[2] = {0.f, 0.f};
#pragma unroll
  for (int bk = 0; bk < 2; ++bk)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      pv[bk][j] = __expf(pv[bk][j] - mu);
      ps[bk] += pv[bk][j];
    }
  A.den = A.den * alpha + (ps[0] + ps[1]);
  bf16x8 ph[2], pl[2];
  split8(pv[0], ph[0], pl[0]);
  split8(pv[1], ph[1], pl[1]);
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    f32x4 a = A.acc[dt] * alpha;
    a = mfma16(vf[0][dt], ph[0], a);
    a = mfma16(vf[1][dt], ph[1], a);
    a = mfma16(vf[0][dt], pl[0], a);
    a = mfma16(vf[1][dt], pl[1], a);
    A.acc[dt] = a;
  }
}

// attn_block for one block of 32 source keys (keys [0, khi) valid; no residual parts, no key factors) whose
// K and V^T fragments are already in registers: the fragments attn_block reads from LDS, in the same order, so
// the result is the same bits.
__device__ __forceinline__ void attn_block_rf(AttnState& A, int lane, const bf16x8 (&kf)[4], const bf16x8 (&vf)[4], int khi,
                                              float qs) {
  f32x4 s[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    s[h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      s[h] = mfma16(kf[h * 2 + db], A.qh[db], s[h]);
      s[h] = mfma16(kf[h * 2 + db], A.ql[db], s[h]);
    }
  }
  float pv[8];
  float mb = -INFINITY;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int key = (j >> 2) * 16 + 4 * (lane >> 4) + (j & 3);
    pv[j] = s[j >> 2][j & 3] * qs + ((key >= 0 && key < khi) ? 0.f : -INFINITY);
    mb = fmaxf(mb, pv[j]);
  }
  mb = xor32_max(xor16_max(mb));
  const float mn = fmaxf(A.m, mb);
  const float mu = mn == -INFINITY ? 0.f : mn;
  const float alpha = __expf(A.m - mu);
  A.m = mn;
  float ps = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    pv[j] = __expf(pv[j] - mu);
    ps += pv[j];
  }
  A.den = A.den * alpha + ps;
  bf16x8 ph, pl;
  split8(pv, ph, pl);
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    f32x4 a = A.acc[dt] * alpha;
    a = mfma16(vf[dt], ph, a);
    a = mfma16(vf[dt], pl, a);
    A.acc[dt] = a;
  }
}

// attn_block on K, V^T fragments and their residual parts already in registers, with the key RMS factors of
// the lane's 8 keys (the values attn_block reads from LDS, in the same order): the same bits.
__device__ __forceinline__ void attn_block_rfx(AttnState& A, int lane, const bf16x8 (&kf)[4], const bf16x8 (&kl)[4],
                                               const bf16x8 (&vf)[4], const bf16x8 (&vl)[4], int khi, float qs,
                                               const f32x4 (&rkv)[2]) {
  f32x4 s[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    s[h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      s[h] = mfma16(kf[h * 2 + db], A.qh[db], s[h]);
      s[h] = mfma16(kf[h * 2 + db], A.ql[db], s[h]);
      s[h] = mfma16(kl[h * 2 + db], A.qh[db], s[h]);
    }
  }
  float pv[8];
  float mb = -INFINITY;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int key = (j >> 2) * 16 + 4 * (lane >> 4) + (j & 3);
    const float sc = qs * rkv[j >> 2][j & 3];
    pv[j] = s[j >> 2][j & 3] * sc + ((key >= 0 && key < khi) ? 0.f : -INFINITY);
    mb = fmaxf(mb, pv[j]);
  }
  mb = xor32_max(xor16_max(mb));
  const float mn = fmaxf(A.m, mb);
  const float mu = mn == -INFINITY ? 0.f : mn;
  const float alpha = __expf(A.m - mu);
  A.m = mn;
  float ps = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    pv[j] = __expf(pv[j] - mu);
    ps += pv[j];
  }
  A.den = A.den * alpha + ps;
  bf16x8 ph, pl;
  split8(pv, ph, pl);
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    f32x4 a = A.acc[dt] * alpha;
    a = mfma16(vf[dt], ph, a);
    a = mfma16(vf[dt], pl, a);
    a = mfma16(vl[dt], ph, a);
    A.acc[dt] = a;
  }
}

// attn_block2 on K and V^T fragments already in registers (the fragments it reads from LDS, in the same order):
// the same bits.
__device__ __forceinline__ void attn_block2_rf(AttnState& A, int lane, const bf16x8 (&k0f)[4], const bf16x8 (&v0f)[4], int khi0,
                                               const bf16x8 (&k1f)[4], const bf16x8 (&v1f)[4], int khi1, float qs) {
  f32x4 s[2][2];
#pragma unroll
  for (int bk = 0; bk < 2; ++bk)
#pragma unroll
    for (int h = 0; h < 2; ++h) s[bk][h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int hl = 0; hl < 2; ++hl)
#pragma unroll
      for (int bk = 0; bk < 2; ++bk)
#pragma unroll
        for (int h = 0; h < 2; ++h) s[bk][h] = mfma16((bk ? k1f : k0f)[h * 2 + db], hl ? A.ql[db] : A.qh[db], s[bk][h]);
  float pv[2][8];
  float mb = -INFINITY;
#pragma unroll
  for (int bk = 0; bk < 2; ++bk) {
    const int khi = bk ? khi1 : khi0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int key = (j >> 2) * 16 + 4 * (lane >> 4) + (j & 3);
      pv[bk][j] = s[bk][j >> 2][j & 3] * qs + (key < khi ? 0.f : -INFINITY);
      mb = fmaxf(mb, pv[bk][j]);
    }
  }
  mb = xor32_max(xor16_max(mb));
  const float mn = fmaxf(A.m, mb);
  const float mu = mn == -INFINITY ? 0.f : mn;
  const float alpha = __expf(A.m - mu);
  A.m = mn;
  float ps[2] = {0.f, 0.f};
#pragma unroll
  for (int bk = 0; bk < 2; ++bk)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      pv[bk][j] = __expf(pv[bk][j] - mu);
      ps[bk] += pv[bk][j];
    }
  A.den = A.den * alpha + (ps[0] + ps[1]);
  bf16x8 ph[2], pl[2];
  split8(pv[0], ph[0], pl[0]);
  split8(pv[1], ph[1], pl[1]);
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    f32x4 a = A.acc[dt] * alpha;
    a = mfma16(v0f[dt], ph[0], a);
    a = mfma16(v1f[dt], ph[1], a);
    a = mfma16(v0f[dt], pl[0], a);
    a = mfma16(v1f[dt], pl[1], a);
    A.acc[dt] = a;
  }
}

__device__ __forceinline__ void attn_begin(AttnState& A, const char* Qh, const char* Ql, int lane) {
#pragma unroll
  for (int db = 0; db < 2; ++db) {
    A.qh[db] = ldsfrag(Qh + db * 1024 + lane * 16);
    A.ql[db] = ldsfrag(Ql + db * 1024 + lane * 16);
  }
  A.m = -INFINITY;
  A.den = 0.f;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) A.acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// merges the 4 waves' states (mrg: 18 KB of LDS) and stores the tile's output rows of head hd of sample b
// (split, written through; query rows >= M get zeros). Wave w finishes the 16-d slice dt = w. The states are
// exchanged lane-contiguously ([wave][dt][lane] accumulators, [wave][lane] maxima and denominators), so no
// LDS access has bank conflicts.
template <class S>
__device__ __forceinline__ void attn_merge_store(Ctx<S>& c, AttnState& A, float* mrg, float* y, int b, int hd, int qt) {
  f32x4* macc = reinterpret_cast<f32x4*>(mrg);  // [4 waves][4 dt][64 lanes]
  float* mm = mrg + NWAVES * 4 * 64 * 4;         // [4 waves][64 lanes]
  float* md = mm + NWAVES * 64;                  // [4 waves][64 lanes]
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) macc[(c.wave * 4 + dt) * 64 + c.lane] = A.acc[dt];
  mm[c.wave * 64 + c.lane] = A.m;
  md[c.wave * 64 + c.lane] = A.den;
  __syncthreads();
  float mw[NWAVES], mdv[NWAVES], M = -INFINITY;
  f32x4 ma[NWAVES];
#pragma unroll
  for (int w = 0; w < NWAVES; ++w) {
    mw[w] = mm[w * 64 + c.lane];
    mdv[w] = md[w * 64 + c.lane];
    ma[w] = macc[(w * 4 + c.wave) * 64 + c.lane];
  }
  lds_batch(mw);
  lds_batch(mdv);
  lds_batch(ma);
#pragma unroll
  for (int w = 0; w < NWAVES; ++w) M = fmaxf(M, mw[w]);
  float den = 0.f;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int w = 0; w < NWAVES; ++w) {
    const float f = mw[w] == -INFINITY ? 0.f : __expf(mw[w] - M);
    den += mdv[w] * f;
    acc += ma[w] * f;
  }
  den = xor32_sum(xor16_sum(den));
  const int q = qt * 16 + (c.lane & 15);
  const f32x4 out = (den > 0.f && q < c.p.Mq) ? acc * (1.0f / den) : f32x4{0.f, 0.f, 0.f, 0.f};
  if (st_h4(y, spiece(b * c.p.Mqp + q, hd * HD + c.wave * 16 + 4 * (c.lane >> 4), c.RT), out)) range_error(c.p.bar);
}

// Attention tasks: task u -> (sample-head hh, query tile qt), u in [0, nqt * nhb), placed (Params::pl) on
// workgroups that the stages before leave idle, so their prefetch of the attention operands overlaps those
// stages. Heads in complete groups of 8 are arranged so that the query tiles of one head run on one XCD
// (consecutive workgroups are on consecutive XCDs, so u % 8 is the XCD class) and share its L2; the
// remaining heads follow compactly.
// Where the tasks outnumber the G workgroups by X <= G (batched launches; Shape::RW_ATTN), the X
// workgroups that run two tasks run two query tiles of one sample-head, so that the second finds the head's
// keys and values (and, for self-attention, the sample's own rows) still staged in LDS: pair k < X is query
// tiles 2 j, 2 j + 1 of sample-head k % nhb (j = k / nhb), its first tile task k and its second task k + G
// (the same workgroup); tasks X .. G - 1 are the tiles in no pair, ordered by query tile, then sample-head.
struct AttnTask {
  int hh, qt;
  bool ok;
};
template <bool PAIRS>
__device__ __forceinline__ AttnTask attn_task(int u, int nqt, int nhb, int G) {
  AttnTask a;
  const int X = nqt * nhb - G;
  if (PAIRS && X > 0 && X <= G && X <= nhb * (nqt / 2) && u >= 0) {
    if (u < X) {
      a.hh = u % nhb;
      a.qt = 2 * (u / nhb);
    } else if (u >= G) {
      const int k = min(u - G, X - 1);
      a.hh = k % nhb;
      a.qt = 2 * (k / nhb) + 1;
    } else {
      // the r-th tile in no pair: the sample-heads m .. nhb - 1 of tiles 2 jf and 2 jf + 1 (the partly
      // paired tile pair), then every sample-head of the later tiles
      const int jf = X / nhb, m = X % nhb, r = u - X;
      if (m > 0 && r < 2 * (nhb - m)) {
        a.qt = 2 * jf + r / (nhb - m);
        a.hh = m + r % (nhb - m);
      } else {
        const int r2 = m > 0 ? r - 2 * (nhb - m) : r;
        a.qt = 2 * jf + (m > 0 ? 2 : 0) + r2 / nhb;
        a.hh = r2 % nhb;
      }
    }
    a.ok = u < G + X && a.qt < nqt;
    return a;
  }
  const int g8 = nhb & ~7, rem = nhb - g8;
  if (u < nqt * g8) {
    const int k = u >> 3;
    a.qt = k % nqt;
    a.hh = (u & 7) + 8 * (k / nqt);
  } else {
    const int r = u - nqt * g8;
    a.qt = rem ? r / rem : 0;
    a.hh = g8 + (rem ? r % rem : 0);
  }
  a.ok = u >= 0 && a.qt < nqt && a.hh < nhb;
  return a;
}
__device__ __forceinline__ int attn_count(int nqt, int nhb) { return nqt * nhb; }

template <class S>
__device__ __forceinline__ void sa_prefetch(Ctx<S>& c, int l, int b, int hd, int kvs) {
  const int PM = c.p.PM, PMP = ceil_to(PM, 32);
  char* memK = c.smem + S::WBUF;
  char* memVt = memK + PMP * 128;
  const bf16_t* mk = c.p.memk[l] + (long long)b * c.p.mem_sb;
  const bf16_t* mvt = c.p.memvt + ((long long)(l * c.p.B + b) * S::NH + hd) * PMP * 64;
  const int nk = (PMP / 16) * 2, nv = PMP / 8;
  for (int k = c.dw; k < nk + nv; k += c.dn) {
    if (k < nk) {
      // rows outside [kv_start, PM) are replaced by valid rows (they are masked): every operand is finite
      const int kt = k >> 1, db = k & 1;
      const int key = min(max(kt * 16 + (c.lane & 15), kvs), PM - 1);
      dma16(mk + ((long long)key * S::NH + hd) * HD + db * 32 + 8 * (c.lane >> 4), memK + k * 1024);
    } else {
      const int i = k - nk;
      dma16(mvt + (long long)i * 512 + c.lane * 8, memVt + i * 1024);
    }
  }
}

// Per-launch fp16 copy of every AdaRMS shift slice (step s, layer l, attention / cross-attention / MLP),
// the shift row tile of the fp16 GEMMs (rounded to nearest even, like the GEMM operands): one lane per
// (sample, 8-column group), 16 bytes in the first half of the group's 32-byte slot.
template <class S>
__device__ __forceinline__ void split_shifts(Ctx<S>& c) {
  CP& p = c.p;
  const int ngrp = p.n_steps * p.L * 3 * p.B * (S::H / 8);
  for (int k0 = c.wg * NTHREADS + c.tid; k0 < ngrp; k0 += c.G * NTHREADS * 4) {
    float v[4][8];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int k = min(k0 + u * c.G * NTHREADS, ngrp - 1);
      const int grp = k % (S::H / 8), r = k / (S::H / 8), b = r % p.B, r2 = r / p.B, kind = r2 % 3, sl = r2 / 3;
      const int l = sl % p.L, s = sl / p.L;
      const float* src = c.modrow(b, s) + 9 * l * S::H + 3 * kind * S::H + S::H + 8 * grp;
      const f32x4 a0 = ldf4(src), a1 = ldf4(src + 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) { v[u][j] = a0[j]; v[u][4 + j] = a1[j]; }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int k = k0 + u * c.G * NTHREADS;
      if (k < ngrp) {
        u32x4 h;
#pragma unroll
        for (int j = 0; j < 4; ++j) h[j] = cvt_pk_h(v[u][2 * j], v[u][2 * j + 1]);
        st_sc1(p.shs, (uint32_t)(k * 32), h);
      }
    }
  }
}

// Per-launch V^T copies of the memory and cross-attention V caches (the caches are constant over the
// Euler loop). Task (l, b, head, 32-key block): rows outside the valid range are replaced by valid rows.
template <class S>
__device__ __forceinline__ void transpose_caches(Ctx<S>& c, const int* s_ks) {
  CP& p = c.p;
  const int PMP = ceil_to(p.PM, 32), nmb = PMP / 32, ncb = p.SPP / 32;
  const int nm = p.L * p.B * S::NH * nmb, ntot = nm + p.L * p.B * S::NH * ncb;
  char* raw = c.smem + S::ABUF;  // [4 tasks][32 keys][64 d] bf16
  for (int t0 = c.wg * 4; t0 < ntot; t0 += c.G * 4) {
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = t0 + u;
      if (t < ntot) {
        const bool mem = t < nm;
        const int tt = mem ? t : t - nm, nb = mem ? nmb : ncb;
        const int kb = tt % nb, lbh = tt / nb, hd = lbh % S::NH, lb = lbh / S::NH, b = lb % p.B, l = lb / p.B;
        const int r = kb * 32 + (c.tid >> 3);
        int key;
        const bf16_t* src;
        if (mem) {
          key = min(max(r, s_ks[b]), p.PM - 1);
          src = p.memv[l] + (long long)b * p.mem_sb;
        } else {
          key = max(min(r, s_ks[MAX_BATCH + b] - 1), 0);
          src = p.vca[l] + (long long)b * p.src_sb;
        }
        *reinterpret_cast<u32x4*>(raw + u * 4096 + c.tid * 16) = ld16(src + ((long long)key * S::NH + hd) * HD + (c.tid & 7) * 8);
      }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = t0 + u;
      if (t < ntot) {
        const bool mem = t < nm;
        const int tt = mem ? t : t - nm;
        bf16_t* dst = (mem ? p.memvt : p.cavt) + (long long)tt * 2048;  // (l, b, head, block) blocks of 4 KB
        const int dt = c.tid >> 6, ln = c.tid & 63, dd = dt * 16 + (ln & 15), g = ln >> 4;
        u32x4 v;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int k0 = ((2 * q) >> 2) * 16 + 4 * g + ((2 * q) & 3), k1 = ((2 * q + 1) >> 2) * 16 + 4 * g + ((2 * q + 1) & 3);
          const uint32_t lo = *reinterpret_cast<const bf16_t*>(raw + u * 4096 + k0 * 128 + dd * 2);
          const uint32_t hi = *reinterpret_cast<const bf16_t*>(raw + u * 4096 + k1 * 128 + dd * 2);
          v[q] = lo | (hi << 16);
        }
        st_sc1(dst, (uint32_t)((dt * 64 + ln) * 16), v);
      }
    }
  }
}

// Self-attention stage: task (sample b, head hd, query tile qt). Queries = the tile's own rows; keys =
// memory rows [kv_start, PM) (bf16 cache, pre-normed and rotated, DMA'd during the barrier) || the
// sample's own rows (split q/k/v written by the QKV stage).
template <class S>
__device__ __forceinline__ void sa_stage(Ctx<S>& c, const Desc& d, const int* s_ks, BarCtx& bc, int g) {
  CP& p = c.p;
  const int M = p.Mq, Mqp = p.Mqp, PM = p.PM, PMP = ceil_to(PM, 32), NOWN32 = ceil_to(M, 32);
  const int NQT = Mqp / 16, NKT = NOWN32 / 16, KBO = NOWN32 / 32, NRP = p.NRP, RT = c.RT;
  const int l = d.l;
  char* fr = c.frame(d.s, l);
  const char* qs = fr + S::qs_off(NRP);
  const char* ks = fr + S::ks_off(NRP);
  const char* vt = fr + S::vtb_off(NRP);
  const float* ssqk = (const float*)(fr + S::ssqk_off(NRP));
  float* ysa = (float*)(fr + S::ysa_off(NRP));
  char* memK = c.smem + S::WBUF;
  char* memVt = memK + PMP * 128;
  char* Qh = c.smem + S::ABUF;
  char* Ql = Qh + 2048;
  char* Kh = Ql + 2048;
  char* Kl = Kh + NOWN32 * 128;
  char* Vh = Kl + NOWN32 * 128;
  char* Vl = Vh + NOWN32 * 128;
  float* rk = (float*)(Vl + NOWN32 * 128);
  float* mrg = rk + 128;
  const int NHB = p.B * S::NH;
  const bool want_kv = (d.s == 0 && p.cur_k != nullptr && p.R > 0);
  const int u0 = task_first(c, PL_SA);
  int prev_hh = -1;
  for (int v = u0; v < attn_count(NQT, NHB); v += c.G) {
    const AttnTask at = attn_task<S::RW_ATTN>(v, NQT, NHB, c.G);
    if (!at.ok) continue;
    const int b = at.hh / S::NH, hd = at.hh % S::NH, qt = at.qt;
    const int kvs = s_ks[b];
    // a second query tile of the sample-head just done: its memory rows, own keys and values (and their RMS
    // factors) are still in LDS, and the QKV tasks it waits for have already been waited for
    const bool resident = S::RW_ATTN && at.hh == prev_hh;
    prev_hh = at.hh;
    if (v != u0) {
      wait_vm0();
      __syncthreads();
      if (!resident) sa_prefetch(c, l, b, hd, kvs);
    }
    // the QKV tasks of this head (q, k, v x two column pairs, every row group): the rows' sums of squares
    // and V^T blocks of one head interleave row groups within cache lines
    if (!resident) {
      const int rgq = p.rgs_qkv;
      flag_wait<1>(bc, F_QKV, 6 * rgq, [&](int i) {
        const int k = i % 6, rg = i / 6;
        return rg * 6 * S::NH + (k >> 1) * 2 * S::NH + 2 * hd + (k & 1);
      }, (unsigned long long)g);
    }
    MKX_TR(c, 0);
    // The query rows' sums of squares (two column halves; DMA'd into the merge area, read before the merge
    // reuses it), then the own-row operands: each wave's next DMA is a piece of the Q tile (hi, lo), then K
    // tiles of all own keys and V^T blocks. All are DMAs, so one counted wait covers the first phase.
    float* sq_l = mrg;
    if (c.wave == 0) {
      const int qq = qt * 16 + (c.lane & 15), j = (c.lane >> 4) & 1;
      __builtin_amdgcn_global_load_lds(ssqk + (long long)(hd * 2 + j) * NRP + b * Mqp + qq, (lds_void*)sq_l, 4, 0, 0);
    }
    const int rt0 = b * Mqp / 16;
    // (SA_REG: only the Q tile goes through LDS; each wave loads its own-key block itself below)
    const bool reg = S::SA_REG && !want_kv;
    for (int k = c.wave; k < (resident || reg ? 4 : 4 + 4 * NKT + 8 * KBO); k += NWAVES) {
      if (k < 4) {
        const int db = k >> 1, part = k & 1;
        dma16(qs + ((long long)((2 * hd + db) * RT + rt0 + qt) * 2 + part) * 1024 + c.lane * 16, (part ? Ql : Qh) + db * 1024);
      } else if (k < 4 + 4 * NKT) {
        const int kk = k - 4, kt = kk >> 2, db = (kk >> 1) & 1, part = kk & 1;
        const int rtk = rt0 + min(kt, NQT - 1);
        dma16(ks + ((long long)((2 * hd + db) * RT + rtk) * 2 + part) * 1024 + c.lane * 16, (part ? Kl : Kh) + (kt * 2 + db) * 1024);
      } else {
        const int vv = k - 4 - 4 * NKT;
        dma16(vt + ((long long)at.hh * KBO * 8 + vv) * 1024 + c.lane * 16, ((vv & 1) ? Vl : Vh) + (vv >> 1) * 1024);
      }
    }
    // RMS factors of the own keys (threads < NOWN32; the others load a valid row and discard it). Loaded with
    // no branch and summed only after the own-key wait, so that nothing waits for these loads earlier.
    const int rowk = b * Mqp + min(c.tid, Mqp - 1);
    const float ssk0 = ssqk[(long long)((S::NH + hd) * 2) * NRP + rowk];
    const float ssk1 = ssqk[(long long)((S::NH + hd) * 2 + 1) * NRP + rowk];
    // The memory blocks need only the Q tile and the memory K/V (prefetched before it): every wave issued at
    // least 4 own-key DMAs after its Q piece (M >= 1 gives NKT >= 2 and KBO >= 1, 20 DMAs over 4 waves), so
    // at most 4 outstanding operations means its Q piece has landed (a resident tile loads only its Q tile).
    if (resident || reg) wait_vm0();
    else wait_vm_le<4>();
    exec_barrier();
    MKX_TR(c, 1);
    AttnState A;
    attn_begin(A, Qh, Ql, c.lane);
    const float ssq = sq_l[c.lane & 15] + sq_l[16 + (c.lane & 15)];
    const float qsc = p.sm_scale * rsqrtf(ssq / 64.f + p.qk_eps);
    const int mb0 = kvs >> 5, nmb = PMP / 32 - mb0;
    // SA_REG: this wave's own-key block jo (blocks continue the round-robin over the waves after the memory
    // blocks; at most one per wave, NOWN32 <= 128): its K and V^T chunks (the ones the DMAs above would have
    // put in LDS for it) and the RMS factors of the lane's 8 keys, issued now so that they land during the
    // memory blocks
    const int jo = ((c.wave - nmb) % NWAVES + NWAVES) % NWAVES;
    bf16x8 okh[4], okl[4], ovh[4], ovl[4];
    float ssa[8], ssb[8];
    if (S::SA_REG && reg && jo < KBO) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kt = 2 * jo + (i >> 1), db = i & 1;
        const int rtk = rt0 + min(kt, NQT - 1);
        const char* kp = ks + ((long long)((2 * hd + db) * RT + rtk) * 2) * 1024 + c.lane * 16;
        okh[i] = __builtin_bit_cast(bf16x8, ld16(kp));
        okl[i] = __builtin_bit_cast(bf16x8, ld16(kp + 1024));
        const char* vp = vt + ((long long)at.hh * KBO * 8 + 2 * (jo * 4 + i)) * 1024 + c.lane * 16;
        ovh[i] = __builtin_bit_cast(bf16x8, ld16(vp));
        ovl[i] = __builtin_bit_cast(bf16x8, ld16(vp + 1024));
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int key = jo * 32 + (e >> 2) * 16 + 4 * (c.lane >> 4) + (e & 3);
        const int row = b * Mqp + min(key, Mqp - 1);
        ssa[e] = ssqk[(long long)((S::NH + hd) * 2) * NRP + row];
        ssb[e] = ssqk[(long long)((S::NH + hd) * 2 + 1) * NRP + row];
      }
    }
    for (int beta = c.wave; beta < nmb; beta += NWAVES) {
      const int kb = mb0 + beta;
      attn_block(A, c.lane, memK + kb * 4096, nullptr, memVt + kb * 4096, nullptr, kvs - kb * 32, PM - kb * 32, qsc, nullptr);
    }
    if (S::SA_REG && reg) {
      if (jo < KBO) {
        // the lane's key factors, and zero V for own keys beyond the sample's rows (no producer): element j of
        // a V^T fragment is key (j / 4) 16 + 4 (lane / 16) + j % 4 of the block
        f32x4 rkv[2];
#pragma unroll
        for (int e = 0; e < 8; ++e) rkv[e >> 2][e & 3] = rsqrtf((ssa[e] + ssb[e]) / 64.f + p.qk_eps);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          u32x4 hv = __builtin_bit_cast(u32x4, ovh[dt]), lv = __builtin_bit_cast(u32x4, ovl[dt]);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int key = jo * 32 + (j >> 2) * 16 + 4 * (c.lane >> 4) + (j & 3);
            if (key >= Mqp) {
              const uint32_t keep = (j & 1) ? 0x0000ffffu : 0xffff0000u;
              hv[j >> 1] &= keep;
              lv[j >> 1] &= keep;
            }
          }
          ovh[dt] = __builtin_bit_cast(bf16x8, hv);
          ovl[dt] = __builtin_bit_cast(bf16x8, lv);
        }
        attn_block_rfx(A, c.lane, okh, okl, ovh, ovl, M - jo * 32, qsc, rkv);
      }
    } else {
      if (!resident) {
        wait_vm0();  // the own keys' K and V^T have landed
        __syncthreads();
        if (c.tid < NOWN32) rk[c.tid] = rsqrtf((ssk0 + ssk1) / 64.f + p.qk_eps);
        // own keys beyond the sample's rows have no producer: zero their V
        for (int it = c.tid; it < (NOWN32 - Mqp) * HD; it += NTHREADS) {
          const int key = Mqp + it / HD, dd = it % HD;
          *reinterpret_cast<bf16_t*>(Vh + vt_off(key, dd)) = 0;
          *reinterpret_cast<bf16_t*>(Vl + vt_off(key, dd)) = 0;
        }
        __syncthreads();
      }
      // own-key blocks continue the round-robin over the waves (block beta on wave beta % 4)
      for (int beta = nmb + ((c.wave - nmb) % NWAVES + NWAVES) % NWAVES; beta < nmb + KBO; beta += NWAVES) {
        const int kb = beta - nmb;
        attn_block(A, c.lane, Kh + kb * 4096, Kl + kb * 4096, Vh + kb * 4096, Vl + kb * 4096, 0, M - kb * 32, qsc, rk + kb * 32);
      }
    }
    MKX_TR(c, 2);
    // every wave has read the query rows' sums of squares (sq_l, in the merge area) before the merge writes
    // there (the own-key barriers above order them otherwise)
    if (resident || (S::SA_REG && reg)) exec_barrier();
    attn_merge_store(c, A, mrg, ysa, b, hd, qt);
    if (want_kv && qt == 0) {
      // register rows' k (normed, rotated) and v of step 1, bf16 [L][B][R][NH][64] (src/mk_expert.py:440-470)
      for (int it = c.tid; it < p.R * 8; it += NTHREADS) {
        const int i = p.T + it / 8, dd = (it % 8) * 8;
        bf16x8 kh = ldsfrag(Kh + kchunk_off(i, dd)), kl = ldsfrag(Kl + kchunk_off(i, dd));
        const u32x4 khu = __builtin_bit_cast(u32x4, kh), klu = __builtin_bit_cast(u32x4, kl);
        float kf[8], kr[8], vf[8];
        unpack8(khu, kf);
        unpack8(klu, kr);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          kf[e] = (kf[e] + kr[e]) * rk[i];
          vf[e] = bf2f(*reinterpret_cast<const bf16_t*>(Vh + vt_off(i, dd + e))) +
                  bf2f(*reinterpret_cast<const bf16_t*>(Vl + vt_off(i, dd + e)));
        }
        const long long o = ((((long long)l * p.B + b) * p.R + (i - p.T)) * S::NH + hd) * HD + dd;
        u32x4 wk, wv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          wk[e] = cvt_pk(kf[2 * e], kf[2 * e + 1]);
          wv[e] = cvt_pk(vf[2 * e], vf[2 * e + 1]);
        }
        *reinterpret_cast<u32x4*>(p.cur_k + o) = wk;
        *reinterpret_cast<u32x4*>(p.cur_v + o) = wv;
      }
    }
    flag_publish(bc, F_SA, at.hh * NQT + qt, (unsigned long long)g + 1);
  }
}

// Cross-attention stage: task (sample b, head hd, 16-query tile qt).
//  1. Query projection of the tile's rows for the head (src/mk_expert.py:373-378): q = rstd(h2) (y2 Wq^T) +
//     shift Wq^T over the head's 64 columns (y2 = h2 (1 + scale) split, rows of the tile; the shift row
//     tile as in the GEMM stages), then, with whole head rows in the workgroup, the q norm, its weight and
//     RoPE (:175-193), split into the Q chunks.
//  2. Attention over the valid source rows (:225-251): K and V^T streamed in chunks of 128 rows through a
//     3-slot LDS ring (32 KB per slot: 16 K chunks, then 16 V^T chunks from the per-launch copy); the first
//     three chunks are DMA'd during the barrier. Wave w takes each chunk's 32-row block w; the waves'
//     softmax states are merged at the end.
template <class S>
__device__ __forceinline__ char* ca_slot(Ctx<S>& c, int cc) {
  const int sl = cc % 3;
  return c.smem + (sl < 2 ? S::WBUF + sl * 32768 : S::ABUF);
}

template <class S>
__device__ __forceinline__ void ca_dma_chunk(Ctx<S>& c, int l, int b, int hd, int cc, int S_len) {
  char* slot = ca_slot(c, cc);
  const bf16_t* kb_ = c.p.kca[l] + (long long)b * c.p.src_sb;
  const int ncb = c.p.SPP / 32;
  const bf16_t* vt = c.p.cavt + ((long long)(l * c.p.B + b) * S::NH + hd) * ncb * 2048;
  // 32-key blocks that start beyond the valid length are not loaded (no wave reads them); within a partly
  // valid block, rows beyond the length are replaced by the last valid row (they are masked)
  for (int k = c.dw; k < 32; k += c.dn) {
    if (k < 16) {
      const int kt = k >> 1, db = k & 1;
      if (cc * 128 + (kt >> 1) * 32 >= S_len) continue;
      const int key = min(cc * 128 + kt * 16 + (c.lane & 15), S_len - 1);
      dma16(kb_ + ((long long)key * S::NH + hd) * HD + db * 32 + 8 * (c.lane >> 4), slot + k * 1024);
    } else {
      const int i = k - 16, kb = cc * 4 + (i >> 2);
      if (kb * 32 >= S_len) continue;
      dma16(vt + ((long long)kb * 4 + (i & 3)) * 512 + c.lane * 8, slot + 16384 + i * 1024);
    }
  }
}

template <class S>
__device__ __forceinline__ void ca_prefetch(Ctx<S>& c, int l, int b, int hd, int S_len) {
  const int nch = (S_len + 127) / 128;
  for (int cc = 0; cc < min(nch, 3); ++cc) ca_dma_chunk(c, l, b, hd, cc, S_len);
}

template <class S>
__device__ __forceinline__ void ca_stage(Ctx<S>& c, const Desc& d, const int* s_ks, BarCtx& bc, int g) {
  CP& p = c.p;
  constexpr int KPW = S::KPW;
  const int Mqp = p.Mqp, NQT = Mqp / 16, NRP = p.NRP, RT = c.RT;
  const int l = d.l;
  char* fr = c.frame(d.s, l);
  const float* y2 = (const float*)(fr + S::y2_off(NRP));
  const float* ss2 = (const float*)(fr + S::ss2_off(NRP));
  float* yca = (float*)(fr + S::yca_off(NRP));
  const char* wq = p.wqca + l * p.s_o;
  const char* shs = p.shs + ((long long)(d.s * p.L + l) * 3 + 1) * p.B * S::H * 4;
  // [wave][4 column tiles][q, shift][68 slots] x 16 bytes: lane L at slot L + L / 16, so that the
  // transposed reads of the finishing step fall in distinct banks
  char* red = c.smem + S::ABUF + 32768;
  char* Qh = c.smem + S::ABUF + 32768 + NWAVES * 4 * 2 * 68 * 16;
  char* Ql = Qh + 2048;
  float* mrg = (float*)(Ql + 2048);
  static_assert(32768 + NWAVES * 4 * 2 * 68 * 16 + 4096 + NWAVES * 64 * 18 * 4 <= S::ABUF_BYTES, "cross-attention LDS map");
  float* ssw = (float*)(c.smem + S::SMALL);  // [4 waves][16 rows]
  const int NHB = p.B * S::NH;
  const uint32_t vlane = (uint32_t)c.lane * 16;
  const int cnt = attn_count(NQT, NHB), u0 = task_first(c, PL_CA);
  // The operands that do not depend on the stage before, the Wq fragments of the task's head and the shift
  // fragments (an MFMA row tile whose rows are the samples), are loaded before the barrier completes: the
  // workgroups running this stage are idle in the stage before. (Loads only: the waves that do not poll the
  // barrier reach it without waiting for them.)
  f16x8 wf[4][KPW], sh[KPW];
  auto pre = [&](int hd) {
    const __amdgpu_buffer_rsrc_t rsh =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(shs), (short)0, p.B * S::H * 4, 0x00020000);
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      const int kb = c.wave + NWAVES * i;
      // lane l reads sample l % 16; samples >= B fall outside the buffer and read zeros
      const uint32_t o = (uint32_t)((((c.lane & 15) * S::NKB + kb) * 4 + (c.lane >> 4)) * 32);
      sh[i] = __builtin_bit_cast(f16x8, bload(rsh, o, 0));
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
        wf[nt][i] = wfrag_glb<S>(wq + ((long long)(hd * 4 + nt) * S::NKB + kb) * S::CH, c.lane);
    }
  };
  // (wave 0 too, although its poll then completes only after these loads: the workgroups of this stage
  // enter it two stages before their operands are ready, which leaves the loads several microseconds)
  if (u0 < cnt) pre(attn_task<S::RW_ATTN>(u0, NQT, NHB, c.G).hh % S::NH);
  const int rgo = p.rgs_o;
  int prev_hh = -1;
  for (int v = u0; v < cnt; v += c.G) {
    const AttnTask at = attn_task<S::RW_ATTN>(v, NQT, NHB, c.G);
    if (!at.ok) continue;
    const int b = at.hh / S::NH, hd = at.hh % S::NH, qt = at.qt;
    const int S_len = s_ks[MAX_BATCH + b];
    const int nch = (S_len + 127) / 128;
    // a second query tile of the sample-head just done finds its source keys and values still in the ring
    // when every chunk was resident (at most 3)
    const bool resident = S::RW_ATTN && at.hh == prev_hh && nch <= 3;
    prev_hh = at.hh;
    if (v != u0) {
      wait_vm0();
      __syncthreads();
      if (!S::CA_LATE && !resident && !(S::CA_REG && nch <= 3)) ca_prefetch(c, l, b, hd, S_len);
      pre(hd);
    }
    const int rq = b * Mqp / 16 + qt;  // row tile of the query rows
    // step 1b item of this lane: row r = 4 wave + lane / 16 of the tile, columns 4 cg .. 4 cg + 3 of the
    // head; its RoPE, norm weight (and fp8 scale) constants are loaded before the wait
    const int r = 4 * c.wave + (c.lane >> 4), cg = c.lane & 15;
    const int pos = min(qt * 16 + r, p.Mq - 1);
    const f32x4 cs = ldf4(p.ca_cos + pos * HD + 4 * cg), sn = ldf4(p.ca_sin + pos * HD + 4 * cg);
    const uint2 wn = *reinterpret_cast<const uint2*>(p.qcan + l * HD + 4 * cg);
    const f32x4 scq = S::W8 ? ldf4(p.sc_qca + (long long)l * S::H + hd * HD + 4 * cg) : f32x4{1.f, 1.f, 1.f, 1.f};
    // shift Wq^T: both are inputs of the call, so it is computed before the wait (and the shift fragments'
    // registers are free again before the query rows are loaded)
    f32x4 accb[4][2];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) accb[nt][0] = accb[nt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < KPW; ++i)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) accb[nt][i & 1] = mfma16h(wf[nt][i], sh[i], accb[nt][i & 1]);
    MKX_TR(c, 14);
    // every out-projection task of the row group holding the query rows
    {
      const int rg = row_group_of(rq, RT, rgo);
      const int to = S::HT / p.nt_o;  // out-projection tasks per row group
      flag_wait<1>(bc, F_O, to, [&](int i) { return rg * to + i; }, (unsigned long long)g);
    }
    MKX_TR(c, 0);
    // 1a. operands: sums of squares (first, so that waiting for them never waits for the query rows), then
    // the y2 fragments (fp16) of the query rows
    f16x8 yh[KPW];
    u32x2 ssv[S::HT / 8];
    {
      const __amdgpu_buffer_rsrc_t rs_ = rsrc(ss2);
      const uint32_t so = ss_slot<S::HT>(rq * 16 + (c.lane & 15), c.wave * (S::HT / 4));
#pragma unroll
      for (int i = 0; i < S::HT / 8; ++i) ssv[i] = bload8(rs_, so, (uint32_t)i * 128);
      const __amdgpu_buffer_rsrc_t ry = rsrc(y2);
#pragma unroll
      for (int i = 0; i < KPW; ++i) {
        const int kb = c.wave + NWAVES * i;
        yh[i] = __builtin_bit_cast(f16x8, bload(ry, vlane, (uint32_t)((kb * RT + rq) * 2048)));
      }
    }
    // Everything but the query rows has landed (the prefetched K/V chunks were issued before them); the
    // query rows are waited for where the MFMAs use them.
    // In the row-wise form every workgroup is busy in the stage before, so loads issued ahead of the poll
    // hold it up (they return in issue order): with CA_LATE the K/V chunks are DMA'd only now, after the
    // query rows have landed, and arrive during the query projection.
    if constexpr (S::CA_LATE) {
      wait_vm0();
      if (!resident) ca_prefetch(c, l, b, hd, S_len);
    } else {
      wait_vm_le<KPW>();
    }
    __builtin_amdgcn_sched_barrier(0);  // every query-row load is issued before the first MFMA
    MKX_TR(c, 3);
    {
      // [column tile][k-block parity]: 8 independent accumulation chains
      f32x4 acc[4][2];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) acc[nt][0] = acc[nt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < KPW; ++i)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) acc[nt][i & 1] = mfma16h(wf[nt][i], yh[i], acc[nt][i & 1]);
      const float ssp = ss_pairs_sum<S::HT / 8>(ssv);
      if (c.lane < 16) ssw[c.wave * 16 + c.lane] = ssp;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int sl = c.lane + (c.lane >> 4);
        sts16(red + (((c.wave * 4 + nt) * 2 + 0) * 68 + sl) * 16, as_u4(acc[nt][0] + acc[nt][1]));
        sts16(red + (((c.wave * 4 + nt) * 2 + 1) * 68 + sl) * 16, as_u4(accb[nt][0] + accb[nt][1]));
      }
    }
    // (CA_REG, at most three chunks) this wave's source blocks w, w + 4 and w + 8 into registers: the fragments
    // the LDS ring would hold for it, loaded once the query projection's MFMAs have freed their registers, while
    // the projection is finished
    bf16x8 kvk[3][4], kvv[3][4];
    if (S::CA_REG && nch <= 3) {
      const bf16_t* kb_ = p.kca[l] + (long long)b * p.src_sb;
      const int ncb = p.SPP / 32;
      const bf16_t* vt = p.cavt + ((long long)(l * p.B + b) * S::NH + hd) * ncb * 2048;
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const int kbl = min(j * 4 + c.wave, ncb - 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = min(j * 128 + (2 * c.wave + (i >> 1)) * 16 + (c.lane & 15), max(S_len - 1, 0));
          kvk[j][i] = __builtin_bit_cast(bf16x8, ld16(kb_ + ((long long)key * S::NH + hd) * HD + (i & 1) * 32 + 8 * (c.lane >> 4)));
        }
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) kvv[j][dt] = __builtin_bit_cast(bf16x8, ld16(vt + ((long long)kbl * 4 + dt) * 512 + c.lane * 8));
      }
    }
    __syncthreads();
    MKX_TR(c, 7);
    {
      // 1b. q of row r, columns 4 cg .. 4 cg + 3 (accumulator lane r + 16 (cg % 4) of column tile cg / 4)
      const int nt = cg >> 2, lr = r + 16 * (cg & 3), lb = b + 16 * (cg & 3);
      f32x4 qa[NWAVES], ba[NWAVES];
      float sw[NWAVES];
#pragma unroll
      for (int w = 0; w < NWAVES; ++w) {
        qa[w] = ldf4((const float*)(red + (((w * 4 + nt) * 2 + 0) * 68 + lr + (lr >> 4)) * 16));
        ba[w] = ldf4((const float*)(red + (((w * 4 + nt) * 2 + 1) * 68 + lb + (lb >> 4)) * 16));
        sw[w] = ssw[16 * w + r];
      }
      lds_batch(qa);
      lds_batch(ba);
      lds_batch(sw);
      f32x4 qv = qa[0];
      float bv[4] = {ba[0][0], ba[0][1], ba[0][2], ba[0][3]};
#pragma unroll
      for (int w = 1; w < NWAVES; ++w) {
        qv += qa[w];
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[e] += ba[w][e];
      }
      const float rs = rsqrtf((sw[0] + sw[1] + sw[2] + sw[3]) * (1.0f / (float)S::H) + p.eps);
      f32x4 x;
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = (qv[e] * rs + bv[e]) * scq[e];
      // q norm over the head's 64 columns (the 16 lanes of the row), weight 1 + w, rotate-half RoPE with the
      // partner column d +- 32 on lane ^ 8
      float ss = x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
      ss = row_sum16(ss);
      const float rn = rsqrtf(ss / 64.f + p.qk_eps);
      const f32x4 gw = {1.0f + __uint_as_float(wn.x << 16), 1.0f + __uint_as_float(wn.x & 0xffff0000u),
                        1.0f + __uint_as_float(wn.y << 16), 1.0f + __uint_as_float(wn.y & 0xffff0000u)};
      const f32x4 xn = x * rn * gw;
      const float sgn = cg < 8 ? -1.0f : 1.0f;
      f32x4 u;
#pragma unroll
      for (int e = 0; e < 4; ++e) u[e] = xn[e] * cs[e] + sgn * lane_xor8(xn[e]) * sn[e];
      // Q chunk layout (row r, d = 4 cg): lane r + 16 ((d % 32) / 8), half (d % 8) / 4
      const int dd = 4 * cg;
      const int off = (dd >> 5) * 1024 + (r + 16 * ((dd & 31) >> 3)) * 16 + (dd & 4) * 2;
      u32x2 hi, lo;
      hi[0] = cvt_pk(u[0], u[1]);
      hi[1] = cvt_pk(u[2], u[3]);
      lo[0] = cvt_pk(u[0] - __uint_as_float(hi[0] << 16), u[1] - __uint_as_float(hi[0] & 0xffff0000u));
      lo[1] = cvt_pk(u[2] - __uint_as_float(hi[1] << 16), u[3] - __uint_as_float(hi[1] & 0xffff0000u));
      *reinterpret_cast<u32x2*>(Qh + off) = hi;
      *reinterpret_cast<u32x2*>(Ql + off) = lo;
    }
    if constexpr (S::CA_LATE) wait_vm0();  // this wave's K/V DMAs (the barrier covers the other waves')
    __syncthreads();
    MKX_TR(c, 1);
    AttnState A;
    attn_begin(A, Qh, Ql, c.lane);
    if (S::CA_REG && nch <= 3) {
      // the same blocks from registers
      const int k0 = c.wave * 32, k1 = 128 + c.wave * 32, k2 = 256 + c.wave * 32;
      if (k1 < S_len)
        attn_block2_rf(A, c.lane, kvk[0], kvv[0], S_len - k0, kvk[1], kvv[1], S_len - k1, p.sm_scale);
      else if (k0 < S_len)
        attn_block_rf(A, c.lane, kvk[0], kvv[0], S_len - k0, p.sm_scale);
      if (k2 < S_len) attn_block_rf(A, c.lane, kvk[2], kvv[2], S_len - k2, p.sm_scale);
    } else if (nch <= 3) {
      // every chunk is resident: wave w's 32-key blocks w, w + 4 (one 64-key step) and w + 8
      const int k0 = c.wave * 32, k1 = 128 + c.wave * 32, k2 = 256 + c.wave * 32;
      char* s0 = ca_slot(c, 0);
      char* s1 = ca_slot(c, 1);
      char* s2 = ca_slot(c, 2);
      if (k1 < S_len)
        attn_block2(A, c.lane, s0 + c.wave * 4096, s0 + 16384 + c.wave * 4096, S_len - k0, s1 + c.wave * 4096,
                    s1 + 16384 + c.wave * 4096, S_len - k1, p.sm_scale);
      else if (k0 < S_len)
        attn_block(A, c.lane, s0 + c.wave * 4096, nullptr, s0 + 16384 + c.wave * 4096, nullptr, 0, S_len - k0, p.sm_scale, nullptr);
      if (k2 < S_len)
        attn_block(A, c.lane, s2 + c.wave * 4096, nullptr, s2 + 16384 + c.wave * 4096, nullptr, 0, S_len - k2, p.sm_scale, nullptr);
    }
    if constexpr (S::LONG) {
      if (nch > 3) {
        // chunks 0-2 from the LDS ring (DMA'd before the stage); the later chunks streamed into registers,
        // each wave loading only its own 32-key block of a chunk (the fragments attn_block would read from the
        // ring, from the addresses ca_dma_chunk copies) one chunk ahead of its use: no ring refills and no
        // barriers between chunks. Blocks in the same order with the same arithmetic: the same bits.
        const bf16_t* kb_ = p.kca[l] + (long long)b * p.src_sb;
        const int ncb = p.SPP / 32;
        const bf16_t* vt = p.cavt + ((long long)(l * p.B + b) * S::NH + hd) * ncb * 2048;
        bf16x8 kn[4], vn[4];
        // wave w's block of chunk cc: K chunks 4 w + i of the ring (key tile 2 w + i / 2, d-block i % 2), V^T
        // block 4 cc + w; rows beyond the length repeat the last valid one and blocks beyond it are not used
        auto load_block = [&](int cc) {
          const int kbl = min(cc * 4 + c.wave, ncb - 1);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = min(cc * 128 + (2 * c.wave + (i >> 1)) * 16 + (c.lane & 15), S_len - 1);
            kn[i] = __builtin_bit_cast(bf16x8, ld16(kb_ + ((long long)key * S::NH + hd) * HD + (i & 1) * 32 + 8 * (c.lane >> 4)));
          }
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) vn[dt] = __builtin_bit_cast(bf16x8, ld16(vt + ((long long)kbl * 4 + dt) * 512 + c.lane * 8));
        };
        // one chunk in flight ahead of the one in use (two measured slower)
        load_block(3);
        for (int cc = 0; cc < 3; ++cc) {
          char* slot = ca_slot(c, cc);
          const int k0 = cc * 128 + c.wave * 32;  // (< S_len: more than three chunks)
          attn_block(A, c.lane, slot + c.wave * 4096, nullptr, slot + 16384 + c.wave * 4096, nullptr, 0, S_len - k0, p.sm_scale, nullptr);
        }
        for (int cc = 3; cc < nch; ++cc) {
          bf16x8 kc[4], vc[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            kc[i] = kn[i];
            vc[i] = vn[i];
          }
          if (cc + 1 < nch) load_block(cc + 1);
          const int k0 = cc * 128 + c.wave * 32;
          if (k0 < S_len) attn_block_rf(A, c.lane, kc, vc, S_len - k0, p.sm_scale);
        }
      }
    } else {
      for (int cc = 0; nch > 3 && cc < nch; ++cc) {
        if (cc >= 3) {
          // chunk cc was issued three iterations ago; the younger chunks cc + 1, cc + 2 may still be in
          // flight: 8 DMAs per wave each, except the last chunk, which may issue fewer
          if (cc + 2 < nch - 1) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
          else if (cc + 1 < nch - 1) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
          else wait_vm0();
          __syncthreads();
        }
        char* slot = ca_slot(c, cc);
        const int k0 = cc * 128 + c.wave * 32;
        if (k0 < S_len)
          attn_block(A, c.lane, slot + c.wave * 4096, nullptr, slot + 16384 + c.wave * 4096, nullptr, 0, S_len - k0, p.sm_scale, nullptr);
        if (cc + 3 < nch) {
          __syncthreads();
          ca_dma_chunk(c, l, b, hd, cc + 3, S_len);
        }
      }
    }
    MKX_TR(c, 2);
    attn_merge_store(c, A, mrg, yca, b, hd, qt);
    MKX_TR(c, 13);
    flag_publish(bc, F_CA, at.hh * NQT + qt, (unsigned long long)g + 1);
  }
}

// One block of 32 source keys (keys [0, khi) valid) for NQ query tiles at once: the block's K and V^T
// fragments are read once, each state's chains are those of attn_block (no residual parts, no key factors).
template <int NQ>
__device__ __forceinline__ void attn_block_n(AttnState (&A)[NQ], int lane, const char* K, const char* V, int khi, float qs) {
  bf16x8 kf[4], vf[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) kf[i] = ldsfrag(K + i * 1024 + lane * 16);
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) vf[dt] = ldsfrag(V + dt * 1024 + lane * 16);
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    f32x4 s[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      s[h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        s[h] = mfma16(kf[h * 2 + db], A[q].qh[db], s[h]);
        s[h] = mfma16(kf[h * 2 + db], A[q].ql[db], s[h]);
      }
    }
    float pv[8];
    float mb = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int key = (j >> 2) * 16 + 4 * (lane >> 4) + (j & 3);
      pv[j] = s[j >> 2][j & 3] * qs + ((key >= 0 && key < khi) ? 0.f : -INFINITY);
      mb = fmaxf(mb, pv[j]);
    }
    mb = xor32_max(xor16_max(mb));
    const float mn = fmaxf(A[q].m, mb);
    const float mu = mn == -INFINITY ? 0.f : mn;
    const float alpha = __expf(A[q].m - mu);
    A[q].m = mn;
    float ps = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      pv[j] = __expf(pv[j] - mu);
      ps += pv[j];
    }
    A[q].den = A[q].den * alpha + ps;
    bf16x8 ph, pl;
    split8(pv, ph, pl);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      f32x4 a = A[q].acc[dt] * alpha;
      a = mfma16(vf[dt], ph, a);
      a = mfma16(vf[dt], pl, a);
      A[q].acc[dt] = a;
    }
  }
}

// attn_block_n and attn_block2_n on K and V^T fragments already in registers (the fragments they read from
// LDS, in the same order): the same bits.
template <int NQ>
__device__ __forceinline__ void attn_block_n_rf(AttnState (&A)[NQ], int lane, const bf16x8 (&kf)[4], const bf16x8 (&vf)[4], int khi,
                                                float qs) {
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    f32x4 s[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      s[h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        s[h] = mfma16(kf[h * 2 + db], A[q].qh[db], s[h]);
        s[h] = mfma16(kf[h * 2 + db], A[q].ql[db], s[h]);
      }
    }
    float pv[8];
    float mb = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int key = (j >> 2) * 16 + 4 * (lane >> 4) + (j & 3);
      pv[j] = s[j >> 2][j & 3] * qs + ((key >= 0 && key < khi) ? 0.f : -INFINITY);
      mb = fmaxf(mb, pv[j]);
    }
    mb = xor32_max(xor16_max(mb));
    const float mn = fmaxf(A[q].m, mb);
    const float mu = mn == -INFINITY ? 0.f : mn;
    const float alpha = __expf(A[q].m - mu);
    A[q].m = mn;
    float ps = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      pv[j] = __expf(pv[j] - mu);
      ps += pv[j];
    }
    A[q].den = A[q].den * alpha + ps;
    bf16x8 ph, pl;
    split8(pv, ph, pl);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      f32x4 a = A[q].acc[dt] * alpha;
      a = mfma16(vf[dt], ph, a);
      a = mfma16(vf[dt], pl, a);
      A[q].acc[dt] = a;
    }
  }
}

template <int NQ>
__device__ __forceinline__ void attn_block2_n_rf(AttnState (&A)[NQ], int lane, const bf16x8 (&k0f)[4], const bf16x8 (&v0f)[4],
                                                 int khi0, const bf16x8 (&k1f)[4], const bf16x8 (&v1f)[4], int khi1, float qs) {
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    f32x4 s[2][2];
#pragma unroll
    for (int bk = 0; bk < 2; ++bk)
#pragma unroll
      for (int h = 0; h < 2; ++h) s[bk][h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int hl = 0; hl < 2; ++hl)
#pragma unroll
        for (int bk = 0; bk < 2; ++bk)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            s[bk][h] = mfma16((bk ? k1f : k0f)[h * 2 + db], hl ? A[q].ql[db] : A[q].qh[db], s[bk][h]);
    float pv[2][8];
    float mb = -INFINITY;
#pragma unroll
    for (int bk = 0; bk < 2; ++bk) {
      const int khi = bk ? khi1 : khi0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int key = (j >> 2) * 16 + 4 * (lane >> 4) + (j & 3);
        pv[bk][j] = s[bk][j >> 2][j & 3] * qs + (key < khi ? 0.f : -INFINITY);
        mb = fmaxf(mb, pv[bk][j]);
      }
    }
    mb = xor32_max(xor16_max(mb));
    const float mn = fmaxf(A[q].m, mb);
    const float mu = mn == -INFINITY ? 0.f : mn;
    const float alpha = __expf(A[q].m - mu);
    A[q].m = mn;
    float ps[2] = {0.f, 0.f};
#pragma unroll
    for (int bk = 0; bk < 2; ++bk)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        pv[bk][j] = __expf(pv[bk][j] - mu);
        ps[bk] += pv[bk][j];
      }
    A[q].den = A[q].den * alpha + (ps[0] + ps[1]);
    bf16x8 ph[2], pl[2];
    split8(pv[0], ph[0], pl[0]);
    split8(pv[1], ph[1], pl[1]);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      f32x4 a = A[q].acc[dt] * alpha;
      a = mfma16(v0f[dt], ph[0], a);
      a = mfma16(v1f[dt], ph[1], a);
      a = mfma16(v0f[dt], pl[0], a);
      a = mfma16(v1f[dt], pl[1], a);
      A[q].acc[dt] = a;
    }
  }
}

// attn_block_nq on K, V^T fragments and their residual parts already in registers, with the key RMS factors of
// the lane's 8 keys (what attn_block_nq reads from LDS, in the same order): the same bits.
template <int NQ>
__device__ __forceinline__ void attn_block_nq_rf(AttnState (&A)[NQ], int lane, const bf16x8 (&kf)[4], const bf16x8 (&kl)[4],
                                                 const bf16x8 (&vf)[4], const bf16x8 (&vl)[4], int khi, const float (&qs)[NQ],
                                                 const f32x4 (&rkv)[2]) {
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    f32x4 s[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      s[h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        s[h] = mfma16(kf[h * 2 + db], A[q].qh[db], s[h]);
        s[h] = mfma16(kf[h * 2 + db], A[q].ql[db], s[h]);
        s[h] = mfma16(kl[h * 2 + db], A[q].qh[db], s[h]);
      }
    }
    float pv[8];
    float mb = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int key = (j >> 2) * 16 + 4 * (lane >> 4) + (j & 3);
      const float sc = qs[q] * rkv[j >> 2][j & 3];
      pv[j] = s[j >> 2][j & 3] * sc + ((key >= 0 && key < khi) ? 0.f : -INFINITY);
      mb = fmaxf(mb, pv[j]);
    }
    mb = xor32_max(xor16_max(mb));
    const float mn = fmaxf(A[q].m, mb);
    const float mu = mn == -INFINITY ? 0.f : mn;
    const float alpha = __expf(A[q].m - mu);
    A[q].m = mn;
    float ps = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      pv[j] = __expf(pv[j] - mu);
      ps += pv[j];
    }
    A[q].den = A[q].den * alpha + ps;
    bf16x8 ph, pl;
    split8(pv, ph, pl);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      f32x4 a = A[q].acc[dt] * alpha;
      a = mfma16(vf[dt], ph, a);
      a = mfma16(vf[dt], pl, a);
      a = mfma16(vl[dt], ph, a);
      A[q].acc[dt] = a;
    }
  }
}

// One block of 32 keys for NQ query tiles at once (the arguments of attn_block, with one score scale per
// tile): the block's K and V^T fragments (and residual parts, key factors) are read once, each state's
// chains and softmax arithmetic are those of attn_block.
template <int NQ>
__device__ __forceinline__ void attn_block_nq(AttnState (&A)[NQ], int lane, const char* K, const char* Kl, const char* V,
                                              const char* Vl, int klo, int khi, const float (&qs)[NQ], const float* rk) {
  bf16x8 kf[4], kl[4], vf[4], vl[4];
  f32x4 rkv[2] = {f32x4{1.f, 1.f, 1.f, 1.f}, f32x4{1.f, 1.f, 1.f, 1.f}};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    kf[i] = ldsfrag(K + i * 1024 + lane * 16);
    if (Kl) kl[i] = ldsfrag(Kl + i * 1024 + lane * 16);
  }
  if (rk) {
    rkv[0] = *reinterpret_cast<const f32x4*>(rk + 4 * (lane >> 4));
    rkv[1] = *reinterpret_cast<const f32x4*>(rk + 16 + 4 * (lane >> 4));
  }
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    vf[dt] = ldsfrag(V + dt * 1024 + lane * 16);
    if (Vl) vl[dt] = ldsfrag(Vl + dt * 1024 + lane * 16);
  }
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    f32x4 s[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      s[h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        s[h] = mfma16(kf[h * 2 + db], A[q].qh[db], s[h]);
        s[h] = mfma16(kf[h * 2 + db], A[q].ql[db], s[h]);
        if (Kl) s[h] = mfma16(kl[h * 2 + db], A[q].qh[db], s[h]);
      }
    }
    float pv[8];
    float mb = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int key = (j >> 2) * 16 + 4 * (lane >> 4) + (j & 3);
      const float sc = qs[q] * rkv[j >> 2][j & 3];
      pv[j] = s[j >> 2][j & 3] * sc + ((key >= klo && key < khi) ? 0.f : -INFINITY);
      mb = fmaxf(mb, pv[j]);
    }
    mb = xor32_max(xor16_max(mb));
    const float mn = fmaxf(A[q].m, mb);
    const float mu = mn == -INFINITY ? 0.f : mn;
    const float alpha = __expf(A[q].m - mu);
    A[q].m = mn;
    float ps = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      pv[j] = __expf(pv[j] - mu);
      ps += pv[j];
    }
    A[q].den = A[q].den * alpha + ps;
    bf16x8 ph, pl;
    split8(pv, ph, pl);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      f32x4 a = A[q].acc[dt] * alpha;
      a = mfma16(vf[dt], ph, a);
      a = mfma16(vf[dt], pl, a);
      if (Vl) a = mfma16(vl[dt], ph, a);
      A[q].acc[dt] = a;
    }
  }
}

// Two blocks of 32 source keys as one 64-key step (attn_block2) for NQ query tiles at once, each block's
// fragments read once.
template <int NQ>
__device__ __forceinline__ void attn_block2_n(AttnState (&A)[NQ], int lane, const char* K0, const char* V0, int khi0,
                                              const char* K1, const char* V1, int khi1, float qs) {
  bf16x8 kf[2][4], vf[2][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    kf[0][i] = ldsfrag(K0 + i * 1024 + lane * 16);
    kf[1][i] = ldsfrag(K1 + i * 1024 + lane * 16);
  }
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    vf[0][dt] = ldsfrag(V0 + dt * 1024 + lane * 16);
    vf[1][dt] = ldsfrag(V1 + dt * 1024 + lane * 16);
  }
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    f32x4 s[2][2];
#pragma unroll
    for (int bk = 0; bk < 2; ++bk)
#pragma unroll
      for (int h = 0; h < 2; ++h) s[bk][h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int hl = 0; hl < 2; ++hl)
#pragma unroll
        for (int bk = 0; bk < 2; ++bk)
#pragma unroll
          for (int h = 0; h < 2; ++h) s[bk][h] = mfma16(kf[bk][h * 2 + db], hl ? A[q].ql[db] : A[q].qh[db], s[bk][h]);
    float pv[2][8];
    float mb = -INFINITY;
#pragma unroll
    for (int bk = 0; bk < 2; ++bk) {
      const int khi = bk ? khi1 : khi0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int key = (j >> 2) * 16 + 4 * (lane >> 4) + (j & 3);
        pv[bk][j] = s[bk][j >> 2][j & 3] * qs + (key < khi ? 0.f : -INFINITY);
        mb = fmaxf(mb, pv[bk][j]);
      }
    }
    mb = xor32_max(xor16_max(mb));
    const float mn = fmaxf(A[q].m, mb);
    const float mu = mn == -INFINITY ? 0.f : mn;
    const float alpha = __expf(A[q].m - mu);
    A[q].m = mn;
    float ps[2] = {0.f, 0.f};
#pragma unroll
    for (int bk = 0; bk < 2; ++bk)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        pv[bk][j] = __expf(pv[bk][j] - mu);
        ps[bk] += pv[bk][j];
      }
    A[q].den = A[q].den * alpha + (ps[0] + ps[1]);
    bf16x8 ph[2], pl[2];
    split8(pv[0], ph[0], pl[0]);
    split8(pv[1], ph[1], pl[1]);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      f32x4 a = A[q].acc[dt] * alpha;
      a = mfma16(vf[0][dt], ph[0], a);
      a = mfma16(vf[1][dt], ph[1], a);
      a = mfma16(vf[0][dt], pl[0], a);
      a = mfma16(vf[1][dt], pl[1], a);
      A[q].acc[dt] = a;
    }
  }
}

// register rows' k (normed, rotated) and v of step 1, bf16 [L][B][R][NH][64] (src/mk_expert.py:440-470), from
// the own keys and values staged in LDS (hi + lo parts) and the key RMS factors (sa_stage's own copy of these
// steps is kept inline there: as a call it changes that function's register allocation)
template <class S>
__device__ __forceinline__ void sa_register_kv(Ctx<S>& c, const char* Kh, const char* Kl, const char* Vh, const char* Vl,
                                               const float* rk, int l, int b, int hd) {
  CP& p = c.p;
  for (int it = c.tid; it < p.R * 8; it += NTHREADS) {
    const int i = p.T + it / 8, dd = (it % 8) * 8;
    bf16x8 kh = ldsfrag(Kh + kchunk_off(i, dd)), kl = ldsfrag(Kl + kchunk_off(i, dd));
    const u32x4 khu = __builtin_bit_cast(u32x4, kh), klu = __builtin_bit_cast(u32x4, kl);
    float kf[8], kr[8], vf[8];
    unpack8(khu, kf);
    unpack8(klu, kr);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      kf[e] = (kf[e] + kr[e]) * rk[i];
      vf[e] = bf2f(*reinterpret_cast<const bf16_t*>(Vh + vt_off(i, dd + e))) +
              bf2f(*reinterpret_cast<const bf16_t*>(Vl + vt_off(i, dd + e)));
    }
    const long long o = ((((long long)l * p.B + b) * p.R + (i - p.T)) * S::NH + hd) * HD + dd;
    u32x4 wk, wv;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      wk[e] = cvt_pk(kf[2 * e], kf[2 * e + 1]);
      wv[e] = cvt_pk(vf[2 * e], vf[2 * e + 1]);
    }
    *reinterpret_cast<u32x4*>(p.cur_k + o) = wk;
    *reinterpret_cast<u32x4*>(p.cur_v + o) = wv;
  }
}

// Self-attention with tasks of two query tiles (the Shape::PAIRS instantiations, for launches whose one-tile
// tasks outnumber the workgroups and whose two-tile tasks do not). Task u: sample-head u % nhb, tiles 2 j and 2 j + 1
// (j = u / nhb; a last odd tile alone, its second state a discarded copy of the first). The head's memory
// rows, own keys and values are staged once and both tiles' states run through each key block with the
// block's fragments read once; the second tile's query rows and sums of squares are staged in the merge
// area until both states have read them. Each state's arithmetic is that of sa_stage.
template <class S>
__device__ __forceinline__ void sa_stage_pairs(Ctx<S>& c, const Desc& d, const int* s_ks, BarCtx& bc, int g) {
  CP& p = c.p;
  const int M = p.Mq, Mqp = p.Mqp, PM = p.PM, PMP = ceil_to(PM, 32), NOWN32 = ceil_to(M, 32);
  const int NQT = Mqp / 16, NKT = NOWN32 / 16, KBO = NOWN32 / 32, NRP = p.NRP, RT = c.RT;
  const int l = d.l;
  char* fr = c.frame(d.s, l);
  const char* qs = fr + S::qs_off(NRP);
  const char* ks = fr + S::ks_off(NRP);
  const char* vt = fr + S::vtb_off(NRP);
  const float* ssqk = (const float*)(fr + S::ssqk_off(NRP));
  float* ysa = (float*)(fr + S::ysa_off(NRP));
  char* memK = c.smem + S::WBUF;
  char* memVt = memK + PMP * 128;
  char* Qh = c.smem + S::ABUF;
  char* Ql = Qh + 2048;
  char* Kh = Ql + 2048;
  char* Kl = Kh + NOWN32 * 128;
  char* Vh = Kl + NOWN32 * 128;
  char* Vl = Vh + NOWN32 * 128;
  float* rk = (float*)(Vl + NOWN32 * 128);
  float* mrg = rk + 128;
  float* sq_l = mrg;                 // [tile][column half][16 rows]
  char* Qh1 = (char*)(mrg + 64);     // the second tile's Q chunks (hi, lo)
  char* Ql1 = Qh1 + 2048;
  const int NHB = p.B * S::NH, NP = (NQT + 1) / 2;
  const bool want_kv = (d.s == 0 && p.cur_k != nullptr && p.R > 0);
  const int u = task_first(c, PL_SA);
  if (u >= NHB * NP) return;
  const int hh = u % NHB, qa = 2 * (u / NHB), nq = min(2, NQT - qa);
  const int b = hh / S::NH, hd = hh % S::NH;
  const int kvs = s_ks[b];
  {
    const int rgq = p.rgs_qkv;
    flag_wait<1>(bc, F_QKV, 6 * rgq, [&](int i) {
      const int k = i % 6, rg = i / 6;
      return rg * 6 * S::NH + (k >> 1) * 2 * S::NH + 2 * hd + (k & 1);
    }, (unsigned long long)g);
  }
  MKX_TR(c, 0);
  const int rt0 = b * Mqp / 16;
  if (c.wave == 0) {
    // lane: row lane % 16, column half (lane / 16) % 2, tile lane / 32
    const int qt = qa + ((c.lane >> 5) ? nq - 1 : 0);
    const int qq = qt * 16 + (c.lane & 15), j = (c.lane >> 4) & 1;
    __builtin_amdgcn_global_load_lds(ssqk + (long long)(hd * 2 + j) * NRP + b * Mqp + qq, (lds_void*)sq_l, 4, 0, 0);
  }
  // each wave's first DMAs are its pieces of the two Q tiles, then K tiles of all own keys and V^T blocks
  // (SA_REG: the Q tiles only; each wave loads its own-key block itself below)
  const bool reg = S::SA_REG && !want_kv;
  for (int k = c.wave; k < (reg ? 8 : 8 + 4 * NKT + 8 * KBO); k += NWAVES) {
    if (k < 8) {
      const int t = k >> 2, db = (k >> 1) & 1, part = k & 1;
      const int qt = qa + (t ? nq - 1 : 0);
      char* dst = t ? (part ? Ql1 : Qh1) : (part ? Ql : Qh);
      dma16(qs + ((long long)((2 * hd + db) * RT + rt0 + qt) * 2 + part) * 1024 + c.lane * 16, dst + db * 1024);
    } else if (k < 8 + 4 * NKT) {
      const int kk = k - 8, kt = kk >> 2, db = (kk >> 1) & 1, part = kk & 1;
      const int rtk = rt0 + min(kt, NQT - 1);
      dma16(ks + ((long long)((2 * hd + db) * RT + rtk) * 2 + part) * 1024 + c.lane * 16, (part ? Kl : Kh) + (kt * 2 + db) * 1024);
    } else {
      const int vv = k - 8 - 4 * NKT;
      dma16(vt + ((long long)hh * KBO * 8 + vv) * 1024 + c.lane * 16, ((vv & 1) ? Vl : Vh) + (vv >> 1) * 1024);
    }
  }
  const int rowk = b * Mqp + min(c.tid, Mqp - 1);
  const float ssk0 = ssqk[(long long)((S::NH + hd) * 2) * NRP + rowk];
  const float ssk1 = ssqk[(long long)((S::NH + hd) * 2 + 1) * NRP + rowk];
  // every wave issued at least 4 own-key DMAs after its Q pieces (4 NKT + 8 KBO >= 16 over 4 waves)
  if (reg) wait_vm0();
  else wait_vm_le<4>();
  exec_barrier();
  MKX_TR(c, 1);
  AttnState A[2];
  attn_begin(A[0], Qh, Ql, c.lane);
  attn_begin(A[1], Qh1, Ql1, c.lane);
  float qsc[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const float ssq = sq_l[32 * t + (c.lane & 15)] + sq_l[32 * t + 16 + (c.lane & 15)];
    qsc[t] = p.sm_scale * rsqrtf(ssq / 64.f + p.qk_eps);
  }
  const int mb0 = kvs >> 5, nmb = PMP / 32 - mb0;
  // SA_REG: this wave's own-key block jo and its lanes' key factors into registers, landing during the memory
  // blocks (as in sa_stage)
  const int jo = ((c.wave - nmb) % NWAVES + NWAVES) % NWAVES;
  bf16x8 okh[4], okl[4], ovh[4], ovl[4];
  float ssa[8], ssb[8];
  if (reg && jo < KBO) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kt = 2 * jo + (i >> 1), db = i & 1;
      const int rtk = rt0 + min(kt, NQT - 1);
      const char* kp = ks + ((long long)((2 * hd + db) * RT + rtk) * 2) * 1024 + c.lane * 16;
      okh[i] = __builtin_bit_cast(bf16x8, ld16(kp));
      okl[i] = __builtin_bit_cast(bf16x8, ld16(kp + 1024));
      const char* vp = vt + ((long long)hh * KBO * 8 + 2 * (jo * 4 + i)) * 1024 + c.lane * 16;
      ovh[i] = __builtin_bit_cast(bf16x8, ld16(vp));
      ovl[i] = __builtin_bit_cast(bf16x8, ld16(vp + 1024));
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int key = jo * 32 + (e >> 2) * 16 + 4 * (c.lane >> 4) + (e & 3);
      const int row = b * Mqp + min(key, Mqp - 1);
      ssa[e] = ssqk[(long long)((S::NH + hd) * 2) * NRP + row];
      ssb[e] = ssqk[(long long)((S::NH + hd) * 2 + 1) * NRP + row];
    }
  }
  for (int beta = c.wave; beta < nmb; beta += NWAVES) {
    const int kb = mb0 + beta;
    attn_block_nq<2>(A, c.lane, memK + kb * 4096, nullptr, memVt + kb * 4096, nullptr, kvs - kb * 32, PM - kb * 32, qsc, nullptr);
  }
  if (reg) {
    if (jo < KBO) {
      // the lanes' key factors, and zero V for own keys beyond the sample's rows (no producer)
      f32x4 rkv[2];
#pragma unroll
      for (int e = 0; e < 8; ++e) rkv[e >> 2][e & 3] = rsqrtf((ssa[e] + ssb[e]) / 64.f + p.qk_eps);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        u32x4 hv = __builtin_bit_cast(u32x4, ovh[dt]), lv = __builtin_bit_cast(u32x4, ovl[dt]);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int key = jo * 32 + (j >> 2) * 16 + 4 * (c.lane >> 4) + (j & 3);
          if (key >= Mqp) {
            const uint32_t keep = (j & 1) ? 0x0000ffffu : 0xffff0000u;
            hv[j >> 1] &= keep;
            lv[j >> 1] &= keep;
          }
        }
        ovh[dt] = __builtin_bit_cast(bf16x8, hv);
        ovl[dt] = __builtin_bit_cast(bf16x8, lv);
      }
      attn_block_nq_rf<2>(A, c.lane, okh, okl, ovh, ovl, M - jo * 32, qsc, rkv);
    }
    // every wave has read both tiles' queries and sums of squares (in the merge area) before the merge
    exec_barrier();
  } else {
    wait_vm0();  // the own keys' K and V^T have landed
    __syncthreads();
    if (c.tid < NOWN32) rk[c.tid] = rsqrtf((ssk0 + ssk1) / 64.f + p.qk_eps);
    for (int it = c.tid; it < (NOWN32 - Mqp) * HD; it += NTHREADS) {
      const int key = Mqp + it / HD, dd = it % HD;
      *reinterpret_cast<bf16_t*>(Vh + vt_off(key, dd)) = 0;
      *reinterpret_cast<bf16_t*>(Vl + vt_off(key, dd)) = 0;
    }
    __syncthreads();  // (also: every wave has read both tiles' queries before the merge area is reused)
    for (int beta = nmb + ((c.wave - nmb) % NWAVES + NWAVES) % NWAVES; beta < nmb + KBO; beta += NWAVES) {
      const int kb = beta - nmb;
      attn_block_nq<2>(A, c.lane, Kh + kb * 4096, Kl + kb * 4096, Vh + kb * 4096, Vl + kb * 4096, 0, M - kb * 32, qsc, rk + kb * 32);
    }
  }
  MKX_TR(c, 2);
  attn_merge_store(c, A[0], mrg, ysa, b, hd, qa);
  if (nq == 2) {
    __syncthreads();  // the first merge's partials have been read
    attn_merge_store(c, A[1], mrg, ysa, b, hd, qa + 1);
  }
  if (want_kv && qa == 0) sa_register_kv(c, Kh, Kl, Vh, Vl, rk, l, b, hd);
  flag_publish(bc, F_SA, hh * NQT + qa, (unsigned long long)g + 1);
  // the second tile's epoch: the same wait and barrier cover its rows
  if (nq == 2 && c.tid == 0)
    __hip_atomic_store(&bc.flags[((long long)F_SA * FLAG_MAX + hh * NQT + qa + 1) * FLAG_STRIDE],
                       bc.base + (unsigned long long)g + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Cross-attention with tasks of two query tiles (row-wise form, Params::ca_grp: set where the
// single-tile tasks outnumber the workgroups, the two-tile tasks do not, and every source fits the three LDS
// ring slots). Task u: sample-head u % nhb, tiles 2 j and 2 j + 1 (j = u / nhb; a last odd tile alone, whose
// second state runs on a copy of the first and is discarded). The task loads the head's Wq fragments, the
// sample's source keys and values and both tiles' rows once, projects the two tiles' queries in one pass over
// the k-blocks (per tile the steps of ca_stage), and runs both through each key block with the block's fragments read
// once; each tile's result is merged, stored and published as ca_stage does, so the outputs are the same bits.
template <class S>
__device__ __forceinline__ void ca_stage_pairs(Ctx<S>& c, const Desc& d, const int* s_ks, BarCtx& bc, int g) {
  CP& p = c.p;
  constexpr int KPW = S::KPW;
  const int Mqp = p.Mqp, NQT = Mqp / 16, NRP = p.NRP, RT = c.RT;
  const int l = d.l;
  char* fr = c.frame(d.s, l);
  const float* y2 = (const float*)(fr + S::y2_off(NRP));
  const float* ss2 = (const float*)(fr + S::ss2_off(NRP));
  float* yca = (float*)(fr + S::yca_off(NRP));
  const char* wq = p.wqca + l * p.s_o;
  const char* shs = p.shs + ((long long)(d.s * p.L + l) * 3 + 1) * p.B * S::H * 4;
  // the LDS map of ca_stage; the second tile's query partials, then its queries, are staged in the merge area
  // until both states have read them
  char* red = c.smem + S::ABUF + 32768;
  char* Qh0 = c.smem + S::ABUF + 32768 + NWAVES * 4 * 2 * 68 * 16;
  float* mrg = (float*)(Qh0 + 4096);
  char* Qh1 = (char*)mrg;
  float* ssw = (float*)(c.smem + S::SMALL);  // [tile][4 waves][16 rows]
  const int NHB = p.B * S::NH, NP = (NQT + 1) / 2;
  const uint32_t vlane = (uint32_t)c.lane * 16;
  const int u = task_first(c, PL_CA);
  if (u >= NHB * NP) return;
  const int hh = u % NHB, qa = 2 * (u / NHB), nq = min(2, NQT - qa);
  const int b = hh / S::NH, hd = hh % S::NH;
  const int S_len = s_ks[MAX_BATCH + b];
  // the Wq fragments of the head and the shift fragments, before the wait (as ca_stage)
  f16x8 wf[4][KPW], sh[KPW];
  {
    const __amdgpu_buffer_rsrc_t rsh =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(shs), (short)0, p.B * S::H * 4, 0x00020000);
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      const int kb = c.wave + NWAVES * i;
      const uint32_t o = (uint32_t)((((c.lane & 15) * S::NKB + kb) * 4 + (c.lane >> 4)) * 32);
      sh[i] = __builtin_bit_cast(f16x8, bload(rsh, o, 0));
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
        wf[nt][i] = wfrag_glb<S>(wq + ((long long)(hd * 4 + nt) * S::NKB + kb) * S::CH, c.lane);
    }
  }
  const int r = 4 * c.wave + (c.lane >> 4), cg = c.lane & 15;
  const uint2 wn = *reinterpret_cast<const uint2*>(p.qcan + l * HD + 4 * cg);
  const f32x4 scq = S::W8 ? ldf4(p.sc_qca + (long long)l * S::H + hd * HD + 4 * cg) : f32x4{1.f, 1.f, 1.f, 1.f};
  f32x4 cs[2], sn[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int pos = min((qa + (t ? nq - 1 : 0)) * 16 + r, p.Mq - 1);
    cs[t] = ldf4(p.ca_cos + pos * HD + 4 * cg);
    sn[t] = ldf4(p.ca_sin + pos * HD + 4 * cg);
  }
  f32x4 accb[4][2];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) accb[nt][0] = accb[nt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < KPW; ++i)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) accb[nt][i & 1] = mfma16h(wf[nt][i], sh[i], accb[nt][i & 1]);
  MKX_TR(c, 14);
  // every out-projection task of the row groups holding the two tiles' rows
  const int rq0 = b * Mqp / 16 + qa, rq1 = rq0 + nq - 1;
  {
    const int to = S::HT / p.nt_o;
    const int rg0 = row_group_of(rq0, RT, p.rgs_o), rg1 = row_group_of(rq1, RT, p.rgs_o);
    flag_wait<1>(bc, F_O, to, [&](int i) { return rg0 * to + i; }, (unsigned long long)g);
    if (rg1 != rg0) flag_wait<1>(bc, F_O, to, [&](int i) { return rg1 * to + i; }, (unsigned long long)g);
  }
  MKX_TR(c, 0);
  // both tiles' sums of squares and y2 fragments
  f16x8 yh[2][KPW];
  u32x2 ssv[2][S::HT / 8];
  {
    const __amdgpu_buffer_rsrc_t rs_ = rsrc(ss2), ry = rsrc(y2);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int rq = t ? rq1 : rq0;
      const uint32_t so = ss_slot<S::HT>(rq * 16 + (c.lane & 15), c.wave * (S::HT / 4));
#pragma unroll
      for (int i = 0; i < S::HT / 8; ++i) ssv[t][i] = bload8(rs_, so, (uint32_t)i * 128);
#pragma unroll
      for (int i = 0; i < KPW; ++i) {
        const int kb = c.wave + NWAVES * i;
        yh[t][i] = __builtin_bit_cast(f16x8, bload(ry, vlane, (uint32_t)((kb * RT + rq) * 2048)));
      }
    }
  }
  // the source K/V after the rows (the poll does not wait behind them): with CA_LATE, this wave's three
  // 32-key blocks (w, w + 4, w + 8: the fragments the LDS ring would hold for it) straight into registers, as
  // they are read by this wave only (as LDS DMA, 96 KB took ~2.6 us to issue, holding the waves before the
  // query projection); the other fp8 kernels DMA the ring during the barrier before the stage
  bf16x8 kvk[3][4], kvv[3][4];
  if constexpr (S::CA_LATE) {
    const bf16_t* kb_ = p.kca[l] + (long long)b * p.src_sb;
    const int ncb = p.SPP / 32;
    const bf16_t* vt = p.cavt + ((long long)(l * p.B + b) * S::NH + hd) * ncb * 2048;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      // rows beyond the length repeat a valid one and blocks beyond it are not used
      const int kbl = min(j * 4 + c.wave, ncb - 1);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = min(j * 128 + (2 * c.wave + (i >> 1)) * 16 + (c.lane & 15), max(S_len - 1, 0));
        kvk[j][i] = __builtin_bit_cast(bf16x8, ld16(kb_ + ((long long)key * S::NH + hd) * HD + (i & 1) * 32 + 8 * (c.lane >> 4)));
      }
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) kvv[j][dt] = __builtin_bit_cast(bf16x8, ld16(vt + ((long long)kbl * 4 + dt) * 512 + c.lane * 8));
    }
  } else {
    wait_vm0();
  }
  MKX_TR(c, 3);
  {
    // both tiles' query rows in one pass over the k-blocks ([tile][column tile][k-block parity]); the second
    // tile's partials go to the merge area, the shift partials (the same for both) to red once
    f32x4 acc[2][4][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) acc[t][nt][0] = acc[t][nt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < KPW; ++i)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int t = 0; t < 2; ++t) acc[t][nt][i & 1] = mfma16h(wf[nt][i], yh[t][i], acc[t][nt][i & 1]);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const float ssp = ss_pairs_sum<S::HT / 8>(ssv[t]);
      if (c.lane < 16) ssw[t * 64 + c.wave * 16 + c.lane] = ssp;
    }
    const int sl = c.lane + (c.lane >> 4);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      sts16(red + (((c.wave * 4 + nt) * 2 + 0) * 68 + sl) * 16, as_u4(acc[0][nt][0] + acc[0][nt][1]));
      sts16(red + (((c.wave * 4 + nt) * 2 + 1) * 68 + sl) * 16, as_u4(accb[nt][0] + accb[nt][1]));
      sts16((char*)mrg + ((c.wave * 4 + nt) * 68 + sl) * 16, as_u4(acc[1][nt][0] + acc[1][nt][1]));
    }
  }
  __syncthreads();
  // q of row r, columns 4 cg .. 4 cg + 3, of both tiles (the steps of ca_stage)
  const int dd = 4 * cg;
  const int qoff = (dd >> 5) * 1024 + (r + 16 * ((dd & 31) >> 3)) * 16 + (dd & 4) * 2;
  u32x2 qhi[2], qlo[2];
  {
    const int nt = cg >> 2, lr = r + 16 * (cg & 3), lb = b + 16 * (cg & 3);
    f32x4 ba[NWAVES];
#pragma unroll
    for (int w = 0; w < NWAVES; ++w) ba[w] = ldf4((const float*)(red + (((w * 4 + nt) * 2 + 1) * 68 + lb + (lb >> 4)) * 16));
    lds_batch(ba);
    float bv[4] = {ba[0][0], ba[0][1], ba[0][2], ba[0][3]};
#pragma unroll
    for (int w = 1; w < NWAVES; ++w)
#pragma unroll
      for (int e = 0; e < 4; ++e) bv[e] += ba[w][e];
    const f32x4 gw = {1.0f + __uint_as_float(wn.x << 16), 1.0f + __uint_as_float(wn.x & 0xffff0000u),
                      1.0f + __uint_as_float(wn.y << 16), 1.0f + __uint_as_float(wn.y & 0xffff0000u)};
    const float sgn = cg < 8 ? -1.0f : 1.0f;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      f32x4 qa4[NWAVES];
      float sw[NWAVES];
#pragma unroll
      for (int w = 0; w < NWAVES; ++w) {
        const int slot = ((w * 4 + nt) * (t ? 1 : 2)) * 68 + lr + (lr >> 4);
        qa4[w] = ldf4((const float*)((t ? (char*)mrg : red) + slot * 16));
        sw[w] = ssw[t * 64 + 16 * w + r];
      }
      lds_batch(qa4);
      lds_batch(sw);
      f32x4 qv = qa4[0];
#pragma unroll
      for (int w = 1; w < NWAVES; ++w) qv += qa4[w];
      const float rs = rsqrtf((sw[0] + sw[1] + sw[2] + sw[3]) * (1.0f / (float)S::H) + p.eps);
      f32x4 x;
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = (qv[e] * rs + bv[e]) * scq[e];
      float ss = x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
      ss = row_sum16(ss);
      const float rn = rsqrtf(ss / 64.f + p.qk_eps);
      const f32x4 xn = x * rn * gw;
      f32x4 uq;
#pragma unroll
      for (int e = 0; e < 4; ++e) uq[e] = xn[e] * cs[t][e] + sgn * lane_xor8(xn[e]) * sn[t][e];
      qhi[t][0] = cvt_pk(uq[0], uq[1]);
      qhi[t][1] = cvt_pk(uq[2], uq[3]);
      qlo[t][0] = cvt_pk(uq[0] - __uint_as_float(qhi[t][0] << 16), uq[1] - __uint_as_float(qhi[t][0] & 0xffff0000u));
      qlo[t][1] = cvt_pk(uq[2] - __uint_as_float(qhi[t][1] << 16), uq[3] - __uint_as_float(qhi[t][1] & 0xffff0000u));
    }
  }
  *reinterpret_cast<u32x2*>(Qh0 + qoff) = qhi[0];
  *reinterpret_cast<u32x2*>(Qh0 + 2048 + qoff) = qlo[0];
  __syncthreads();  // every thread has read the second tile's partials in the merge area
  *reinterpret_cast<u32x2*>(Qh1 + qoff) = qhi[1];
  *reinterpret_cast<u32x2*>(Qh1 + 2048 + qoff) = qlo[1];
  if constexpr (!S::CA_LATE) wait_vm0();  // this wave's K/V DMAs (the barrier covers the other waves')
  __syncthreads();
  MKX_TR(c, 1);
  AttnState A[2];
  attn_begin(A[0], Qh0, Qh0 + 2048, c.lane);
  attn_begin(A[1], Qh1, Qh1 + 2048, c.lane);
  __syncthreads();  // every wave holds both tiles' queries: the merge area may be overwritten
  if constexpr (S::CA_LATE) {
    const int k0 = c.wave * 32, k1 = 128 + c.wave * 32, k2 = 256 + c.wave * 32;
    if (k1 < S_len)
      attn_block2_n_rf<2>(A, c.lane, kvk[0], kvv[0], S_len - k0, kvk[1], kvv[1], S_len - k1, p.sm_scale);
    else if (k0 < S_len)
      attn_block_n_rf<2>(A, c.lane, kvk[0], kvv[0], S_len - k0, p.sm_scale);
    if (k2 < S_len) attn_block_n_rf<2>(A, c.lane, kvk[2], kvv[2], S_len - k2, p.sm_scale);
  } else {
    const int k0 = c.wave * 32, k1 = 128 + c.wave * 32, k2 = 256 + c.wave * 32;
    char* s0 = ca_slot(c, 0);
    char* s1 = ca_slot(c, 1);
    char* s2 = ca_slot(c, 2);
    if (k1 < S_len)
      attn_block2_n<2>(A, c.lane, s0 + c.wave * 4096, s0 + 16384 + c.wave * 4096, S_len - k0, s1 + c.wave * 4096,
                       s1 + 16384 + c.wave * 4096, S_len - k1, p.sm_scale);
    else if (k0 < S_len)
      attn_block_n<2>(A, c.lane, s0 + c.wave * 4096, s0 + 16384 + c.wave * 4096, S_len - k0, p.sm_scale);
    if (k2 < S_len) attn_block_n<2>(A, c.lane, s2 + c.wave * 4096, s2 + 16384 + c.wave * 4096, S_len - k2, p.sm_scale);
  }
  MKX_TR(c, 2);
  attn_merge_store(c, A[0], mrg, yca, b, hd, qa);
  if (nq == 2) {
    __syncthreads();  // the first merge's partials have been read
    attn_merge_store(c, A[1], mrg, yca, b, hd, qa + 1);
  }
  MKX_TR(c, 13);
  flag_publish(bc, F_CA, hh * NQT + qa, (unsigned long long)g + 1);
  // the second tile's epoch: the same wait and barrier cover its rows
  if (nq == 2 && c.tid == 0)
    __hip_atomic_store(&bc.flags[((long long)F_CA * FLAG_MAX + hh * NQT + qa + 1) * FLAG_STRIDE],
                       bc.base + (unsigned long long)g + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------------------------------------------
// Step tail (src/mk_expert.py:254-299): o = AdaRMS_final(h_L); v = o Wout^T + bout; x' = x + dt v;
// h0' = x'_real Win + bin (action rows), register tokens (register rows), all fp32; with h0' its layer-0
// AdaRMS operand y0' = h0' (1 + scale) (split) and sums of squares. Tasks [0, NIN): in-projection tasks of
// two 16-column tiles (each recomputes the velocity of the real action dims);
// then A / TAIL_AC output tasks of TAIL_AC dims each (x after the step, which only the next step tail
// reads), placed by the host (Params::pl). Wave w takes the action rows w + 4 k, TAIL_RPW of them per
// batch with their loads issued together; lane owns the 4-column pieces 4 (lane + 64 q). The final
// modulation rows and the task's Wout rows were staged in LDS by the prefetch; the in-projection's constant
// operands (Win columns, bias, register tokens, layer-0 scale) are loaded with the first batch.
constexpr int TAIL_RPW = 3;  // action rows per wave and batch
constexpr int TAIL_AC = 8;   // action dims reduced together
// Launches of the row-wise form (many rows) split the output tasks by rows as well: TAIL_RCH rows (one batch
// per wave) and TAIL_DG dims per task, written to x of the next step before the in-projection tasks, which
// read them there instead of each recomputing the velocity of every row.
constexpr int TAIL_RCH = NWAVES * TAIL_RPW;
constexpr int TAIL_DG = 2 * TAIL_AC;
// output tasks of a step tail (not the launch's first)
template <class S>
__device__ __forceinline__ int tail_nout(CP& p) {
  if constexpr (S::RW) return (p.B * p.T + TAIL_RCH - 1) / TAIL_RCH * ((p.A + TAIL_DG - 1) / TAIL_DG);
  else return (p.A + TAIL_AC - 1) / TAIL_AC;
}

template <int N>
__device__ __forceinline__ void wave_sum_n(float* v) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = wave_sum(v[i]);
}

template <class S>
__device__ __forceinline__ void tail_stage(Ctx<S>& c, const Desc& d, BarCtx& bc, int g) {
  CP& p = c.p;
  constexpr int NP = S::H / 256;  // pieces per lane
  constexpr int R = TAIL_RPW;
  const int nin = d.last ? 0 : S::NIN;
  const int nout = d.first ? 0 : tail_nout<S>(p);
  const int nrows = p.B * p.T;
  const int adim = p.action_dim;
  const float* xcur = (d.first || d.s == 0) ? p.x_in : c.xstep(d.s);
  const float* hL = d.first ? p.x_in : (const float*)(c.frame(d.s, p.L - 1) + S::hl_off(p.NRP));
  float* xp = (float*)(c.smem + S::ABUF);                // [nrows][adim] x' of the real dims
  const float* wo_l = (const float*)(c.smem + S::WBUF);  // Wout rows [adim][H]
  float* win_t = (float*)(c.smem + S::SMALL);            // Win columns of the task [adim][32]
  const int sn = d.first ? 0 : d.s + 1;
  // this workgroup's tasks: its in-projection task (k = 0), then its output task
  const int tin = task_first(c, PL_TIN), tout = task_first(c, PL_TOUT);
  bool first_task = true;
  for (int k = 0; k < 2; ++k) {
    int t = -1;
    // the row-wise form's in-projection tasks read the output tasks' x, so a workgroup with both runs its
    // output task first
    if (k == (S::RW ? 1 : 0)) t = tin < nin ? tin : -1;
    else t = tout < nout ? nin + tout : -1;
    if (t < 0) continue;
    if (!first_task) __syncthreads();  // the previous task's LDS (the first task's is free already)
    first_task = false;
    const bool inproj = t < nin;
    const int a_out = t - nin;
    // in-projection item of this thread (first pass): row, 4-column piece q of the task's 32 columns; its
    // constant operands (row-wise form: the piece's bias, the same in every item, items being 8 per row)
    const int row0 = c.tid >> 3, q0 = c.tid & 7;
    f32x4 sc0 = {0.f, 0.f, 0.f, 0.f}, bv0 = {0.f, 0.f, 0.f, 0.f};
    uint2 rg0 = {0u, 0u};
    f32x4 wt = {0.f, 0.f, 0.f, 0.f};
    if (inproj) {
      if constexpr (S::RW) {
        bv0 = ldf4(p.bin + t * 32 + 4 * q0);
      } else {
        const int b = row0 / p.Mqp, i = row0 - b * p.Mqp, col = t * 32 + 4 * q0;
        if (row0 < p.NRP) {
          sc0 = ldf4(c.modrow(min(b, p.B - 1), sn) + col);  // layer 0 self-attention AdaRMS scale
          if (b < p.B && i < p.T) bv0 = ldf4(p.bin + col);
          else if (b < p.B && i < p.Mq) rg0 = *reinterpret_cast<const uint2*>(p.reg_tok + (long long)(i - p.T) * S::H + col);
        }
      }
      if (c.tid < adim * 8) wt = ldf4(p.win + (long long)(c.tid >> 3) * S::H + t * 32 + 4 * (c.tid & 7));
    }
    if (!d.first && S::RW && inproj) {
      // x after the step, from this step tail's output tasks
      flag_wait<1>(bc, F_TAIL_OUT, nout, [](int i) { return i; }, (unsigned long long)g + 1);
    } else if (!d.first) {
      // every tile of the last layer's output (its reducers), and x of this step (the previous step tail's
      // output dims)
      if constexpr (S::RW) {  // (row-wise form: up to HT x 3 row-group reducers)
        if (p.nred <= 64) flag_wait<1>(bc, F_DOWN, p.nred, [](int i) { return i; }, (unsigned long long)g);
        else flag_wait<4>(bc, F_DOWN, p.nred, [](int i) { return i; }, (unsigned long long)g);
      } else {
        flag_wait<1>(bc, F_DOWN, p.nred, [](int i) { return i; }, (unsigned long long)g);
      }
      if (d.s > 0) flag_wait<1>(bc, F_TAIL_OUT, nout, [](int i) { return i; }, (unsigned long long)(g - (STAGES_PER_LAYER * p.L + 1) + 1));
    }
    // the staged final modulation rows and Wout rows (DMA'd by the prefetch) have landed
    wait_vm0();
    __syncthreads();
    MKX_TR(c, 0);
    if (!d.first && S::RW && inproj) {
      const float* xn = c.xstep(d.s + 1);
      for (int it = c.tid; it < nrows * adim; it += NTHREADS) {
        const int ri = it / adim, a = it - ri * adim;
        xp[it] = xn[(long long)ri * p.A + a];
      }
    } else if (!d.first) {
      const __amdgpu_buffer_rsrc_t rh = rsrc(hL);
      // dims [a_lo, a_hi) of this task (Wout rows staged in LDS from row a_lo): the in-projection's real dims,
      // or an output task's TAIL_AC dims (row-wise form: TAIL_DG dims of rows [r_lo, r_hi)). Lane a holds
      // bout[a] and, in xc[k], x of row k's dim a.
      int a_lo, a_hi, r_lo = 0, r_hi = nrows;
      if constexpr (S::RW) {
        const int ndg = (p.A + TAIL_DG - 1) / TAIL_DG;
        a_lo = inproj ? 0 : (a_out % ndg) * TAIL_DG;
        a_hi = inproj ? adim : min(a_lo + TAIL_DG, p.A);
        r_lo = (a_out / ndg) * TAIL_RCH;
        r_hi = min(r_lo + TAIL_RCH, nrows);
      } else {
        a_lo = inproj ? 0 : a_out * TAIL_AC;
        a_hi = inproj ? adim : min(a_lo + TAIL_AC, p.A);
      }
      const float bo = p.bout[min(c.lane, p.A - 1)];
      float* xn = d.last ? p.x_out : c.xstep(d.s + 1);
      // a launch whose synchronisation gave up (a wait exceeded its spin bound) returns NaN, not a result
      const bool poisoned = d.last && __hip_atomic_load(&p.bar->err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
      for (int r0 = r_lo + c.wave; r0 < r_hi; r0 += NWAVES * R) {
        f32x4 x[R][NP];
        float xc[R];
#pragma unroll
        for (int k = 0; k < R; ++k) {
          const int ri = min(r0 + NWAVES * k, r_hi - 1);
          const int b = ri / p.T, grow = b * p.Mqp + (ri - b * p.T);
#pragma unroll
          for (int q = 0; q < NP; ++q) x[k][q] = as_f4(bload(rh, fpiece(grow, 4 * (c.lane + 64 * q), c.RT), 0));
          xc[k] = xcur[(long long)ri * p.A + min(c.lane, p.A - 1)];
        }
        float ss[R];
#pragma unroll
        for (int k = 0; k < R; ++k) {
          ss[k] = 0.f;
#pragma unroll
          for (int q = 0; q < NP; ++q) ss[k] += x[k][q][0] * x[k][q][0] + x[k][q][1] * x[k][q][1] + x[k][q][2] * x[k][q][2] + x[k][q][3] * x[k][q][3];
        }
        wave_sum_n<R>(ss);
#pragma unroll
        for (int k = 0; k < R; ++k) {
          const int ri = min(r0 + NWAVES * k, r_hi - 1);
          const float rs = rsqrtf(ss[k] * (1.0f / (float)S::H) + (S::YS ? p.eps_final : p.eps));
          const float* ml = tail_mods_lds(c, ri / p.T);
#pragma unroll
          for (int q = 0; q < NP; ++q) {
            const int col = 4 * (c.lane + 64 * q);
            x[k][q] = x[k][q] * rs * (1.0f + ldf4(ml + col)) + ldf4(ml + S::H + col);
          }
        }
        for (int a0 = a_lo; a0 < a_hi; a0 += TAIL_AC) {
          float dd[TAIL_AC * R];
#pragma unroll
          for (int j = 0; j < TAIL_AC; ++j) {
            const int a = min(a0 + j, a_hi - 1);
#pragma unroll
            for (int k = 0; k < R; ++k) dd[j * R + k] = 0.f;
#pragma unroll
            for (int q = 0; q < NP; ++q) {
              const f32x4 w = ldf4(wo_l + (a - a_lo) * S::H + 4 * (c.lane + 64 * q));
#pragma unroll
              for (int k = 0; k < R; ++k)
                dd[j * R + k] += x[k][q][0] * w[0] + x[k][q][1] * w[1] + x[k][q][2] * w[2] + x[k][q][3] * w[3];
            }
          }
          wave_sum_n<TAIL_AC * R>(dd);
          float sel[R];
#pragma unroll
          for (int k = 0; k < R; ++k) sel[k] = 0.f;
#pragma unroll
          for (int j = 0; j < TAIL_AC; ++j)
            if (c.lane == a0 + j) {
#pragma unroll
              for (int k = 0; k < R; ++k) sel[k] = dd[j * R + k];
            }
          if (c.lane >= a0 && c.lane < min(a0 + TAIL_AC, a_hi)) {
#pragma unroll
            for (int k = 0; k < R; ++k) {
              const int ri = r0 + NWAVES * k;
              if (ri >= r_hi) continue;
              if (inproj) {
                xp[ri * adim + c.lane] = xc[k] + c.dt * (sel[k] + bo);
              } else {
                // x after the step: x + dt v on the real dims, dt v on the padded ones
                const float xa = c.lane < adim ? xc[k] : 0.f;
                st_sc1_b32(xn, (uint32_t)(((long long)ri * p.A + c.lane) * 4),
                           poisoned ? 0x7fc00000u : __float_as_uint(xa + c.dt * (sel[k] + bo)));
              }
            }
          }
        }
      }
    } else if (inproj) {
      for (int it = c.tid; it < nrows * adim; it += NTHREADS) {
        const int ri = it / adim, a = it - ri * adim;
        xp[it] = xcur[(long long)ri * p.A + a];
      }
    }
    if (inproj) {
      if (c.tid < adim * 8) *reinterpret_cast<f32x4*>(win_t + (c.tid >> 3) * 32 + 4 * (c.tid & 7)) = wt;
      __syncthreads();
      MKX_TR(c, 1);
      float* h0n = c.h0(sn);
      if constexpr (S::RW) {
        // items: row, 4-column piece q of the task's tiles 2 t (q < 4) and 2 t + 1; a thread's items are rows
        // 32 apart (many, in this form), IB of them per batch with their loads (the row's sample's layer-0
        // AdaRMS scale, a register row's token) issued together, so that a batch waits for one memory round
        // trip, not one per row
        constexpr int IB = 4;
        const int q = q0, col = t * 32 + 4 * q;
        for (int row1 = row0; row1 < p.NRP; row1 += IB * (NTHREADS / 8)) {
          f32x4 sc[IB];
          uint2 rg[IB];
#pragma unroll
          for (int k = 0; k < IB; ++k) {
            const int row = min(row1 + k * (NTHREADS / 8), p.NRP - 1);
            const int b = row / p.Mqp, i = row - b * p.Mqp;
            sc[k] = ldf4(c.modrow(min(b, p.B - 1), sn) + col);  // layer 0 self-attention AdaRMS scale
            const int ir = min(max(i - p.T, 0), max(p.R - 1, 0));  // (a valid register row, used for register rows only)
            rg[k] = p.R > 0 ? *reinterpret_cast<const uint2*>(p.reg_tok + (long long)ir * S::H + col) : uint2{0u, 0u};
          }
#pragma unroll
          for (int k = 0; k < IB; ++k) {
            const int row = row1 + k * (NTHREADS / 8);
            if (row >= p.NRP) break;
            const int b = row / p.Mqp, i = row - b * p.Mqp;
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (b < p.B && i < p.T) {
              v = bv0;
              const float* xr = xp + (b * p.T + i) * adim;
              for (int a = 0; a < adim; ++a) v += xr[a] * ldf4(win_t + a * 32 + 4 * q);
            } else if (b < p.B && i < p.Mq) {
              v = f32x4{__uint_as_float(rg[k].x << 16), __uint_as_float(rg[k].x & 0xffff0000u), __uint_as_float(rg[k].y << 16),
                        __uint_as_float(rg[k].y & 0xffff0000u)};
            }
            st_sc1(h0n, fpiece(row, col, c.RT), as_u4(v));
            const f32x4 vs = S::YS ? v * p.yinv : v;  // (the AdaRMS operand scaling)
            if (st_h4(c.y0(sn), spiece(row, col, c.RT), vs * (1.0f + sc[k]))) range_error(p.bar);
            float ss = vs[0] * vs[0] + vs[1] * vs[1] + vs[2] * vs[2] + vs[3] * vs[3];
            ss = quad_sum(ss);  // the 4 pieces of one 16-column tile are 4 adjacent lanes
            if ((q & 3) == 0) st_sc1_b32(c.ss0(sn), ss_slot<S::HT>(row, 2 * t + (q >> 2)), __float_as_uint(ss));
          }
        }
      } else {
        // item: row, 4-column piece q of the task's tiles 2 t (q < 4) and 2 t + 1
        for (int it = c.tid; it < p.NRP * 8; it += NTHREADS) {
          const int row = it >> 3, q = it & 7;
          const int b = row / p.Mqp, i = row - b * p.Mqp;
          const int col = t * 32 + 4 * q;
          f32x4 v, sc;
          uint2 rg;
          if (it == c.tid) {
            v = bv0;
            sc = sc0;
            rg = rg0;
          } else {
            v = f32x4{0.f, 0.f, 0.f, 0.f};
            rg = uint2{0u, 0u};
            sc = ldf4(c.modrow(min(b, p.B - 1), sn) + col);
            if (b < p.B && i < p.T) v = ldf4(p.bin + col);
            else if (b < p.B && i < p.Mq) rg = *reinterpret_cast<const uint2*>(p.reg_tok + (long long)(i - p.T) * S::H + col);
          }
          if (b < p.B && i < p.T) {
            const float* xr = xp + (b * p.T + i) * adim;
            for (int a = 0; a < adim; ++a) v += xr[a] * ldf4(win_t + a * 32 + 4 * q);
          } else if (b < p.B && i < p.Mq) {
            v = f32x4{__uint_as_float(rg.x << 16), __uint_as_float(rg.x & 0xffff0000u), __uint_as_float(rg.y << 16),
                      __uint_as_float(rg.y & 0xffff0000u)};
          }
          st_sc1(h0n, fpiece(row, col, c.RT), as_u4(v));
          const f32x4 vs = S::YS ? v * p.yinv : v;  // (the AdaRMS operand scaling)
          if (st_h4(c.y0(sn), spiece(row, col, c.RT), vs * (1.0f + sc))) range_error(p.bar);
          float ss = vs[0] * vs[0] + vs[1] * vs[1] + vs[2] * vs[2] + vs[3] * vs[3];
          ss = quad_sum(ss);  // the 4 pieces of one 16-column tile are 4 adjacent lanes
          if ((q & 3) == 0) st_sc1_b32(c.ss0(sn), ss_slot<S::HT>(row, 2 * t + (q >> 2)), __float_as_uint(ss));
        }
      }
    }
    flag_publish(bc, inproj ? F_TAIL_IN : F_TAIL_OUT, inproj ? t : a_out, (unsigned long long)g + 1);
  }
}

// ------------------------------------------------------------------------------------------------
// DMA of the constant operands of this workgroup's first task of stage d (weight tile or cached K/V, Wout
// rows) and of the stage's per-sample modulation slices.
template <class S>
__device__ __forceinline__ void prefetch_body(Ctx<S>& c, const Desc& d, const int* s_ks) {
  CP& p = c.p;
  MKX_TRW(c, 8);
  bool ca_pairs = false, sa_pairs = false;
  if constexpr (S::RW && !S::CA_REG) ca_pairs = d.st == ST_CA && p.ca_grp;
  if constexpr (S::PAIRS) sa_pairs = d.st == ST_SA;
  if (sa_pairs) {
    // two-tile self-attention tasks: task u runs sample-head u % (B NH)
    const int nhb = p.B * S::NH, u = task_first(c, d.pk);
    if (u < nhb * ((p.Mqp / 16 + 1) / 2)) {
      const int hh = u % nhb;
      sa_prefetch(c, d.l, hh / S::NH, hh % S::NH, s_ks[hh / S::NH]);
    }
  } else if (ca_pairs) {
    // two-tile cross-attention tasks: task u runs sample-head u % (B NH); the fp8 kernels without two-tile
    // self-attention DMA its source K/V here, the others after the poll
    if constexpr (!S::CA_LATE) {
      const int nhb = p.B * S::NH, u = task_first(c, d.pk);
      if (u < nhb * ((p.Mqp / 16 + 1) / 2)) {
        const int hh = u % nhb;
        ca_prefetch(c, d.l, hh / S::NH, hh % S::NH, s_ks[MAX_BATCH + hh / S::NH]);
      }
    }
  } else if (d.st == ST_SA || d.st == ST_CA) {
    const int nqt = p.Mqp / 16;
    const AttnTask at = attn_task<S::RW_ATTN>(task_first(c, d.pk), nqt, p.B * S::NH, c.G);
    if (at.ok) {
      const int b = at.hh / S::NH, hd = at.hh % S::NH;
      if (d.st == ST_SA) sa_prefetch(c, d.l, b, hd, s_ks[b]);
      else if (!S::CA_LATE && !(S::CA_REG && s_ks[MAX_BATCH + b] <= 384))
        ca_prefetch(c, d.l, b, hd, s_ks[MAX_BATCH + b]);  // (CA_LATE: after the poll; CA_REG: into registers)
    }
  } else if (d.st == ST_TAIL) {
    // workgroups with a tail task: the final modulation rows, and the Wout rows of the task's dims (the real
    // dims for an in-projection task)
    char* mb = c.smem + S::MODS;
    const int tout = task_first(c, PL_TOUT);
    // (the row-wise form's in-projection tasks read x after the step instead)
    const bool tin = !S::RW && task_first(c, PL_TIN) < (d.last ? 0 : S::NIN);
    if (!d.first && (tin || tout < tail_nout<S>(p))) {
      for (int b = 0; b < p.B; ++b) dma_f32(c, mb + b * 2 * S::H * 4, c.modrow(b, d.s) + 9 * p.L * S::H, 2 * S::H);
      if (tin) {
        dma_f32(c, c.smem + S::WBUF, p.wout, p.action_dim * S::H);
      } else if constexpr (S::RW) {
        const int a_lo = (tout % ((p.A + TAIL_DG - 1) / TAIL_DG)) * TAIL_DG;
        dma_f32(c, c.smem + S::WBUF, p.wout + (long long)a_lo * S::H, min(TAIL_DG, p.A - a_lo) * S::H);
      } else {
        dma_f32(c, c.smem + S::WBUF, p.wout + (long long)tout * TAIL_AC * S::H, min(TAIL_AC, p.A - tout * TAIL_AC) * S::H);
      }
    }
  } else {
    const int t = task_first(c, d.pk);
    char* mb = c.smem + p.lds_mods;
    if (t < d.ntask) {
      dma_task_w(c, d, t, c.smem + S::WBUF);
      MKX_TRW(c, 9);
    }
    // gate and the next AdaRMS scale: the residual stages' tasks, and the down projection's reducers (its
    // split tasks only store partial sums)
    if constexpr (S::RW) {
      // one 16-column tile per gated-residual task and per reducer (Params::tpr = 1): its slices only
      if (d.kind == K_RES && t < d.ntask) dma_mods_tile(c, d, t % d.tiles);
      else if (d.kind == K_SPLIT && task_first(c, PL_RED) < p.nred) dma_mods_tile(c, d, task_first(c, PL_RED) % S::HT);
    } else if ((d.kind == K_RES && t < d.ntask) || (d.kind == K_SPLIT && task_first(c, PL_RED) < p.nred)) {
      for (int b = 0; b < p.B; ++b) {
        const float* mr = c.modrow(b, d.s);
        dma_f32(c, mb + b * 2 * S::H * 4, mr + d.mod_off, S::H);
        dma_f32(c, mb + (b * 2 + 1) * S::H * 4, mr + d.mod_off2, S::H);
      }
    }
  }
}

// the prefetch of the next stage is issued by waves 1-3 while wave 0 completes the barrier
template <class S>
__device__ __forceinline__ void prefetch(Ctx<S>& c, const Desc& d, const int* s_ks) {
  if (c.wave == 0) return;
  c.dw = c.wave - 1;
  c.dn = NWAVES - 1;
  prefetch_body(c, d, s_ks);
  MKX_TRW(c, 10);
  c.dw = c.wave;
  c.dn = NWAVES;
}

// AdaRMS GEMM stages: the stage's split shift slices (B H hi / lo pairs, written in the launch's first stage)
// into LDS, by waves 1-3
template <class S>
__device__ __forceinline__ void prefetch_shifts(Ctx<S>& c, const Desc& d) {
  // (the row-wise form's tasks load their shift fragments after the poll)
  if (S::RW || c.wave == 0 || !(d.kind == K_QKV || d.kind == K_GU) || d.st == ST_TAIL || d.st == ST_SA || d.st == ST_CA ||
      task_first(c, d.pk) >= d.ntask)
    return;
  c.dw = c.wave - 1;
  c.dn = NWAVES - 1;
  dma_f32(c, c.smem + c.p.lds_mods, (const float*)d.shs, c.p.B * S::H);
  c.dw = c.wave;
  c.dn = NWAVES;
}

// Stage kinds in which this workgroup has a task: bit st (ST_QKV .. ST_DOWN, the down projection's
// reducers included; ST_TAIL: a step tail with an in-projection or output task), bit TAIL_LAST_BIT: the
// launch's last step tail (output tasks only). Workgroup 0 takes part in every stage, so that its stage
// boundary timestamps cover all of them.
constexpr int TAIL_LAST_BIT = 8;
template <class S>
__device__ __forceinline__ unsigned task_mask(Ctx<S>& c) {
  CP& p = c.p;
  if (c.wg == 0) return ~0u;
  const int nattn = attn_count(p.Mqp / 16, p.B * S::NH), nout = tail_nout<S>(p);
  unsigned m = 0;
  if (task_first(c, PL_QKV) < 6 * S::NH * p.rgs_qkv) m |= 1u << ST_QKV;
  if (task_first(c, PL_SA) < (S::PAIRS ? p.B * S::NH * ((p.Mqp / 16 + 1) / 2) : nattn)) m |= 1u << ST_SA;
  if (task_first(c, PL_O) < (S::HT / p.nt_o) * p.rgs_o) m |= 1u << ST_O;
  if (task_first(c, PL_CA) < (S::RW && !S::CA_REG && p.ca_grp ? p.B * S::NH * ((p.Mqp / 16 + 1) / 2) : nattn)) m |= 1u << ST_CA;
  if (task_first(c, PL_CAO) < (S::HT / p.nt_cao) * p.rgs_cao) m |= 1u << ST_CAO;
  if (task_first(c, PL_GU) < S::IT) m |= 1u << ST_GU;
  if (task_first(c, PL_DOWN) < (S::HT / p.nt_down) * S::SK || task_first(c, PL_RED) < p.nred) m |= 1u << ST_DOWN;
  const bool tout = task_first(c, PL_TOUT) < nout;
  if (tout || task_first(c, PL_TIN) < S::NIN) m |= 1u << ST_TAIL;
  if (tout) m |= 1u << TAIL_LAST_BIT;
  return m;
}

// the first stage after q in which this workgroup has a task (g = total if none)
__device__ __forceinline__ StagePos next_stage(unsigned mask, StagePos q, int total, int L) {
  while (true) {
    advance(q, L);
    if (q.g >= total) break;
    const int bit = q.l == L ? (q.g == total - 1 ? TAIL_LAST_BIT : ST_TAIL) : q.k;
    if ((mask >> bit) & 1u) break;
  }
  return q;
}

// ------------------------------------------------------------------------------------------------
template <int H, int I, bool W8, bool ROWWISE, bool YSHIFT = false, bool PAIRS = false, bool LONGSRC = false>
__global__ void __launch_bounds__(NTHREADS, 1) mkx_megakernel(Params params) {
  using S = Shape<H, I, W8, ROWWISE, YSHIFT, PAIRS, LONGSRC>;
  __shared__ __attribute__((aligned(1024))) char smem[S::LDS];
  CP& p = *(CP*)(__builtin_amdgcn_kernarg_segment_ptr());
  Ctx<S> c(p, smem);
  const float dt = p.dt[0];
  c.dt = dt;
  int* s_ks = (int*)(smem + S::SMALL + 3 * 1024);  // kv_start[MAX_BATCH], ca_len[MAX_BATCH]
  if (c.tid < p.B) {
    s_ks[c.tid] = min(max(p.kv_start[c.tid], 0), p.PM);
    s_ks[MAX_BATCH + c.tid] = min(max(p.ca_len[c.tid], 0), p.SP);
  }
  // A launch after one that timed out (timeout bit still set: the caller has not run mkx_check, which resets
  // the synchronisation state) does no work and returns NaN, so the failure cannot pass unnoticed. Only the
  // timeout bit decides: the range bit may be set by a workgroup of this very launch (its first stage stores
  // GEMM operands), and a workgroup that returned here would leave the others waiting for its arrivals. A
  // range error latched by an earlier launch still poisons this launch's output (the last step tail reads
  // both bits) until mkx_check reports it.
  if (__hip_atomic_load(&p.bar->err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & ERR_TIMEOUT) {
    if (c.wg == 0)
      for (int i = c.tid; i < p.B * p.T * p.A; i += NTHREADS) p.x_out[i] = __uint_as_float(0x7fc00000u);
    return;
  }
  BarCtx bc;
  bc.bs = p.bar;
  bc.x = xcc_id();
  bc.nx = p.nx[bc.x];
  bc.xmask = p.xmask;
  bc.spin_limit = p.spin_limit;
  bc.failed = false;
  bc.base = __hip_atomic_load(&p.bar->gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  bc.flags = p.flags;
  // one agent-scope acquire per launch: no cache of this XCD holds lines from before the launch
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  __syncthreads();
  if (p.profile && c.wg == 0 && c.tid == 0) p.prof[0] = clock100() * 10;

  const int total = 1 + p.n_steps * (STAGES_PER_LAYER * p.L + 1);
  // a workgroup goes from each of its stages straight to the next stage in which it has a task (its weight
  // or K/V prefetch for that task is issued right away), passing over the stages between
  const unsigned mask = task_mask(c);
  StagePos pos{0, -1, p.L, 0};
  Desc cur = describe(c, pos);
  for (int g = 0; g < total;) {
    {
      // parameters are re-read from the kernarg segment in every stage instead of being kept live (and
      // spilled) across the whole loop
      CP* pl = (CP*)__builtin_amdgcn_kernarg_segment_ptr();
      asm volatile("" : "+s"(pl));
      Ctx<S> c(*pl, smem);
      c.dt = dt;
      c.ep = (unsigned)g;
      if (cur.st == ST_SA) {
        if constexpr (S::PAIRS) sa_stage_pairs(c, cur, s_ks, bc, g);
        else sa_stage(c, cur, s_ks, bc, g);
      }
      else if (cur.st == ST_CA) {
        // (the CA_REG instantiations never run two-tile tasks: the host takes the two-tile instantiations for
        // fp8 launches that pair)
        if constexpr (S::RW && !S::CA_REG) {
          if (c.p.ca_grp) ca_stage_pairs(c, cur, s_ks, bc, g);
          else ca_stage(c, cur, s_ks, bc, g);
        } else {
          ca_stage(c, cur, s_ks, bc, g);
        }
      }
      else if (cur.st == ST_TAIL) tail_stage(c, cur, bc, g);
      else if constexpr (S::RW) gemm_stage_rows(c, cur, bc, g);
      else gemm_stage(c, cur, bc, g);
      if (g == 0) {
        transpose_caches(c, s_ks);
        split_shifts(c);
      }
    }
    c.ep = (unsigned)g;
    MKX_TR(c, 4);
    pos = next_stage(mask, pos, total, p.L);
    const int gn = pos.g;
    if (g == 0) {
      // the per-launch copies (V^T of the caches, split shifts) are read by every later stage (prefetches
      // included): the launch's one grid barrier
      wait_vm0();
      bar_arrive(bc, 1);
      bar_wait(bc, 1);
    } else {
      __syncthreads();  // this stage's LDS is no longer read: the next stage's prefetch may overwrite it
    }
    if (gn < total) {
      cur = describe(c, pos);
      // waves 1-3 issue the prefetch; wave 0, which polls the ready epochs, keeps no loads in flight
      if (c.wave != 0) {
        prefetch(c, cur, s_ks);
        prefetch_shifts(c, cur);
      }
    }
    c.ep = (unsigned)gn;
    MKX_TR(c, 6);
    // (workgroup 0 has no stage to pass over: gn = g + 1)
    if (p.profile && c.wg == 0 && c.tid == 0) p.prof[g + 1] = clock100() * 10;
    g = gn;
  }
  // every workgroup has passed (or passed over) every stage boundary: count them like barrier arrivals (the
  // arrival counters then read (gen + total) x workgroups, the state the next launch's barrier expects)
  wait_vm0();
  __syncthreads();
  if (c.tid == 0) __hip_atomic_fetch_add(&p.bar->arrive[bc.x][0], (unsigned long long)(total - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (c.wg == 0 && c.tid == 0) __hip_atomic_store(&p.bar->gen, bc.base + (unsigned long long)total, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace mkx
