/*
 * mkx — C ABI of the MI355X (gfx950) persistent megakernel for the Euler loop of a
 * flow-matching DiT action expert.
 *
 * The entry points replace the reference's Python expert-call boundary, class ExpertMegakernel in
 * src/mk_expert.py (muninn-huginn/reki-megakernel):
 *   mkx_create   <- ExpertMegakernel.__init__   (src/mk_expert.py:436-481: pack weights once, own scratch)
 *   mkx_run      <- ExpertMegakernel.run        (src/mk_expert.py:483-515: marshal caches, one launch)
 *   mkx_barriers <- ExpertMegakernel.barriers   (src/mk_expert.py:517-518: stage boundaries per launch)
 *   mkx_query    <- attributes the reference reads off the object (nprog, bar, prof; test_mk.py:44-45,
 *                   tune_mk.py:79-95)
 *   mkx_ring_append <- the register cache's per-frame append after each expert call (append_frame,
 *                   src/profile_breakdown.py:97-104) that refills past.register_step['mem_kv'] / cu_kv
 *   mkx_source_create / _run / _destroy <- the cross-attention source K/V of REKI's register_prepare
 *                   (mk_expert.py:22-24, 491-492: past.cross_attn_kv, which the expert call reads)
 *   mkx_modulations <- the final projection of REKI's _step_modulations (mk_expert.py:529), the mods rows
 *                   the kernel reads (mk_expert.py:336-340)
 *   mkx_destroy, mkx_last_error, mkx_status_string: lifetime and error reporting the Python object
 *                   had implicitly (the reference only asserts, src/mk_expert.py:444, 464, 480, 488, 496).
 *
 * Conventions: all tensor pointers are device pointers (hipMalloc'd or torch CUDA tensors). bf16 is
 * stored as uint16. Weight matrices are row-major [out, in] like torch.nn.Linear.weight, stacked over
 * layers exactly as the reference stacks them (src/mk_expert.py:445-460). No entry point aborts or
 * hangs on bad input: every one returns an mkx_status, and mkx_last_error() describes the last failure
 * on the calling thread.
 */
#ifndef MKX_H
#define MKX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MKX_ABI_VERSION 1
#define MKX_MAX_LAYERS 32

typedef enum {
  MKX_OK = 0,
  MKX_EINVAL = 1,        /* shape / dtype / pointer / stride invalid (reference: assert) */
  MKX_ENORESIDENT = 2,   /* the persistent grid cannot be co-resident (reference: hangs, README.md:262-263) */
  MKX_EHIP = 3,          /* a HIP runtime call failed; mkx_last_error() names it */
  MKX_ETIMEOUT = 4,      /* a barrier or ready-epoch wait exceeded its spin bound; results are invalid */
  MKX_ENOMEM = 5,
  MKX_EUNSUPPORTED = 6,  /* a shape the library has no kernel instantiation for */
  MKX_ERANGE = 7         /* a weight (at creation) or a GEMM operand (at run time) exceeds the fp16 range 65504
                            of the GEMM operands; a launch with such an operand returns NaN */
} mkx_status;

typedef enum { MKX_WEIGHTS_BF16 = 0, MKX_WEIGHTS_FP8_E4M3 = 1 } mkx_weight_dtype;
typedef enum { MKX_ACT_SILU = 0, MKX_ACT_GELU_TANH = 1 } mkx_activation;

typedef struct mkx_handle mkx_handle;

/* Expert shapes. Reference: read off the REKI model in ExpertMegakernel.__init__ (src/mk_expert.py:438-463). */
typedef struct {
  int32_t L;            /* layers */
  int32_t H;            /* width = NH * HD */
  int32_t NH;           /* heads (MHA: n_kv_heads == NH, src/mk_expert.py:444) */
  int32_t HD;           /* head dim (64) */
  int32_t I;            /* MLP width */
  int32_t A;            /* padded action width (action_in_proj.in_features, 32) */
  int32_t max_rows;     /* max own rows per sample, M_q = T_act + R_reg (reference: TP = 16) */
  int32_t max_batch;    /* max samples per launch */
  int32_t max_mem_rows; /* max PM (register-memory rows) */
  int32_t max_src_rows; /* max SP (padded cross-attention source rows) */
  int32_t weight_dtype; /* mkx_weight_dtype */
  int32_t activation;   /* mkx_activation (reference: SiLU, src/mk_expert.py:464) */
  float eps;            /* AdaRMS eps (input_layernorm.eps, src/mk_expert.py:461) */
  float qk_eps;         /* q/k RMSNorm eps (q_norm.eps, src/mk_expert.py:463) */
} mkx_dims;

/* Weights, stacked over layers (src/mk_expert.py:445-460). Linear weights are bf16, or e4m3 bytes with
 * per-output-channel fp32 scales when weight_dtype == MKX_WEIGHTS_FP8_E4M3 (the *_scale pointers are
 * then [L, out] and required; NULL for bf16). mkx_create copies them into the handle's own layout. */
typedef struct {
  const void* wqkv;   /* [L, 3H, H]  rows q;k;v (torch.cat of q_proj, k_proj, v_proj, :446-447) */
  const void* wo;     /* [L, H, H]   self_attn.o_proj */
  const void* wqca;   /* [L, H, H]   cross_attn.q_proj */
  const void* woca;   /* [L, H, H]   cross_attn.o_proj */
  const void* wg;     /* [L, I, H]   mlp.gate_proj */
  const void* wu;     /* [L, I, H]   mlp.up_proj */
  const void* wd;     /* [L, H, I]   mlp.down_proj */
  const float* wqkv_scale, *wo_scale, *wqca_scale, *woca_scale, *wg_scale, *wu_scale, *wd_scale;
  const void* qn;     /* [L, HD] bf16 self_attn.q_norm.weight (used as 1 + w) */
  const void* kn;     /* [L, HD] bf16 self_attn.k_norm.weight */
  const void* qcan;   /* [L, HD] bf16 cross_attn.q_norm.weight */
  const float* win;   /* [A, H] fp32: action_in_proj.weight transposed (:457) */
  const float* bin;   /* [H]    fp32 action_in_proj.bias */
  const float* wout;  /* [A, H] fp32 action_out_proj.weight */
  const float* bout;  /* [A]    fp32 action_out_proj.bias */
} mkx_weights;

/* One call: integrate n_steps Euler steps for B samples (src/mk_expert.py:483-515).
 * Own rows of sample b are [T_act action rows || R_reg register rows]; only the action rows feed the
 * step tail. Register rows take reg_tok as their layer-0 input in every step (reg_tok may be NULL when
 * R_reg == 0, the reference's layout). Per-layer caches are passed as arrays of L device pointers so
 * REKI-style per-layer tensors need no torch.stack (:489-492). Strides are in elements. */
typedef struct {
  const float* x_in;    /* [B, T_act, A] fp32: x after the previous step (reference: x_t after step 1) */
  float* x_out;         /* [B, T_act, A] fp32: x after the last step (may alias x_in) */
  const float* mods;    /* fp32 rows of MODW = 9 L H + 2 H: sample b, step s at mods + b*mods_stride_b +
                           (mod_row0 + s) * mods_stride_step (reference: mods[N, MODW], row 1 + s, :336) */
  int64_t mods_stride_b, mods_stride_step;
  int32_t mod_row0;     /* first modulation row used (1 for steps 2..N, 0 for step 1) */
  const float* dt;      /* [1] fp32 device scalar (reference: dt tensor, :320) */
  const void* memk[MKX_MAX_LAYERS];  /* per layer [B, PM, NH, HD] bf16, pre-normed and rotated (past.register_step['mem_kv']) */
  const void* memv[MKX_MAX_LAYERS];
  int64_t mem_stride_b;               /* elements between samples (PM*NH*HD when packed) */
  const int32_t* kv_start;            /* [B] first valid memory row (reference: cu_kv[0], :321) */
  const void* kca[MKX_MAX_LAYERS];    /* per layer [B, SP, NH, HD] bf16, pre-normed and rotated (past.cross_attn_kv) */
  const void* vca[MKX_MAX_LAYERS];
  int64_t src_stride_b;
  const int32_t* ca_len;              /* [B] valid source rows S (reference: cu_src[1], :322) */
  const float* sa_cos, *sa_sin;       /* [M_q, HD] fp32 RoPE of own rows in self-attention (past.register_step['sa_pe']) */
  const float* ca_cos, *ca_sin;       /* [M_q, HD] fp32 RoPE of own rows in cross-attention ('ca_pe') */
  const void* reg_tok;                /* [R_reg, H] bf16 register-row input, or NULL when R_reg == 0 */
  void* cur_k;                        /* optional out [L, B, R_reg, NH, HD] bf16: normed+rotated K of register rows, first step */
  void* cur_v;                        /* optional out [L, B, R_reg, NH, HD] bf16: V of register rows, first step */
  int32_t n_steps, action_dim, T_act, R_reg, B, PM, SP;
} mkx_step_args;

typedef enum {
  MKX_Q_GRID = 0,          /* workgroups in the persistent launch (reference: nprog = SM count, :473) */
  MKX_Q_BLOCK = 1,         /* threads per workgroup */
  MKX_Q_BARRIER_COUNT = 2, /* workgroup passages of stage boundaries since the last query (reference: mk.bar after the run, test_mk.py:44) */
  MKX_Q_ERROR_FLAG = 3,    /* device error flag of the last launch (spin bound exceeded = 1) */
  MKX_Q_PROFILE_LEN = 5,   /* entries of the caller's timestamp buffer, 0 when profiling is off */
  MKX_Q_WEIGHT_BYTES = 6,  /* bytes of packed linear weights streamed per Euler step */
  MKX_Q_LDS_BYTES = 7,     /* dynamic LDS per workgroup */
  MKX_Q_GEMM_FORM = 8,     /* GEMM form of the last launch: 0 passes, 1 row-wise, -1 before the first launch
                              (no reference counterpart: the reference has one form; tune_mk.py:69-72 overrides
                              its tile config instead) */
  MKX_Q_OPERAND_SHIFT = 9  /* the AdaRMS operand shift of later launches (mkx_set_operand_shift) */
} mkx_query_key;

/* ExpertMegakernel.__init__ (src/mk_expert.py:436-481). Validates dims, copies and repacks the weights
 * on `stream` (synchronised before return), allocates scratch, checks co-residency. Launches are
 * cooperative; with the environment variable MKX_PLAIN_LAUNCH=1 set at creation they are plain launches
 * of the same grid (one workgroup per CU, co-resident when the GPU runs nothing else), which some
 * profilers require. */
int mkx_create(const mkx_dims* dims, const mkx_weights* weights, void* stream, mkx_handle** out);

/* ExpertMegakernel.run (src/mk_expert.py:483-515): one persistent launch on `stream` (a hipStream_t;
 * NULL = default stream). Inputs are borrowed for the duration of the call. A handle's scratch is shared
 * by its calls: use one handle per stream (the reference is not re-entrant either). Asynchronous; call
 * mkx_check after synchronising to learn whether a barrier or ready-epoch wait timed out.
 * Scratch grows on the first call at a larger shape (n_steps, B * (T_act + R_reg), PM, SP), which
 * allocates and synchronises: under stream capture such a call returns MKX_EINVAL, and once any launch of
 * the handle has been captured a growing call returns MKX_EUNSUPPORTED (the graph holds the current
 * scratch). Warm up eagerly at the largest shape before capturing, or use a second handle.
 * A launch whose waits gave up writes NaN into x_out, and so does every later launch on the handle (doing no
 * other work) until mkx_check resets the synchronisation state. */
int mkx_run(mkx_handle* h, const mkx_step_args* args, void* stream);

/* Reads the device error flag of the last launch (synchronises `stream`): MKX_OK, MKX_ETIMEOUT, or MKX_ERANGE
 * (a GEMM operand beyond the fp16 range; that launch returned NaN), and then resets the handle's
 * synchronisation state, so the next launch runs normally. */
int mkx_check(mkx_handle* h, void* stream);

/* Spin bound of every grid-barrier and ready-epoch wait of later launches, in polls (0 = the default,
 * 2^20 polls, about 0.5 s). A wait that exceeds it sets the error flag and every later wait of the launch
 * returns at once, so a launch that cannot complete still drains. No counterpart in the reference, whose
 * grid barrier spins without bound (README.md:262-263); tests use a tiny bound to exercise the path. */
int mkx_set_spin_limit(mkx_handle* h, uint32_t polls);

/* AdaRMS operand shift of later launches: the fp16 GEMM operand y = h (1 + scale) of every AdaRMS is stored as
 * y 2^-shift, with the sums of squares of h 2^-shift and eps 2^-2 shift, so that the row's rsqrt(ss / H + eps)
 * carries the factor 2^shift back (exact powers of two; 0, the default, leaves every result bit unchanged).
 * The remedy for MKX_ERANGE from mkx_check: a residual stream whose y passes 65504 overflows the fp16 operand
 * (the launch returns NaN); with shift s it may reach 65504 2^s. Entries of y below 6.1e-5 2^s fall into
 * fp16's subnormal range and keep fewer significant bits, so a shift is for checkpoints that need it. No
 * counterpart in the reference, whose bf16 operands have no such limit (src/mk_expert.py:119). MKX_EINVAL
 * unless 0 <= shift <= 30. */
int mkx_set_operand_shift(mkx_handle* h, int32_t shift);

/* ExpertMegakernel.barriers (src/mk_expert.py:517-518): stage boundaries one launch of n_steps passes
 * (1 + n_steps (7 L + 1); the first is a grid barrier, the others per-task ready epochs). */
int64_t mkx_barriers(const mkx_handle* h, int32_t n_steps);

/* Per-boundary timestamps (tune_mk.py PROFILE mode, src/mk_expert.py:66-69): later launches store, from
 * workgroup 0, the ns clock when it passes stage boundary nb into buf[nb] (buf[0] = launch start). buf is a caller-owned
 * device int64 array of len entries (>= mkx_barriers(n_steps) + 1); NULL turns profiling off. */
int mkx_set_profile(mkx_handle* h, int64_t* buf, int32_t len);

/* Register-memory ring append, the step after an expert call (no handle needed). Reference: the memory
 * the expert reads, past.register_step['mem_kv'] with kv_start = cu_kv[0] (src/mk_expert.py:489-490, 321),
 * which REKI's register cache refills after every call from the call's register rows (append_frame,
 * timed at src/profile_breakdown.py:97-104; 32 register tokens per frame kept over 3 frames, README.md:27).
 * Per layer l and sample b, memory rows [kv_start, PM) are valid, K normed and rotated at the row index.
 * Out row j = in row j + R for j < PM - R (K rotated by shift_cos/shift_sin, normally -R positions),
 * else the call's register row j - (PM - R) of cur_k/cur_v (K rotated by new_cos/new_sin, from its
 * position in the call to row j); rows below kv_start_out = max(kv_start_in - R, 0) are zeroed. kv_start_in
 * is clamped to [0, PM]. NULL tables mean no rotation. Rotations are fp32 products and one sum per
 * element (no fused multiply-add), rounded to bf16 to nearest even. Out buffers must not overlap the in
 * buffers (ping-pong two sets); asynchronous on `stream`. */
typedef struct {
  int32_t L, B, NH, HD;   /* HD must be 64 */
  int32_t PM;             /* memory rows per sample */
  int32_t R;              /* rows appended per call, 1 <= R <= PM */
  const void* cur_k;      /* [L, B, R, NH, HD] bf16 register-row K of the call (normed, rotated; run_first's cur_k) */
  const void* cur_v;      /* [L, B, R, NH, HD] bf16 */
  const void* memk_in[MKX_MAX_LAYERS];  /* per layer [B, PM, NH, HD] bf16 */
  const void* memv_in[MKX_MAX_LAYERS];
  void* memk_out[MKX_MAX_LAYERS];       /* per layer [B, PM, NH, HD] bf16 */
  void* memv_out[MKX_MAX_LAYERS];
  int64_t mem_stride_b;                  /* elements between samples, in and out buffers */
  const int32_t* kv_start_in;            /* [B] device */
  int32_t* kv_start_out;                 /* [B] device, not aliasing kv_start_in */
  const float* shift_cos;                /* [HD] fp32 rotation of kept rows, or NULL */
  const float* shift_sin;
  const float* new_cos;                  /* [HD] fp32 rotation of appended rows, or NULL */
  const float* new_sin;
} mkx_ring_args;

int mkx_ring_append(const mkx_ring_args* args, void* stream);

/* Cross-attention source caches: per layer l, K = norm_rope(bf16(ctx Wk[l]^T)) and V = bf16(ctx Wv[l]^T)
 * as bf16 [B, SP, NH, 64], rows >= ca_len[b] zero. Reference: past.cross_attn_kv (src/mk_expert.py:491-492),
 * made by REKI's register_prepare (mk_expert.py:22-24; README.md:279-281: "the cross-attention K/V
 * projections of the VLM source (31 M weights)"). norm_rope: per head, x * rsqrt(mean(x^2) + eps) *
 * (1 + k_norm[l]) rounded to bf16, then x * cos + rotate_half(x) * sin at the row's source position,
 * rounded to bf16. fp32 accumulation on bf16 MFMA.
 * mkx_source_create copies and repacks the weights once (synchronising `stream`) and owns a context
 * staging buffer of max_rows rows; mkx_source_run is asynchronous on `stream`, and calls on one handle
 * share that buffer (one handle per stream). */
typedef struct mkx_source mkx_source;

typedef struct {
  int32_t L, NH, HD;       /* HD must be 64 */
  int32_t C;               /* context width, a multiple of 32 */
  int32_t max_rows;        /* max B * SP per call */
  float eps;               /* k-norm eps (cross_attn.k_norm.eps) */
} mkx_source_dims;

typedef struct {
  int32_t B, SP;           /* samples, source rows per sample (padded); B * SP <= max_rows */
  const void* ctx;         /* [B, SP, C] bf16 VLM context, 16-byte aligned */
  const int32_t* ca_len;   /* [B] device: valid source rows (clamped to [0, SP]) */
  const float* cos;        /* [SP, 64] fp32 RoPE table of source positions */
  const float* sin;
  void* kca[MKX_MAX_LAYERS]; /* per layer [B, SP, NH, 64] bf16 out, 8-byte aligned */
  void* vca[MKX_MAX_LAYERS];
  int64_t src_stride_b;    /* elements between samples of kca / vca */
} mkx_source_args;

/* wk, wv: [L, NH * 64, C] bf16 cross_attn.k_proj / v_proj weights stacked over layers; k_norm: [L, 64]
 * bf16 cross_attn.k_norm.weight (used as 1 + w). All device pointers. */
int mkx_source_create(const mkx_source_dims* dims, const void* wk, const void* wv, const void* k_norm, void* stream,
                      mkx_source** out);
int mkx_source_run(mkx_source* h, const mkx_source_args* args, void* stream);

/* mkx_source_run for callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc); no counterpart in the reference. Same arguments, kernels and
 * results as mkx_source_run, but the call's packed context is staged in a static device array of the
 * library (16 MiB per GPU, held until the process ends) instead of the handle's buffer, and the call
 * allocates nothing. A context whose packed form ((ceil32(B * SP) + 160) rows of C * 2 bytes: the rows rounded
 * up to 32 plus 160 rows of padding for the largest workgroup's reads) exceeds 16 MiB is refused with MKX_EINVAL. Every call on one GPU shares that array: calls that overlap on one GPU
 * (concurrent streams, other threads) race and must be serialised by the caller. */
int mkx_source_run_noalloc(mkx_source* h, const mkx_source_args* args, void* stream);
int mkx_source_destroy(mkx_source* h);

/* Modulation projection: out[r][n] = sum_k silu(c[r][k]) w[n][k] + bias[n], every AdaRMS scale, shift and
 * gate of every layer and Euler step of a call in one product (N = MODW = 9 L H + 2 H). Reference: the
 * mods rows the expert reads (src/mk_expert.py:336-340), made by REKI's _step_modulations
 * (mk_expert.py:529: mods, dt = model._step_modulations(num_steps, state_cond)), whose last layer this is.
 * fp32 in and out, bf16 weights; silu(c) is split into bf16 hi + lo MFMA operands. Asynchronous. */
typedef struct {
  int32_t R;               /* rows: samples x Euler steps */
  int32_t K;               /* input width H: 256, 512, 768 or 1024 */
  int32_t N;               /* output columns, a multiple of 16 */
  const float* c;          /* [R, c_stride] fp32, 16-byte aligned: the input before the final SiLU */
  int64_t c_stride;        /* a multiple of 4 */
  const void* w;           /* [N, K] bf16, 16-byte aligned */
  const float* bias;       /* [N] fp32, 16-byte aligned */
  float* out;              /* [R, out_stride] fp32, 16-byte aligned */
  int64_t out_stride;      /* a multiple of 4 */
  int32_t w_fragment_order; /* 0: w row-major [N, K]; 1: w pre-packed as [N / 16][K / 32][64][8] with
                               element (g, t, l, e) = W[16 g + l % 16][32 t + 8 (l / 16) + e] */
} mkx_modproj_args;

int mkx_modulations(const mkx_modproj_args* args, void* stream);

/* Modulation input: c[b][k] = silu(temb(t_k) W1^T + b1) W2^T + b2 + state_cond[b] for the Euler schedule
 * t_k = 1 - k / N (k < N), temb(t) = [cos(1000 t f_i) | sin(1000 t f_i)], f_i = 10000^(-i / (tdim / 2)): the small
 * MLP whose output mkx_modulations projects, the rest of REKI's _step_modulations (src/mk_expert.py:529:
 * mods, dt = model._step_modulations(num_steps, state_cond)) in one launch. bf16 weights, fp32 biases, input
 * and output; the embedding is computed in fp64 and rounded to fp32. Asynchronous. */
typedef struct {
  int32_t N;               /* Euler steps (rows per sample), 1 .. 4096 */
  int32_t B;               /* samples, >= 1 */
  int32_t H;               /* width: 256, 512, 768 or 1024 */
  int32_t tdim;            /* embedding width: a multiple of 32, 32 .. 512 */
  const void* t1_w;        /* [H, tdim] bf16, 16-byte aligned */
  const float* t1_b;       /* [H] fp32, 16-byte aligned */
  const void* t2_w;        /* [H, H] bf16, 16-byte aligned */
  const float* t2_b;       /* [H] fp32, 16-byte aligned */
  const float* state_cond; /* [B, sc_stride] fp32, 16-byte aligned */
  int64_t sc_stride;       /* a multiple of 4, >= H */
  float* out;              /* c: element (b, k, n) at b * out_stride_b + k * out_stride_k + n, 16-byte aligned */
  int64_t out_stride_b;    /* multiples of 4 */
  int64_t out_stride_k;
} mkx_modin_args;

int mkx_modulation_input(const mkx_modin_args* args, void* stream);

/* Synchronisation micro-benchmarks (no handle). Reference: the barrier-only kernel _barrier_only
 * (src/tune_mk.py:28-33), timed at :66-68 to price the reference's grid barrier (results/opt/tune/v5.json:3-4).
 * MKX_PROBE_BARRIER: every workgroup of a one-per-CU grid passes n grid barriers (this library's barrier,
 * the one the Euler launch runs after its first stage) with nothing between them; reports microseconds per
 * barrier. MKX_PROBE_HANDOFF: a chain of n hand-offs between two groups of `fan` workgroups on different
 * XCDs: a producer stores `bytes` write-through, waits for the acknowledgements and publishes a ready epoch;
 * `fan` consumers poll the epoch and then load all `bytes`; a consumer produces the next hand-off. Reports
 * microseconds per hand-off: the cost of one stage boundary of the Euler launch for an operand of that size.
 * Launches `reps` times (median and minimum reported); allocates and frees its own buffers; synchronous. */
typedef enum { MKX_PROBE_BARRIER = 0, MKX_PROBE_HANDOFF = 1 } mkx_probe_kind;
typedef struct {
  int32_t kind;       /* mkx_probe_kind */
  int32_t n;          /* barriers, or hand-offs in the chain: even, 2 .. 2048 */
  int32_t bytes;      /* hand-off: bytes each consumer loads: 4096, 24576 or 73728 */
  int32_t fan;        /* hand-off: consumers per hand-off, 1 .. CUs / 2 */
  int32_t reps;       /* launches, 1 .. 100 */
  int32_t timed_out;  /* out: 1 if a wait of some launch exceeded its spin bound (the times are then invalid) */
  int32_t xcd_first[2]; /* out, hand-off: the XCDs of the first producer and its first consumer (workgroups 0, 1) */
  double us_median;   /* out: microseconds per barrier or hand-off, median over the launches */
  double us_min;      /* out: the fastest launch's */
} mkx_probe_args;

int mkx_probe(mkx_probe_args* args, void* stream);

int64_t mkx_query(const mkx_handle* h, int32_t key);
int mkx_destroy(mkx_handle* h);
const char* mkx_last_error(void);
const char* mkx_status_string(int status);
int32_t mkx_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* MKX_H */
