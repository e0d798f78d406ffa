/*
 * th_hip.h -- C ABI of libth_hip.so, the MI355X (gfx950) kernel library that
 * executes torch-helion OpIR kernels.
 *
 * Every entry point is extern "C", takes plain pointers and sizes, and never
 * aborts: it returns TH_OK (0) or a negative th_status and leaves a message in
 * th_last_error() (thread-local). Launches are asynchronous on the stream
 * passed in (a hipStream_t, NULL = the default stream). The caller owns every
 * device buffer. Descriptors are validated on the host before any launch.
 *
 * In the reference, one OpIR KernelSpec becomes one generated Helion kernel
 * module whose host function allocates its outputs and returns them
 * (reference: src/torch_helion/codegen/emit.py:188-221 gemm, :254-324 ssd,
 * :327-357 attention, driven by emit_program at codegen/emit.py:500-520 and
 * executed numerically only by codegen/interpret.py:18-51). Here the same
 * KernelSpec becomes one call below with caller-allocated outputs.
 */
#ifndef TH_HIP_H
#define TH_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TH_ABI_VERSION 7

typedef enum th_status {
  TH_OK = 0,
  TH_ERR_INVALID = -1,     /* bad descriptor: null pointer, bad shape/stride */
  TH_ERR_UNSUPPORTED = -2, /* valid request this build has no kernel for */
  TH_ERR_HIP = -3,         /* a HIP runtime call failed */
  TH_ERR_NOT_INIT = -4     /* th_init was not called for the current device */
} th_status;

typedef enum th_dtype {
  TH_F32 = 0,
  TH_BF16 = 1,
  TH_F16 = 2,
  TH_F8E4M3 = 3, /* OCP float8_e4m3fn (max 448) */
  TH_I32 = 4,
  TH_I64 = 5
} th_dtype;

/* ------------------------------------------------------------------ setup */

/* ABI version of the loaded library (TH_ABI_VERSION it was built with). */
int th_abi_version(void);

/* Select and initialise a device: checks it is gfx950 and raises the LDS
 * limit of the kernels that need more than 64 KiB. Call once per device. */
int th_init(int device);

/* Message of the last failing call on this thread ("" if none). */
const char* th_last_error(void);

/* --------------------------------------------------------------- gemm kind
 * OpIR `gemm` KernelSpec (reference: optimizer/opir.py:13-20, executed by
 * codegen/interpret.py:22-35, emitted by codegen/emit.py:188-221):
 *   acc_i = lhs[M, K] @ rhs_i[K, N]          (i < n_acc, all sharing lhs)
 *   r     = (sumsq * inv_k + eps) ^ -1/2,    sumsq = sum_k lhs^2   (optional)
 *   a_i   = acc_i * r  if bit i of rscale_mask else acc_i
 * With lhs_gain (TH_F8E4M3 weights only) the products use lhs[m, k] * g[k]
 * while sumsq stays the sum of the unscaled lhs^2: the RMSNorm gain sits on
 * the activation side, (x r g) W = r ((x g) W), so the weights are the
 * model's own, not diag(g) W (whose quantisation would differ).
 * followed by a fixed catalogue of fused output ops (th_epi_op) that the
 * Python lowering matches against the kernel's epilogue SSA. Epilogues
 * outside the catalogue run as TH_EPI_ACC (fp32) + th_epilogue_vm.
 */
typedef enum th_epi_op {
  TH_EPI_ACC = 0,          /* a_i                                            */
  TH_EPI_ROPE = 1,         /* a_i*cos + rotate_half_heads(a_i)*sin           */
  TH_EPI_ROPE_PAIR = 2,    /* a_i*cos + a_j*sin  (a_j = pre-rotated acc)     */
  TH_EPI_SILU = 3,         /* a_i * sigmoid(a_i)                             */
  TH_EPI_SWIGLU = 4,       /* (a_i * sigmoid(a_i)) * a_j                     */
  TH_EPI_ADD = 5,          /* a_i + extra_e                                  */
  TH_EPI_SOFTPLUS_ADD = 6, /* log(1 + exp(a_i + extra_e))                    */
  TH_EPI_MUL = 7           /* a_i * extra_e                                  */
} th_epi_op;

#define TH_MAX_ACC 4
#define TH_MAX_OUT 6
#define TH_MAX_EXTRA 4

typedef struct th_epi_out {
  int32_t op;     /* th_epi_op */
  int32_t a, b;   /* accumulator indices (b only for ROPE_PAIR / SWIGLU) */
  int32_t e;      /* extra operand index for ADD / SOFTPLUS_ADD / MUL, else -1 */
  void* ptr;      /* [M, N] row-major output (or [M, col_end - col_begin], see below) */
  int64_t ld;     /* row stride of ptr, in elements */
  int32_t dtype;  /* TH_F32 or TH_BF16 */
  /* Column window: the output holds accumulator columns [col_begin, col_end)
   * only, column n at ptr[m * ld + n - col_begin]; its extra operand is read
   * at the same relative column. Both multiples of 8 (and of the RoPE head
   * dim for ROPE ops); col_end = 0 means N. Several outputs with disjoint
   * windows of one accumulator are how one launch computes sibling
   * projections of a shared input (bf16 / fp32 only). */
  int32_t col_begin, col_end;
  int32_t pad_;
} th_epi_out;

typedef struct th_gemm_desc {
  int64_t M, N, K;
  int32_t n_acc;          /* 0 .. TH_MAX_ACC */
  int32_t in_dtype;       /* TH_BF16 (MFMA bf16), TH_F32 (MFMA f32), or TH_F8E4M3:
                             bf16 lhs x e4m3 rhs with per-column scales (M <= 128) */
  const void* lhs;        /* [M, K] row-major, in_dtype */
  int64_t ld_lhs;
  const void* rhs_packed; /* th_gemm_pack_rhs output for (N, K, n_acc, in_dtype) */
  int32_t sumsq;          /* 1: compute the RMS row scale r */
  uint32_t rscale_mask;
  float inv_k, eps;
  int32_t n_extra;
  int32_t pad_;
  const void* extra[TH_MAX_EXTRA]; /* [M, N] operands read at the output tile */
  int64_t ld_extra[TH_MAX_EXTRA];
  int32_t extra_dtype[TH_MAX_EXTRA];
  const float* rope_cos;  /* [rope_period, rope_head_dim] fp32 (ROPE ops) */
  const float* rope_sin;
  int32_t rope_head_dim;  /* columns of one head; rotation pairs n, n+hd/2 */
  int32_t rope_period;    /* table row = output row % rope_period */
  int32_t n_out;
  int32_t pad2_;
  th_epi_out out[TH_MAX_OUT];
  float* sumsq_out;       /* optional [M] fp32: raw sum_k lhs^2 */
  const float* rhs_scale; /* TH_F8E4M3: [n_acc][N] fp32, acc_i[:, n] *= rhs_scale[i*N + n] */
  float* workspace;       /* th_gemm_workspace_bytes(...) bytes, 16-byte aligned: required for TH_F8E4M3;
                             optional for TH_F32 (small grids then split K over workgroups through it) */
  int64_t workspace_bytes;
  const float* lhs_gain;  /* optional [K] fp32 per-column gain of lhs (TH_F8E4M3 only; 16-byte aligned) */
  const float* rs_parts;  /* optional [M, n_rs_parts] fp32, row stride ld_rs_parts (TH_BF16, or TH_F8E4M3
                             without lhs_gain; with sumsq): each row's sum of squares is the in-order
                             sum of these parts instead of sum_k lhs^2, for an lhs whose producer
                             applied an RMSNorm gain and kept the sums of the unscaled values
                             (th_ssd_chunked's y_gain, rs_parts; th_gemm's gain_out, ss_parts_out).
                             n_rs_parts and ld_rs_parts multiples of 4, 16-byte aligned. No
                             counterpart in the reference (its RMSNorm is one kernel). */
  int64_t ld_rs_parts;
  int32_t n_rs_parts;
  int32_t pad3_;
  const float* gain_out;  /* optional [N] fp32, 16-byte aligned (TH_F8E4M3 weights): output gain_out_index,
                             a bf16 output over all N columns, is stored as bf16(bf16(v) * gain_out[n])
                             instead of v, and ss_parts_out receives each row's sum of bf16(v)^2 in
                             parts of 256 columns: the next GEMM's lhs with its RMSNorm gain applied,
                             and the sums that GEMM's rs_parts takes. N a multiple of 1024. No
                             counterpart in the reference (its RMSNorm is one kernel). */
  float* ss_parts_out;    /* with gain_out: [M, N / 256] fp32, row stride ld_ss_parts_out, 16-byte aligned */
  int64_t ld_ss_parts_out;
  int32_t gain_out_index;
  int32_t pad4_;
} th_gemm_desc;

/* Per-accumulator column tile th_gemm uses for (N, n_acc, in_dtype) when an
 * output is fused RoPE; a block computes n_acc * tile columns, and fused RoPE
 * (TH_EPI_ROPE) needs the tile to be a multiple of the head dim. (Without
 * RoPE, one bf16 accumulator over a multiple of 256 columns may run on
 * 256-column tiles instead, which the packed layout allows.) Returns 0 for
 * invalid arguments. */
int th_gemm_acc_tile(int64_t N, int32_t n_acc, int32_t in_dtype);

/* Bytes of the packed right-hand side for th_gemm (weights are packed once
 * at upload; activation operands are packed per call into a workspace). */
int64_t th_gemm_packed_bytes(int64_t N, int64_t K, int32_t n_acc, int32_t in_dtype);

/* Pack n_acc row-major [K, N] operands (dtype src_dtype, row stride ld_src)
 * into the K-contiguous, accumulator-interleaved layout th_gemm reads
 * (TH_F8E4M3: e4m3 bytes in, copied unchanged).
 * Replaces the reference's per-kernel weight arguments w0..w{n-1}
 * (optimizer/partition.py:121-124, bound at codegen/emit.py:469-476). */
int th_gemm_pack_rhs(const void* const* src, const int64_t* ld_src, int32_t src_dtype,
                     int64_t N, int64_t K, int32_t n_acc, int32_t in_dtype,
                     void* packed, void* stream);

/* Workspace th_gemm uses for these sizes: 0 for TH_BF16; for TH_F8E4M3 the
 * split-K partial sums it needs; for TH_F32 grids too small to occupy the GPU,
 * the partial sums of the split over workgroups (optional: without it the K
 * loop is split inside each workgroup), else 0. -1 for invalid arguments. */
int64_t th_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t n_acc, int32_t in_dtype);

/* One OpIR gemm KernelSpec. */
int th_gemm(const th_gemm_desc* desc, void* stream);

/* th_gemm that allocates nothing and takes no workspace. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops such as the decode step, harnesses
 * that forbid hipMalloc). With TH_F8E4M3 weights the split-K partial sums live
 * in a file-scope device array of TH_GEMM_NOALLOC_SCRATCH_BYTES per GPU (held
 * until the process ends); desc->workspace is ignored, and sizes that need
 * more (th_gemm_workspace_bytes) are refused with TH_ERR_INVALID. Every call on
 * one GPU shares that array and nothing in it needs to start at zero, so calls
 * that overlap on one GPU (on concurrent streams) race; calls in stream order
 * do not. bf16 / fp32 weights need no scratch: the call is th_gemm. */
#define TH_GEMM_NOALLOC_SCRATCH_BYTES (32 << 20)
int th_gemm_noalloc(const th_gemm_desc* desc, void* stream);

/* ------------------------------------------------------------ RMSNorm
 * The stand-alone normalisation kernel (gemm kind with gemms=[] and sumsq;
 * reference: optimizer/partition.py:165-177, optimizer/passes.py:357-370):
 *   out[m, :] = x[m, :] * (sum_k x[m,k]^2 * inv_k + eps)^-1/2 * gain[:]
 */
typedef struct th_rmsnorm_desc {
  int64_t M, K;
  const void* x; int64_t ld_x; int32_t x_dtype;
  int32_t out_dtype;
  const float* gain;      /* [K] fp32 */
  void* out; int64_t ld_out;
  float inv_k, eps;
  float* out32; int64_t ld_out32;   /* optional fp32 copy of out */
} th_rmsnorm_desc;

int th_rmsnorm(const th_rmsnorm_desc* desc, void* stream);

/* --------------------------------------------------------- attention kind
 * softmax(q k^T * scale [+ causal mask]) v over [B, S, H, d] views of
 * token-major [B*S, H*d] tensors (reference: optimizer/evaluate.py:139-146,
 * codegen/emit.py:327-357). Extended with grouped KV heads (heads_q is a
 * multiple of heads_kv; q head h reads kv head h / (heads_q / heads_kv)) and
 * a causal flag (query i sees keys j <= i + seq_kv - seq_q).
 */
typedef struct th_attn_desc {
  int32_t batch, seq_q, seq_kv, heads_q, heads_kv, head_dim;
  float scale;
  int32_t causal;
  int32_t dtype;          /* TH_BF16 or TH_F32 for q, k, v and o */
  int32_t pad_;
  const void* q; int64_t ld_q;  /* row stride in elements (>= heads*head_dim) */
  const void* k; int64_t ld_k;
  const void* v; int64_t ld_v;
  void* o; int64_t ld_o;
} th_attn_desc;

int th_attention_prefill(const th_attn_desc* desc, void* stream);

/* ------------------------------------------------------ decode attention
 * One new query token per sequence against a KV cache: for every sequence b
 * and query head h (kv head h / (heads_q / heads_kv)),
 *   o[b, h] = softmax(q[b, h] . K[b, 0:len_b, kvh]^T * scale) V[b, 0:len_b, kvh]
 * The reference has no decode path; this is the attention kind of
 * optimizer/evaluate.py:139-146 with one query row and a cache laid out as
 * [batch][max_len][heads_kv][head_dim] (element strides below). The keys of a
 * sequence are split n_split ways (0 = chosen by the library); with more than
 * one split the partial results go through the workspace.
 */
typedef struct th_decode_desc {
  int32_t batch, heads_q, heads_kv, head_dim;  /* head_dim 64 or 128, heads_q/heads_kv <= 16 */
  int32_t max_len;        /* cache capacity in tokens */
  int32_t n_split;        /* 0: choose; else the number of key ranges per (sequence, kv head) */
  int32_t fixed_len;      /* keys per sequence when lengths is NULL (1..max_len) */
  int32_t dtype;          /* TH_BF16 for q, caches and o */
  float scale;
  int32_t pad_;
  const int32_t* lengths; /* optional [batch] device array of valid keys per sequence, 1..max_len
                             (a value outside that range is clamped to it) */
  const void* q; int64_t ld_q;                         /* [batch, heads_q*head_dim] */
  const void* k_cache; int64_t k_stride_b, k_stride_t; /* element strides: sequence, token (< 2^24) */
  const void* v_cache; int64_t v_stride_b, v_stride_t;
  void* o; int64_t ld_o;                               /* [batch, heads_q*head_dim] */
  float* workspace; int64_t workspace_bytes;
} th_decode_desc;

/* Workspace th_attention_decode needs for these sizes (0 when it needs none). */
int64_t th_attention_decode_workspace_bytes(int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t head_dim,
                                            int32_t max_len, int32_t n_split);

int th_attention_decode(const th_decode_desc* desc, void* stream);

/* ------------------------------------------------------------ SSD scan
 * The Mamba-2 scan, per (batch b, head h) over token-major operands:
 *   y_t = sum_{s<=t} (C_t . B_s) exp(cum_t - cum_s) dt_s x_s + D_h x_t  [* gate_t]
 * evaluated chunk by chunk (states of each chunk, an inter-chunk carry, then
 * the outputs) with every exponent a difference of running sums inside one
 * chunk or between chunk ends, so nothing overflows at any length. (The
 * bf16 path splits some of these differences in two at a block boundary,
 * which keeps both parts <= 0 when dt*A <= 0 everywhere, as Mamba's
 * A = -exp(A_log) and dt = softplus(.) guarantee.)
 * Two operand forms:
 *   ssd_chunked kind (new): cum = running sum of dt*A, with dt [T, H] and A [H];
 *   ssd kind (reference: optimizer/evaluate.py:123-138, codegen/emit.py:254-324):
 *   cum and dt given as [T, H*pad] with one value per head group (column
 *   h*pad), D given as a full [T, H*P] constant.
 * B/C are shared by heads_per_group = heads / ngroups heads.
 */
typedef struct th_ssd_desc {
  int32_t batch, seq, heads, head_dim, state_dim, ngroups, chunk;
  int32_t dtype;                      /* TH_BF16 or TH_F32: x, b, c, dt, cum, dskip, gate */
  const void* x;  int64_t ld_x;       /* [B*S, H*P] */
  const void* b;  int64_t ld_b;       /* [B*S, G*N] */
  const void* c;  int64_t ld_c;       /* [B*S, G*N] */
  const void* dt; int64_t ld_dt;      /* [B*S, H*dt_stride] */
  int32_t dt_stride;                  /* columns between heads in dt and cum (1 or pad) */
  int32_t pad_;
  const void* cum; int64_t ld_cum;    /* NULL: cum from dt and A; else precomputed running sum */
  const float* A;                     /* [H] (used when cum == NULL) */
  const float* D;                     /* [H] or NULL */
  const void* dskip; int64_t ld_dskip;/* optional full [B*S, H*P] D (reference form) */
  const void* gate; int64_t ld_gate;  /* optional [B*S, H*P] multiplier of the result */
  int32_t gate_dtype, y_dtype;
  void* y; int64_t ld_y;              /* [B*S, H*P] */
  float* y32; int64_t ld_y32;         /* optional fp32 copy of y */
  float* workspace;                   /* th_ssd_workspace_bytes(...) bytes, or
                                         th_ssd_gtile_workspace_bytes(...) (16-byte aligned) */
  int64_t workspace_bytes;
  const float* y_gain;                /* optional [H*P] fp32 (16-byte aligned): y is stored times this
                                         per-column gain (the next RMSNorm's); bf16 y of 16-byte aligned
                                         rows, no y32 or dskip, head_dim a multiple of 32 (the MFMA path) */
  float* rs_parts;                    /* with y_gain: [B*S, H*P/32] fp32, row stride ld_rs_parts: per
                                         token and 32-column block, the sum of squares of y before the
                                         gain (th_gemm's rs_parts). No counterpart in the reference. */
  int64_t ld_rs_parts;
} th_ssd_desc;

int64_t th_ssd_workspace_bytes(int32_t batch, int32_t seq, int32_t heads, int32_t head_dim,
                               int32_t state_dim, int32_t chunk);

/* The workspace th_ssd_chunked runs fastest with: th_ssd_workspace_bytes plus,
 * for state_dim 128 with several heads per B/C group, the chunks' G^T = C_t B_s^T
 * tiles of every group. When the workspace holds them (and the bf16 MFMA path
 * runs), the state pass forms each chunk's tiles once per group, its work dealt
 * over the group's heads, and the output pass reads them instead of every head
 * forming them again; the results are the same bits either way. For other shapes
 * the tiles save less than they cost to store and reload, and the size is
 * th_ssd_workspace_bytes's. No counterpart in the reference (its ssd kind is one
 * dense expression, optimizer/evaluate.py:123-138). -1 for invalid arguments. */
int64_t th_ssd_gtile_workspace_bytes(int32_t batch, int32_t seq, int32_t heads, int32_t head_dim,
                                     int32_t state_dim, int32_t chunk, int32_t ngroups);

/* One OpIR ssd / ssd_chunked KernelSpec. */
int th_ssd_chunked(const th_ssd_desc* desc, void* stream);

/* --------------------------------------------------------- conv1d kind
 * Depthwise causal convolution over each sequence of a token-major tensor
 * (reference eager definition: models/mamba.py:278-283, not capturable there):
 *   y[b,t,ch] = act( sum_{j<k} w[ch,j] * x[b, t-(k-1)+j, ch] ),  x = 0 before t = 0
 */
typedef struct th_conv_desc {
  int32_t batch, seq, width, kernel;
  int32_t activation;                 /* 0 none, 1 SiLU */
  int32_t x_dtype, y_dtype;
  int32_t pad_;
  const void* x; int64_t ld_x;        /* [B*S, width] */
  const float* w;                     /* [width, kernel] fp32 */
  void* y; int64_t ld_y;
  float* y32; int64_t ld_y32;         /* optional fp32 copy */
} th_conv_desc;

int th_conv1d_causal(const th_conv_desc* desc, void* stream);

/* ------------------------------------------------------- embedding kind
 * Row gather of a token-embedding table (the `embedding` OpGraph op that
 * the capture handler makes of aten.embedding; the reference's MambaModel
 * has no embedding and takes float [B,S,D] hidden states,
 * models/mamba.py:343-359):
 *   out[t, :] = table[ids[t], :]
 * An id outside [0, vocab) writes a row of zeros and, when n_invalid is
 * given, adds 1 to *n_invalid (the caller zeroes it; torch raises instead).
 */
typedef struct th_embedding_desc {
  int64_t tokens;                     /* number of ids */
  int32_t dim, vocab;
  int32_t dtype;                      /* TH_BF16 or TH_F32: table and out */
  int32_t ids_dtype;                  /* TH_I64 or TH_I32 */
  const void* table; int64_t ld_table;  /* [vocab, dim] */
  const void* ids;                    /* [tokens], contiguous */
  void* out; int64_t ld_out;          /* [tokens, dim] */
  float* out32; int64_t ld_out32;     /* optional fp32 copy */
  int32_t* n_invalid;                 /* optional device counter */
} th_embedding_desc;

int th_embedding(const th_embedding_desc* desc, void* stream);

/* ------------------------------------------------- epilogue VM (fallback)
 * Evaluates an OpIR epilogue SSA (registered ops, reference:
 * capture/ops.py:34-37, executed as in codegen/interpret.py:27-34) that the
 * fused catalogue does not cover. Operands are [M, N] tensors or [M, 1]
 * columns; values live in fp32 slots of a caller-provided workspace of
 * n_slots * M * N floats. One pass per op.
 */
typedef enum th_vm_code {
  TH_VM_LOAD = 0,   /* slot <- operand a (column operands broadcast) */
  TH_VM_ADD = 1, TH_VM_SUB = 2, TH_VM_MUL = 3, TH_VM_DIV = 4, TH_VM_MAX = 5, TH_VM_POW = 6,
  TH_VM_EXP = 7, TH_VM_LOG = 8,
  TH_VM_ROW_SUM = 9, TH_VM_ROW_MAX = 10, /* result broadcast over the row */
  TH_VM_COPY = 11
} th_vm_code;

#define TH_VM_MAX_IN 16
#define TH_VM_MAX_OPS 96
#define TH_VM_MAX_OUT 8

typedef struct th_vm_operand {
  const void* ptr; int64_t ld; int32_t dtype;
  int32_t column;         /* 1: [M, 1] operand broadcast along the row */
} th_vm_operand;

typedef struct th_vm_op {
  int32_t code, dst, a, b; /* slots; for LOAD, a is an operand index */
  float scalar;
  int32_t mode;            /* 0: slot op slot, 1: slot op scalar, 2: scalar op slot */
} th_vm_op;

typedef struct th_vm_out {
  void* ptr; int64_t ld; int32_t dtype; int32_t slot;
} th_vm_out;

typedef struct th_vm_desc {
  int64_t M, N;
  int32_t n_in, n_ops, n_out, n_slots;
  th_vm_operand in[TH_VM_MAX_IN];
  th_vm_op ops[TH_VM_MAX_OPS];
  th_vm_out out[TH_VM_MAX_OUT];
  float* workspace;        /* n_slots * M * N fp32 */
} th_vm_desc;

int th_epilogue_vm(const th_vm_desc* desc, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TH_HIP_H */
