/*
 * exl3_mi355x.h -- C ABI of the MI355X (gfx950) EXL3 quantized-matmul library.
 *
 * This is the drop-in boundary for the turboexl3 plugins' quant path.  The
 * reference exposes it as mlx-serve's quant plugin table, `QuantTable`, an
 * extern struct of C-callconv function pointers
 * (turboexl3_qwen38/overlay/mlx_serve/abi/quant.zig:24-108), which
 * turboexl3_ds41 fills in turboexl3_ds41/plugin.zig:28-43.  The kit that
 * defines `Str`, `Verdict`, `Claim`, `Array`, `Stream`, `Weight`, `LoadCtx`,
 * `Source`, `PackDir` and `Swiglu` is an external dependency absent from the
 * reference tree, so those types are re-declared here from their use sites
 * (cited per type).  MLX handles become plain descriptors: a device pointer
 * with dtype and shape, and a hipStream_t.
 *
 * Paths in citations are relative to /root/reference/plugins/.
 *
 * Threading: every entry is thread-compatible.  Work is recorded on the stream
 * passed in; calls that share a weight must be ordered on one stream.
 * `claims`, `validate` and `bill` never touch the GPU
 * (turboexl3_qwen38/overlay/mlx_serve/abi/quant.zig:22-23).
 * Errors are named refusals, never a silent fallback: every entry that can
 * fail returns an `exl3_verdict` whose `why` is a static string.
 */
#ifndef EXL3_MI355X_H
#define EXL3_MI355X_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Version of this table; `exl3_quant_table.version` carries it
 * (quant.zig:16 `version: u32 = 1`). */
#define EXL3_ABI_VERSION 1u

/* kit `Str`: a byte slice, not NUL-terminated (used as `Str.of(..)` /
 * `.slice()` throughout turboexl3_ds41/config.zig:43-61). */
typedef struct exl3_str {
  const char *ptr;
  size_t len;
} exl3_str;

/* kit `Verdict{code, why}` with codes ok, unsupported, failed, too_large
 * (refusals: turboexl3_ds41/plugin.zig:50,93,187; quant.zig:98). */
enum {
  EXL3_OK = 0,
  EXL3_UNSUPPORTED = 1,
  EXL3_FAILED = 2,
  EXL3_TOO_LARGE = 3,
};
typedef struct exl3_verdict {
  int32_t code;
  const char *why; /* static string; "" when ok */
} exl3_verdict;

/* kit `Claim`: `.no` and `.by_marker` are the values the reference returns
 * (turboexl3_ds41/config.zig:43-47, turboexl3_qwen38/config.zig:18-28). */
enum {
  EXL3_CLAIM_NO = 0,
  EXL3_CLAIM_BY_MODE = 1,
  EXL3_CLAIM_BY_MARKER = 2,
};
typedef int32_t exl3_claim;

/* Element types, numbered as mlx-c's `mlx_dtype` (the ABI passes dtypes as
 * that enum: quant.zig:113 "mlx-c's `mlx_dtype`"). */
enum {
  EXL3_DT_BOOL = 0,
  EXL3_DT_U8 = 1,
  EXL3_DT_U16 = 2,
  EXL3_DT_U32 = 3,
  EXL3_DT_U64 = 4,
  EXL3_DT_I8 = 5,
  EXL3_DT_I16 = 6,
  EXL3_DT_I32 = 7,
  EXL3_DT_I64 = 8,
  EXL3_DT_F16 = 9,
  EXL3_DT_F32 = 10,
  EXL3_DT_F64 = 11,
  EXL3_DT_BF16 = 12,
};

/* kit `Array` (an MLX array handle) as a descriptor of a dense row-major
 * device buffer.  An array with data == NULL is "empty" (the reference's
 * `.{}` / `ctx == null`, e.g. `inds` of a dense SwiGLU,
 * turboexl3_ds41/plugin.zig:271).  `owned` is set on arrays this library
 * allocated; free them with exl3_array_free. */
#define EXL3_MAX_DIMS 4
typedef struct exl3_array {
  void *data;
  int32_t dtype;
  int32_t ndim;
  int64_t shape[EXL3_MAX_DIMS];
  uint32_t owned;
  uint32_t _pad;
} exl3_array;

/* kit `Stream`: here a hipStream_t (NULL = the device's null stream). */
typedef void *exl3_stream;

/* kit `Weight{w, scales, biases, side, flags}` (turboexl3_ds41/plugin.zig:89,
 * 183, 231-237): for EXL3, w = trellis u16 [in/16, out/16, n] (a bank:
 * [E, in/16, out/16, n]), scales = suh f16 [in] ([E, in]), biases = svh f16
 * [out] ([E, out]).  `priv` holds the weight's decode parameters (codebook,
 * window, rate) so no process-global decode state exists
 * (contrast sushi_ds41/src/sushi/exl3/root.zig:117-120). */
typedef struct exl3_weight {
  exl3_array w;
  exl3_array scales;
  exl3_array biases;
  exl3_array side;
  uint32_t flags;
  uint32_t _pad;
  void *priv;
} exl3_weight;

/* A host-side view of one stored tensor, as a weight source hands it out. */
typedef struct exl3_host_tensor {
  const void *data;
  int32_t dtype;
  int32_t ndim;
  int64_t shape[EXL3_MAX_DIMS];
} exl3_host_tensor;

/* kit `Source`: where a format reads a pack's tensors (quant.zig:17-18;
 * `ctx.source.tensor(name)` in turboexl3_ds41/plugin.zig:147,194).
 * `tensor` fills *out with a borrowed host view and returns 1, or returns 0
 * when the pack has no such tensor. */
typedef struct exl3_source {
  void *self;
  int (*tensor)(void *self, exl3_str name, exl3_host_tensor *out);
} exl3_source;

/* kit `PackDir` (`d.fileBytes(name)`, turboexl3_ds41/plugin.zig:62). */
typedef struct exl3_pack_dir {
  void *self;
  uint64_t (*file_bytes)(void *self, exl3_str name);
} exl3_pack_dir;

/* kit `LoadCtx` (fields used: host, block_json, dir, source, stream;
 * turboexl3_ds41/plugin.zig:52-80,86-91).  `device` selects the GPU;
 * `state` is written by `open` and read by the loads. */
typedef struct exl3_load_ctx {
  uint32_t size;
  int32_t device;
  exl3_str block_json;
  exl3_str config_json;
  const exl3_source *source;
  const exl3_pack_dir *dir;
  exl3_stream stream;
  void *state;
} exl3_load_ctx;

/* kit `Swiglu` options (`.limit`, `.verify_rows`:
 * turboexl3_qwen38/src/direct/moe.zig:65, turboexl3_ds41/plugin.zig:272-280).
 * limit > 0 clamps gate to min(g, limit) and up to [-limit, limit] (a NaN
 * passes through).  verify_rows: routed calls take the decode chain (the
 * grouped GEMV items) at any row count, as the reference sends verify rows
 * down its decode chain (sushi_ds41/src/sushi/exl3/root.zig:149). */
typedef struct exl3_swiglu_opts {
  uint32_t size;
  int32_t limit;
  bool verify_rows;
} exl3_swiglu_opts;

/* kit `Span(T)`: a pointer and a count (quant.zig:15), one type per element
 * type the table's entries take. */
typedef struct exl3_weight_span {
  const exl3_weight *ptr;
  size_t len;
} exl3_weight_span;
typedef struct exl3_array_span {
  const exl3_array *ptr;
  size_t len;
} exl3_array_span;
typedef struct exl3_u32_span {
  const uint32_t *ptr;
  size_t len;
} exl3_u32_span;
typedef struct exl3_u8_span {
  const uint8_t *ptr;
  size_t len;
} exl3_u8_span;

/* `LinearParts` (quant.zig:111-128): the options of the split entries
 * (linear_split / finish / prepared / pieces / piece); each entry reads the
 * fields its comment names.  `side` NULL: no side stream (the entry's own
 * stream does all the work). */
typedef struct exl3_linear_parts {
  uint32_t size;
  int32_t dtype;        /* EXL3_DT_* of the call's activations: the output's */
  exl3_stream side;     /* linear_split: the stream for the work after the prepare */
  bool inner;           /* linear_split: stop at the inner product */
  bool prepared;        /* linear_piece: x holds rows the caller prepared */
  exl3_array held;      /* linear_piece: what linear_pieces made */
  exl3_u32_span rows;   /* linear_pieces: each piece's row count, in row order */
  exl3_array_span parts; /* linear_finish: the inner products, in row order */
} exl3_linear_parts;

/* `SharedSwiglu` (quant.zig:183-197): the gated shared expert of
 * swiglu_shared.  y = routed + sigmoid(logit) * shared(x); `logit` [rows]
 * per row, or NULL with `gate_vec` [D] (the logit computed in the launch);
 * `logits` [rows, E] with `k`: the routing (softmax, top-k) done in the
 * launches, inds / scores then empty.  `sigtab` (MLX's sigmoid table) is
 * not read: the sigmoid is computed, then rounded to x's dtype. */
typedef struct exl3_shared_swiglu {
  uint32_t size;
  const exl3_weight *gate;
  const exl3_weight *up;
  const exl3_weight *down;
  exl3_array sigtab;
  exl3_array logit;
  exl3_array gate_vec;
  exl3_array logits;
  uint32_t k;
} exl3_shared_swiglu;

/* The attention entries' options (quant.zig:129-182).  This library leaves
 * those entries NULL (the host runs its own chain), so the types are
 * declared only for the table's signatures. */
typedef struct exl3_attn_in exl3_attn_in;
typedef struct exl3_attn_in_out exl3_attn_in_out;
typedef struct exl3_gate exl3_gate;
typedef struct exl3_q_planes exl3_q_planes;
typedef struct exl3_indexer exl3_indexer;

/* `Weight.flags` bit of a grouped linear (turboexl3_ds41/plugin.zig:105-106):
 * G linears `<base>.slice.<g>` stored as a G-bank; matmul takes
 * x [..., G, in] and gives y [..., G, out], group g through linear g. */
#define EXL3_WEIGHT_GROUPED 1u

/* ---------------------------------------------------------------- entries
 * One flat symbol per QuantTable entry, each also reachable through the table
 * below.  Each replaces the reference entry cited beside it.
 */

/* QuantTable.claims (quant.zig:29; turboexl3_ds41/config.zig:43-47):
 * exllamav3's block (`quant_method: "exl3"`) on a DeepSeek-V4.1 pack
 * (config `model_type` "deepseek_v41") by marker, anything else `no`; the
 * claim of exl3_quant_table_get(). */
exl3_claim exl3_claims(exl3_str block_json, exl3_str config_json);

/* turboexl3_qwen38's claim rule (turboexl3_qwen38/config.zig:18-32) as a
 * quant table's claim: a Qwen3.8 pack (config `model_type` "qwen4_exp" or
 * "qwen4_exp_text") whose config names a non-null `trunk_quant` block, by
 * marker; anything else `no` (exl3_validate refuses the blocks it does not
 * decode by name).  The claim of exl3_quant_table_qwen38_get(). */
exl3_claim exl3_claims_qwen38(exl3_str block_json, exl3_str config_json);

/* QuantTable.validate (quant.zig:31; turboexl3_ds41/config.zig:49-54, and
 * turboexl3's block rules as turboexl3_qwen38/config.zig:86-105 restates
 * them): refuses by name NotExl3, Exl3CodebookUnsupported (anything but mul1
 * or mcg, e.g. 3inst), Exl3WindowUnsupported (window outside 8..16),
 * Exl3RateUnsupported (k with 16k not an even integer in 16..128),
 * Exl3TopKExceedsReduceBank (num_experts_per_tok > 32). */
exl3_verdict exl3_validate(exl3_str block_json, exl3_str config_json,
                           const exl3_pack_dir *dir);

/* QuantTable.bill (quant.zig:33; turboexl3_ds41/config.zig:56-61): resident
 * bytes once loaded = the stored bytes (the HBM layout is the pack layout). */
uint64_t exl3_bill(exl3_str block_json, exl3_str model_dir, uint64_t stored);

/* QuantTable.open / close (quant.zig:34-35; turboexl3_ds41/plugin.zig:52-82):
 * parses the block (codebook, window) into ctx->state and initialises the
 * device, after the load-time self-check (exl3_self_check, for the block's
 * codebook on ctx->device, on ctx->stream) has passed: a failed check
 * refuses the open with its name; close frees ctx->state (loaded weights
 * outlive it). */
exl3_verdict exl3_open(exl3_load_ctx *ctx);
void exl3_close(exl3_load_ctx *ctx);

/* QuantTable.load_tensor (quant.zig:37; turboexl3_ds41/plugin.zig:86-103):
 * `<name>.trellis` (i16/u16 [in/16, out/16, n]), `<name>.suh` (f16 [in]),
 * `<name>.svh` (f16 [out]) from ctx->source, copied to device memory on
 * ctx->stream.  in_dim != 0 must equal in.  A pack that stores the name as
 * `<name>.slice.<g>` linears (g = 0, 1, ..: DeepSeek-V4.1's grouped `wo_a`,
 * turboexl3_ds41/plugin.zig:108-125) loads as a grouped linear: a G-bank
 * with flags EXL3_WEIGHT_GROUPED.  Refusals: MissingWeight, NotShaped (the
 * reference's `not_shaped` text). */
exl3_verdict exl3_load_tensor(const exl3_load_ctx *ctx, exl3_str name, uint32_t in_dim,
                              exl3_weight *out);

/* QuantTable.load_bank (quant.zig:39; turboexl3_ds41/plugin.zig:127-185):
 * the routed experts `<prefix>.<e><suffix>` for e = 0.. (name =
 * `<prefix>.<proj>`, split at its last '.') stacked on a new first axis. */
exl3_verdict exl3_load_bank(const exl3_load_ctx *ctx, exl3_str name, uint32_t in_dim,
                            exl3_weight *out);

/* QuantTable.release (quant.zig:40; turboexl3_ds41/plugin.zig:231-237):
 * frees every array the weight owns and zeroes it. */
void exl3_release(exl3_weight *w);

/* QuantTable.matmul (quant.zig:41-42; turboexl3_ds41/plugin.zig:243-248 ->
 * turboexl3 `linear`): out = x @ W^T, x [..., in] in f16/bf16/f32, out
 * [..., out] in x's dtype.  Rounding points (quant.zig:52-55):
 * xp = f16(H(f16(x)*suh)/sqrt(128)); z = f16(sum_k xp*W) (f32 accumulate);
 * y = f16(H(z)/sqrt(128)*svh) then x's dtype.  If out->data is NULL the
 * library allocates the result (owned = 1); otherwise it writes into the
 * caller's buffer, which must have x's dtype and the result's shape.  A
 * grouped linear (G linears, flags EXL3_WEIGHT_GROUPED) takes x [..., G, in]
 * and gives [..., G, out], x[..., g, :] through linear g
 * (turboexl3_ds41/plugin.zig:243-261, sushi_ds41/src/sushi/exl3/linear.zig:24-36). */
exl3_verdict exl3_matmul(const exl3_weight *w, exl3_array x, exl3_stream s, exl3_array *out);

/* exl3_matmul without any allocation: no counterpart in the reference; for
 * callers that cannot call hipMalloc (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation).  Same kernels and the
 * same results as exl3_matmul, bit for bit, with one exception: a weight
 * that holds a matrix through exl3_resident (a rate without the prefill
 * GEMM) or exl3_unrotate takes a dense GEMM in exl3_matmul above 16 rows,
 * while this entry always runs the trellis kernels (within the matmul bar
 * of each other, not bit for bit).  A
 * split-K wait that gives up here sets the array's status word, which
 * exl3_stream_status reports.  `out` must be the caller's
 * buffer (x's dtype, the result's shape).  Scratch comes from one array per
 * GPU, 64 MiB, held by the library from its load onto that GPU until the
 * process ends: 8 MiB of split-K slots (GEMV, up to 16 rows) and 56 MiB of
 * staging (the GEMM's prepared rows, rows * in * 2 bytes, and its split-K
 * planes); a call needing more is refused with EXL3_TOO_LARGE before any
 * launch (exl3_matmul serves it).  The first call on a GPU sets the array up
 * (its address, the slots' empty mark) and must run outside graph capture;
 * later calls may be captured.  Calls share their GPU's array: calls that
 * overlap in time on one GPU (on different streams) race on it, so the
 * caller orders them. */
exl3_verdict exl3_matmul_noalloc(const exl3_weight *w, exl3_array x, exl3_stream s,
                                 exl3_array out);

/* Up to four linears that read the same rows, in one launch: outs[i] =
 * x @ W_i^T, each in x's dtype (turboexl3's linearShared,
 * sushi_ds41/src/sushi/exl3/linear.zig:34-60: q/k/v, gate/up).  The weights
 * must share the input width, rate, codebook and window (else refused:
 * the caller runs exl3_matmul per weight).  Output ownership per outs[i] as
 * exl3_matmul.  Not a QuantTable entry. */
exl3_verdict exl3_matmul_shared(const exl3_weight *const *ws, uint32_t count, exl3_array x,
                                exl3_stream s, exl3_array *outs);

/* QuantTable.moe (quant.zig:43-45): turboexl3_ds41 refuses it ("routed
 * experts run through swiglu", turboexl3_ds41/plugin.zig:263-265); so does
 * this library, with the same reason. */
exl3_verdict exl3_moe(const exl3_weight *bank, exl3_array x, exl3_array lhs, exl3_array rhs,
                      bool sorted, exl3_stream s, exl3_array *out);

/* QuantTable.swiglu (quant.zig:48-50; turboexl3_ds41/plugin.zig:267-283 ->
 * turboexl3 `moe` / `moeClamped`): x [B, S, D] through the banks' experts
 * inds [B, S, K] (i32/u32) weighted by scores [B, S, K] (f32/f16/bf16):
 * y = sum_k score_k * down_e(silu(gate_e(x)) * up_e(x)), in x's dtype.
 * Empty inds: the dense SwiGLU MLP of the (single-bank) weights.  Output
 * ownership as exl3_matmul. */
exl3_verdict exl3_swiglu(const exl3_weight *gate, const exl3_weight *up, const exl3_weight *down,
                         exl3_array x, exl3_array inds, exl3_array scores,
                         const exl3_swiglu_opts *opts, exl3_stream s, exl3_array *out);

/* QuantTable.linear_split (quant.zig:56-58): matmul with the work after x's
 * prepare recorded on opts->side (NULL side: all on s); with opts->inner it
 * stops before the finish and *out is the inner product z f16 [rows, out]
 * that linear_finish takes, else y [rows, out] in x's dtype.  With a side
 * stream, x's prepared rows live in *out's allocation behind the result, so
 * free *out only after the side stream's work. */
exl3_verdict exl3_linear_split(const exl3_weight *w, exl3_array x, const exl3_linear_parts *opts,
                               exl3_stream s, exl3_array *out);

/* QuantTable.linear_finish (quant.zig:59-60): the finish of opts->parts (one
 * inner product z f16, or a call's row pieces in row order): y [rows, out]
 * in opts->dtype. */
exl3_verdict exl3_linear_finish(const exl3_weight *w, const exl3_linear_parts *opts,
                                exl3_stream s, exl3_array *out);

/* QuantTable.linear_prepared (quant.zig:61-62): matmul of rows the caller
 * prepared (xp f16 [rows, in], xp = f16(H(f16(x) * suh) / sqrt(128)) per
 * 128-block): y [rows, out] in opts->dtype. */
exl3_verdict exl3_linear_prepared(const exl3_weight *w, exl3_array xp,
                                  const exl3_linear_parts *opts, exl3_stream s, exl3_array *out);

/* QuantTable.linear_pieces (quant.zig:63-65): the weight in the form a call's
 * row pieces share.  The kernels decode the packed trellis on the fly at
 * every width, so that form is the trellis itself: *out is a borrowed view
 * of it (owned = 0), made without a launch.  Refused when the pieces
 * (opts->rows) would not all take the kernel path (GEMV or GEMM) of the
 * whole call, whose sums are then ordered differently. */
exl3_verdict exl3_linear_pieces(const exl3_weight *w, const exl3_linear_parts *opts,
                                exl3_stream s, exl3_array *out);

/* QuantTable.linear_piece (quant.zig:66-68): one piece's inner product
 * z f16 [rows, out] against opts->held (what linear_pieces made for this
 * weight): of x [..., in], or with opts->prepared of rows the caller
 * prepared (f16). */
exl3_verdict exl3_linear_piece(const exl3_weight *w, exl3_array x, const exl3_linear_parts *opts,
                               exl3_stream s, exl3_array *out);

/* QuantTable.swiglu_shared (quant.zig:94-97; SharedSwiglu :183-197; the
 * host's chain it replaces: turboexl3_qwen38/src/direct/moe.zig:113-160):
 * y = swiglu(x; gate, up, down, routes) + sigmoid(logit) * shared(x), with
 * shared(x) = down_s(silu(gate_s(x)) * up_s(x)) the dense SwiGLU of
 * opts->gate / up / down (unclamped), the shared expert riding the routed
 * GEMV launches as one more expert slot per row.  Routes: inds / scores as
 * in exl3_swiglu, or empty with opts->logits [rows, E] and opts->k: the
 * softmax's top k renormalized, computed in the first launch.  The logit:
 * opts->logit [rows], or opts->gate_vec [D] (the dot with x's row, in the
 * launch), both in x's dtype; sigmoid(logit) is rounded to x's dtype.
 * Refused (the host runs its chain) at prefill-sized batches and when the
 * shared expert's widths, rate or codebook differ from the banks'. */
exl3_verdict exl3_swiglu_shared(const exl3_weight *gate, const exl3_weight *up,
                                const exl3_weight *down, exl3_array x, exl3_array inds,
                                exl3_array scores, const exl3_shared_swiglu *opts,
                                exl3_stream s, exl3_array *out);

/* QuantTable.resident (quant.zig:96-99): memory for speed, spent only where
 * it buys speed.  Admits ws' single linears.  At a rate without the prefill
 * GEMM (any n but the integer rates and n = 24, 40: those run 16-row GEMV
 * passes above 16 rows), the decoded matrix (W_inner f16 [in, out], in *
 * out * 2 bytes) is held from its first matmul at prefill widths (over 16
 * rows) on, and that matmul becomes the prepare, a dense f16 GEMM
 * (hipBLASLt) over the held matrix and the finish.  At the GEMM's rates the
 * fused decode GEMM outruns that path, so the matmul keeps the GEMM and
 * nothing is held: the admission reserves the bytes (resident_pending) for
 * exl3_unrotate, whose public matrices do outrun it.  Decode widths keep the
 * EXL3 GEMV.  *bytes = what ws' matrices take.  Refused EXL3_TOO_LARGE past
 * room (0: no bound), admitting none; an empty ws drops every kept matrix. */
exl3_verdict exl3_resident(exl3_weight_span ws, uint64_t room, exl3_stream s, uint64_t *bytes);

/* QuantTable.resident_pending (quant.zig:100-101): the bytes admitted and
 * not held yet. */
uint64_t exl3_resident_pending(void);

/* QuantTable.unrotate (quant.zig:102-104): ws in groups of sizes[g] weights
 * that read one input; each group's matrices out of the format's basis,
 * W_public = diag(suh) H W_inner H diag(svh) / 128 (the reference's
 * reconstructPublic, sushi_ds41/src/sushi/exl3/expert_exl3.zig:440-488, in
 * its operation order; f16 bit for bit), joined side by side in `act`
 * (EXL3_DT_F16/BF16/F32) as one [in, sum of outs] matrix; each member's
 * W_inner is freed and its prefill matmuls in `act` become one dense GEMM
 * over its columns.  took[g]: whether group g took (members admitted by
 * exl3_resident, one input width and device, in no other group). */
exl3_verdict exl3_unrotate(exl3_weight_span ws, exl3_u8_span sizes, int32_t act, exl3_stream s,
                           bool *took);

/* QuantTable.linear_joined (quant.zig:105-107): x [..., in] times the joined
 * matrix of the un-rotated group whose members are ws, in order: [..., sum
 * of outs] in x's dtype (the group's act).  Refused when ws is not such a
 * group and at decode widths (up to 16 rows). */
exl3_verdict exl3_linear_joined(exl3_weight_span ws, exl3_array x, exl3_stream s,
                                exl3_array *out);

/* ----------------------------------------------------- the plugin table */

/* kit `QuantTable`, the whole layout (quant.zig:24-107): the entries
 * turboexl3_ds41 fills (turboexl3_ds41/plugin.zig:28-43), the split
 * entries, swiglu_shared, the resident entries, and NULL for the
 * attention entries, where the host runs its own chain. */
typedef struct exl3_quant_table {
  uint32_t size;
  uint32_t version;
  exl3_str name;
  exl3_claim (*claims)(exl3_str block_json, exl3_str config_json);
  exl3_verdict (*validate)(exl3_str block_json, exl3_str config_json, const exl3_pack_dir *dir);
  uint64_t (*bill)(exl3_str block_json, exl3_str model_dir, uint64_t stored);
  exl3_verdict (*open)(exl3_load_ctx *ctx);
  void (*close)(exl3_load_ctx *ctx);
  exl3_verdict (*load_tensor)(const exl3_load_ctx *ctx, exl3_str name, uint32_t in_dim,
                              exl3_weight *out);
  exl3_verdict (*load_bank)(const exl3_load_ctx *ctx, exl3_str name, uint32_t in_dim,
                            exl3_weight *out);
  void (*release)(exl3_weight *w);
  exl3_verdict (*matmul)(const exl3_weight *w, exl3_array x, exl3_stream s, exl3_array *out);
  exl3_verdict (*moe)(const exl3_weight *bank, exl3_array x, exl3_array lhs, exl3_array rhs,
                      bool sorted, exl3_stream s, exl3_array *out);
  exl3_verdict (*register_kernels)(const void *host);
  exl3_verdict (*swiglu)(const exl3_weight *gate, const exl3_weight *up, const exl3_weight *down,
                         exl3_array x, exl3_array inds, exl3_array scores,
                         const exl3_swiglu_opts *opts, exl3_stream s, exl3_array *out);
  exl3_verdict (*linear_split)(const exl3_weight *w, exl3_array x, const exl3_linear_parts *opts,
                               exl3_stream s, exl3_array *out);
  exl3_verdict (*linear_finish)(const exl3_weight *w, const exl3_linear_parts *opts,
                                exl3_stream s, exl3_array *out);
  exl3_verdict (*linear_prepared)(const exl3_weight *w, exl3_array xp,
                                  const exl3_linear_parts *opts, exl3_stream s, exl3_array *out);
  exl3_verdict (*linear_pieces)(const exl3_weight *w, const exl3_linear_parts *opts,
                                exl3_stream s, exl3_array *out);
  exl3_verdict (*linear_piece)(const exl3_weight *w, exl3_array x, const exl3_linear_parts *opts,
                               exl3_stream s, exl3_array *out);
  exl3_verdict (*attn_in)(const exl3_weight *q, const exl3_weight *k, const exl3_weight *v,
                          exl3_array x, const exl3_attn_in *opts, exl3_stream s,
                          exl3_attn_in_out *out);
  exl3_verdict (*attn_prep)(const exl3_weight *q, const exl3_weight *k, const exl3_weight *v,
                            const exl3_weight *w4, exl3_array x, exl3_stream s, exl3_array *out);
  exl3_verdict (*linear_prepared_idx)(const exl3_weight *w, exl3_array xp, exl3_array x,
                                      exl3_stream s, exl3_array *out);
  exl3_verdict (*gated_out)(const exl3_weight *o, exl3_array attn, const exl3_gate *gate,
                            exl3_stream s, exl3_array *out);
  exl3_verdict (*merged_gated_out)(const exl3_weight *o, exl3_array pacc, exl3_array pml,
                                   const exl3_gate *gate, exl3_stream s, exl3_array *out);
  exl3_verdict (*q_planes)(const exl3_weight *q, exl3_array x, const exl3_q_planes *opts,
                           exl3_stream s, exl3_array *out);
  exl3_verdict (*indexer)(const exl3_weight *idx, exl3_array x, const exl3_indexer *opts,
                          exl3_stream s, exl3_array *out);
  exl3_verdict (*swiglu_shared)(const exl3_weight *gate, const exl3_weight *up,
                                const exl3_weight *down, exl3_array x, exl3_array inds,
                                exl3_array scores, const exl3_shared_swiglu *opts, exl3_stream s,
                                exl3_array *out);
  exl3_verdict (*resident)(exl3_weight_span ws, uint64_t room, exl3_stream s, uint64_t *bytes);
  uint64_t (*resident_pending)(void);
  exl3_verdict (*unrotate)(exl3_weight_span ws, exl3_u8_span sizes, int32_t act, exl3_stream s,
                           bool *took);
  exl3_verdict (*linear_joined)(exl3_weight_span ws, exl3_array x, exl3_stream s,
                                exl3_array *out);
} exl3_quant_table;

/* The exported table (the reference exports it as `exportName(name,
 * version)`, quant.zig:22; plugin name turboexl3_ds41/plugin.zig:22):
 * "turboexl3_mi355x", claiming as turboexl3_ds41 does (exl3_claims). */
const exl3_quant_table *exl3_quant_table_get(void);

/* The same entries under the name "turboexl3_mi355x_qwen38", claiming as
 * turboexl3_qwen38 does (exl3_claims_qwen38): the table a host serving
 * Qwen3.8 packs loads. */
const exl3_quant_table *exl3_quant_table_qwen38_get(void);

/* ------------------------------------------------------- support entries */

/* Frees an array this library allocated (owned != 0); no-op otherwise.  The
 * entries that hand back a new array (out->data NULL, the reference's
 * convention, quant.zig:41-50) take it from a pool per (device, stream), and
 * this returns its memory to the pool of the stream it was made for, so a
 * steady serving loop of new arrays and frees calls no hipMalloc or hipFree
 * after its first step.  The next call on that stream may reuse the memory
 * at once (work on a stream is ordered); a caller that read the array on
 * another stream synchronizes that stream before freeing it.  A pool keeps
 * at most 1 GiB (the oldest blocks beyond it go back to the driver);
 * exl3_scratch_release empties it. */
void exl3_array_free(exl3_array *a);

/* A weight over device arrays the caller already holds (borrowed, not freed
 * by release): the reference's `share` of source arrays
 * (turboexl3_ds41/plugin.zig:213-218) for callers whose weights are already
 * resident.  block_json supplies codebook and window (NULL/empty: mul1, 16).
 * Besides turboexl3's mul1 and mcg it takes the pack format's table
 * codebooks (sushi_ds41/src/sushi/exl3/expert_exl3.zig:54-60,288-357):
 * spec1 and std1 (hash-mask) and pair1 (a weight pair from one codeword),
 * whose block names a shipped table and its digest (`codebook_table`:
 * pair1-w16-v1, spec1-w15, spec1-w16 or std1; `codebook_digest`), resolved
 * as codebook_tables.zig:266-279 does, refusing by name
 * Exl3CodebookTableUnknown, ...DigestMismatch, ...LegacyConfig,
 * ...CodebookMismatch, ...WindowMismatch, and Exl3CodebookTableRateMissing
 * for a rate the table has no row for.  validate and open keep turboexl3's
 * rule (mul1 or mcg). */
exl3_verdict exl3_weight_wrap(exl3_array trellis, exl3_array suh, exl3_array svh,
                              exl3_str block_json, int32_t device, exl3_weight *out);

/* The decoded tile matrix W_inner f16 [in, out] of a single-bank weight (a
 * bank: expert `expert`), bit-exact to the reference decode
 * (sushi_ds41/src/sushi/exl3/expert_exl3.zig:416-438; the Metal
 * `q3_exl3_dig_decmat_*` kernels, turboexl3_ds41/src/exl3/kernels/exl3/
 * q3_exl3_dig_decmat_5120x2304_mul1hk3.metal:1-52).  out: f16 [in, out]. */
exl3_verdict exl3_decode_matrix(const exl3_weight *w, int32_t expert, exl3_array out,
                                exl3_stream s);

/* The prepare and finish halves of matmul as their own launches
 * (quant.zig:52-55, turboexl3's `linear_prepared` / `linear_finish` split):
 * prepare: x [rows, in] -> xp f16 [rows, in]; finish: z f16 [rows, out] ->
 * y [rows, out] in y's dtype. */
exl3_verdict exl3_prepare(const exl3_weight *w, exl3_array x, exl3_array xp, exl3_stream s);
exl3_verdict exl3_finish(const exl3_weight *w, exl3_array z, exl3_array y, exl3_stream s);

/* The inner product alone: xp f16 [rows, in] -> z f16 [rows, out]
 * (sushi_ds41/src/sushi/exl3/expert_exl3.zig:503-532). */
exl3_verdict exl3_inner(const exl3_weight *w, exl3_array xp, exl3_array z, exl3_stream s);

/* A Source over a pack's safetensors files: the pack loader for hosts without
 * a Source of their own.  The reference's host (mlx-serve) hands the format an
 * MLX Source over the same files (turboexl3_ds41/plugin.zig:86-103,127-185:
 * <base>.trellis i16 [in/16, out/16, n], <base>.suh f16 [in], <base>.svh f16
 * [out]); this one maps each file read-only and hands out host views into the
 * mappings, valid until exl3_safetensors_close.  Returns NULL, with *why set
 * (a missing file, a header past its file, offsets that disagree with a
 * tensor's shape and dtype, an unknown dtype, a name in two files), or the
 * source to put in exl3_load_ctx.source. */
exl3_source *exl3_safetensors_open(const char *const *paths, uint32_t count, exl3_verdict *why);
void exl3_safetensors_close(exl3_source *src);

/* A PackDir over a directory (the kit's `dir.fileBytes(name)`,
 * turboexl3_ds41/plugin.zig:62): file_bytes(name) = the size of root/name,
 * 0 when absent or when name leaves the directory.  NULL if root is not a
 * directory. */
exl3_pack_dir *exl3_pack_dir_open(const char *root);
void exl3_pack_dir_close(exl3_pack_dir *dir);

/* Frees the library's scratch for (device, stream): prepared rows, split-K
 * slots and counters, MoE staging, and every smaller buffer a growing call
 * replaced.  The library keeps scratch per (device, stream) and, when a call
 * needs more, makes a larger buffer and keeps the old one (a HIP graph
 * captured earlier on the stream may still read it), so growth never
 * invalidates a captured graph; call this once no graph captured on the
 * stream will be replayed again (e.g. before destroying the stream).  The
 * next call on the stream makes its scratch anew.  It also returns to the
 * driver the memory of output arrays freed with exl3_array_free that the
 * stream's pool keeps (see exl3_array_free).  Refused while the stream is
 * being captured.  No counterpart in the reference (MLX owns its
 * temporaries there). */
exl3_verdict exl3_scratch_release(int32_t device, exl3_stream s);

/* Status of the split-K hand-offs of (device, stream)'s calls since the last
 * check.  A GEMV or routed-MoE launch that splits k has the workgroup of the
 * last split wait for the other splits' partial sums; the wait is bounded,
 * and one that gives up (a partial sum that never arrived) leaves NaN in its
 * outputs and sets a status word instead of blocking.  This synchronizes the
 * stream, returns FAILED (with the reason) if any wait gave up, and then
 * resets the slots so later calls are sound; ok otherwise.  It also reads
 * the device's exl3_matmul_noalloc array (shared by every stream on the
 * device: the caller synchronizes the streams that use it first) and resets
 * it the same way.  No counterpart in the reference (MLX's kernels do not
 * hand off across workgroups). */
exl3_verdict exl3_stream_status(int32_t device, exl3_stream s);

/* Diagnostic: the split-K wait's bound in polls for launches issued from now
 * on (a negative value restores the default, about 2^20 polls).  Lowering it
 * to 0 makes waits give up whenever a partial sum has not landed yet, which
 * tests of exl3_stream_status use; every kernel still exits normally. */
void exl3_set_splitk_poll_bound(int32_t polls);

/* Diagnostic for failure-handling tests: while set (nonzero), launches have
 * the splits other than the last skip their partial-sum stores, so the last
 * split's bounded wait gives up (at the bound above) and the status word is
 * set; every kernel still exits normally.  Off by default. */
void exl3_set_splitk_test_drop(int32_t on);

/* The load-time self-check that exl3_open runs before it accepts a pack
 * (turboexl3_ds41/src/exl3/quant.zig:469-503 `accept` -> selfcheck.zig:
 * 861-930).  Host part: SHA-256 against its standard's example, and the
 * manifest's golden planes (turboexl3_ds41/src/exl3/kernels/exl3/
 * manifest.json: splitmix64-seeded mul1 code at K = 2 and 3, 5120 x 2304)
 * against their code digests.  Device part, on `device`: every state of the
 * mul1 codebook through the kernels' decode against the manifest's table
 * digest (exl3_open checks the block's codebook: mul1 or mcg); each plane's
 * W_hat from exl3_decode_matrix against its digest; one-hot rows through
 * exl3_inner -- the prefill GEMM, all rows in one call, and the decode GEMV,
 * 16 rows a call -- equal to W_hat bit for bit.  A failure is refused
 * (EXL3_FAILED) with "Exl3SelfCheckFailed" and the check's name; a device
 * part that passed is not run again in the process.  device < 0: the host
 * part only (needs no GPU).  Not a QuantTable entry. */
exl3_verdict exl3_self_check(int32_t device);

/* Diagnostic for tests of the refusal path: the named check of the
 * self-check ("sha256", "code", "states", "decode", "gemm", "gemv") is made
 * to fail (its expected digest replaced, or one element of its output
 * flipped), and the self-check runs in full on every call while a fault is
 * set; NULL or "" clears it. */
void exl3_set_self_check_fault(const char *check);

/* Library version string and the kernel variant a matmul of `rows` rows
 * takes ("gemv", "gemm"; a grouped linear, `rows` rows per group:
 * "gemm-groups", one prepare and one grouped GEMM launch for every group,
 * or "per-group"): diagnostics for tests and benchmarks. */
const char *exl3_version(void);
const char *exl3_matmul_path(const exl3_weight *w, int64_t rows);

/* The kernel path a swiglu of `rows` rows takes (topk 0: no routes;
 * verify_rows as exl3_swiglu_opts): "dense-gemv", "dense-gemm",
 * "dense-items", "routed-gemv" (grouped GEMV items of up to 4 slots of one
 * expert) or "routed-gemm" (grouped GEMM over items of up to 256 slots, for
 * prefill-sized expert batches): a diagnostic for tests and benchmarks. */
const char *exl3_swiglu_path(const exl3_weight *gate, const exl3_weight *up,
                             const exl3_weight *down, int64_t rows, int32_t topk,
                             bool verify_rows);

#ifdef __cplusplus
}
#endif
#endif
