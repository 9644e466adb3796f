// exl3_kernels.h -- host-callable launchers of the EXL3 HIP kernels (internal
// to libexl3_mi355x.so; the public boundary is include/exl3_mi355x.h).
//
// Every launcher checks on the host the shape facts its kernel's indexing and
// grid assume and returns a nonzero hipError_t-style code (or -1 for a shape
// refusal) instead of launching when they do not hold.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace exl3 {

// A weight's decode constants as the kernels take them: the window mask
// and, for the table codebooks, its rate's row
// (sushi_ds41/src/sushi/exl3/codebook_tables.zig): hash-mask {mult, mask0};
// pair1 {mult, mask0, mask1} and rsh = 32 - rot, the v_alignbit_b32 shift
// that rotates left by rot.
struct CbRow {
  uint32_t mask = 0xFFFFu;
  uint32_t mult = 0, mask0 = 0, mask1 = 0, rsh = 0;
};

// Decode parameters of one EXL3 weight: n halfwords per 16x16 tile (even,
// 16..128), kernel codebook form (0 mul1, 1 mcg, 2 hash-mask: spec1 and
// std1, 3 pair1; the Codebook enum of exl3_device.h), window bits (8..16)
// and the table codebooks' row for n (row: {mult, mask0, mask1, rot}).
// The kernel codebook forms Format.codebook holds (the Codebook enum of the
// device code, restated for host code that does not include it).
constexpr int CB_FORM_MUL1 = 0, CB_FORM_MCG = 1, CB_FORM_HASH = 2, CB_FORM_PAIR1 = 3;

struct Format {
  int n = 0;
  int codebook = 0;
  int window = 16;
  uint32_t row[4] = {0, 0, 0, 0};
  uint32_t mask() const { return (window >= 16) ? 0xFFFFu : ((1u << window) - 1u); }
  bool integer_rate() const { return n % 16 == 0 && n >= 16 && n <= 128; }
  // the prefill GEMM's rates: the integer ones and the half-integer n = 24, 40
  // (exllamav3's K 1.5 and 2.5; turboexl3_ds41/src/bank/frac.zig:42-44)
  bool gemm_rate() const { return integer_rate() || n == 24 || n == 40; }
  CbRow dec() const {
    CbRow d;
    d.mask = mask();
    d.mult = row[0];
    d.mask0 = row[1];
    d.mask1 = row[2];
    d.rsh = (32u - (row[3] & 31u)) & 31u;
    return d;
  }
  bool same_decode(const Format &o) const {
    return codebook == o.codebook && window == o.window && row[0] == o.row[0] &&
           row[1] == o.row[1] && row[2] == o.row[2] && row[3] == o.row[3];
  }
};

// Device scratch a GEMV or routed-MoE call uses for its split-K hand-off:
// partial-sum slots, each holding the empty mark (all-ones bytes) between
// calls -- every call leaves the slots it used empty again, so one slot
// buffer serves any sequence of calls on one stream whatever their shapes --
// and a status word (zero) that a split-K wait which gives up sets.
struct Scratch {
  float *partial = nullptr;
  size_t partial_floats = 0;
  uint32_t *status = nullptr;
};
// A slot buffer is a 256-byte header holding the status word, then the slots.
constexpr size_t SLOT_HEADER_BYTES = 256;

// exl3_matmul_noalloc's scratch (exl3_noalloc.hip): 64 MiB per device, of
// which a slot buffer of 8 MiB (2M partial-sum floats) and 56 MiB of staging
// for the GEMM's prepared rows and split-K planes.
constexpr size_t NOALLOC_BYTES = (size_t)64 << 20;
constexpr size_t NOALLOC_SLOT_BYTES = (size_t)8 << 20;
// The array's address on `device` (current), set up on the first call per
// device (refused with hipErrorStreamCaptureUnsupported while s is capturing).
hipError_t noalloc_scratch(int device, hipStream_t s, void **base);
// The array's status word on `device` (the caller has synchronized the
// calls' stream): *gave_up set when a split-K wait gave up, after which the
// slots hold the empty mark again and the word is zero.  Nothing to read on a
// device where no call has set the array up.
hipError_t noalloc_status(int device, bool *gave_up);
// The split-K wait's bound in polls (PARTIAL_POLL_MAX unless lowered by
// set_splitk_poll_max; a negative value restores it).
int splitk_poll_max();
void set_splitk_poll_max(int polls);
// Failure-handling tests: launches issued while set have the splits other
// than the last skip their partial-sum stores (the last split's wait then
// gives up at its bound; every kernel exits normally).
int splitk_drop();
void set_splitk_drop(int on);

// Output / activation element types understood by the kernels.
enum ActType { ACT_F16 = 0, ACT_BF16 = 1, ACT_F32 = 2 };

// prepare: x [rows, in] (ACT_*) -> xp f16 [rows, in]; suh f16 [in], or with
// groups > 1 suh [groups, in] and row r taking suh row r % groups (a grouped
// linear's x [rows / groups, groups, in] read in place).
hipError_t launch_prepare(const void *x, int xdt, const uint16_t *suh, uint16_t *xp, int rows,
                          int in, hipStream_t s, int groups = 1);
// The prefill GEMM over a grouped linear (G linears stored as a G-bank,
// trellis [G][in/16][out/16][n], svh [G][out]): xp f16 [rows, G, in]
// (prepared, slot r G + g = row r of group g) -> y [rows, G, out] in ydt,
// one launch over every group's 256-row tiles (integer rates).
hipError_t launch_gemm_groups(const uint16_t *trellis, const Format &f, const uint16_t *xp,
                              const uint16_t *svh, void *y, int ydt, int rows, int groups,
                              int in, int out, hipStream_t s);
// finish: z f16 [rows, out] -> y [rows, out] (ACT_*); svh f16 [out].
hipError_t launch_finish(const uint16_t *z, const uint16_t *svh, void *y, int ydt, int rows,
                         int out, hipStream_t s);
// decode: trellis [in/16][out/16][n] -> W_inner f16 [in, out].
// Every state of f's codebook into w (65536 f16; pair1: 131072, a weight
// pair per codeword), through the kernels' device decode.
hipError_t launch_decode_states(const Format &f, uint16_t *w, hipStream_t s);
hipError_t launch_decode_matrix(const uint16_t *trellis, const Format &f, int in, int out,
                                uint16_t *w, hipStream_t s);

// un-rotation: W_inner f16 [in, out] -> W_public [in, out] in ydt (ACT_*),
// rows ld elements apart, in the reference's reconstructPublic order.
hipError_t launch_unrotate(const uint16_t *w_inner, const uint16_t *suh, const uint16_t *svh,
                           int in, int out, void *dst, int64_t ld, int ydt, hipStream_t s);

// The GEMV split: whole 128-input blocks per split (ksplit splits of tps
// k-tile rows) for a GEMV over `groups` weights of (in, out).
// tps_max: the most k-tiles a split takes (dense GEMV 64, MoE items 128).
void gemv_plan(int in, int out, int groups, int rows, int *ksplit, int *tps, int tps_max);
int gemv_ksplit(int in, int out, int groups, int rows);
// Largest row count the GEMV path serves (the MFMA M); wider calls take the GEMM.
constexpr int GEMV_ROWS_MAX = 16;

// GEMV (rows <= GEMV_ROWS_MAX), one launch: prepare (or, with prepared, xp
// f16 rows as given), decode GEMV, split-K sum, z rounded to f16, finish into
// y; or, with y == nullptr, z f16 [rows, out] written to zout.
hipError_t launch_gemv(const uint16_t *trellis, const Format &f, const void *x, int xdt,
                       bool prepared, const uint16_t *suh, const uint16_t *svh, void *y, int ydt,
                       uint16_t *zout, int rows, int in, int out, Scratch &sc, hipStream_t s);
// Up to four linears that read the same rows (same in, rate, codebook and
// window), one launch; sc[i] is linear i's scratch.
struct GemvLinear {
  const uint16_t *trellis;
  const uint16_t *suh;
  const uint16_t *svh;
  void *y;
  uint16_t *zout;
  int out;
};
hipError_t launch_gemv_multi(const GemvLinear *ls, int count, const Format &f, const void *x,
                             int xdt, bool prepared, int ydt, int rows, int in, Scratch *sc,
                             hipStream_t s);
// The decode step's fusions around a GEMV launch (all off when zero):
//  * up: SwiGLU prologue, x = f16(silu(x) * up) (x and up f16);
//  * nssq: RMSNorm prologue, x is the f32 residual h [rows][in], nssq its
//    sums of squares per 128 columns [rows][in / 128] (<= 64 of them), x =
//    f16(h * rsqrt(sum / in + eps) * norm_w); rows in one prepare batch;
//  * res (one linear): res [rows][out] += f32(y) instead of storing y, and
//    res_ssq [rows][out / 128] = the new res's sums of squares per group.
struct GemvFuse {
  const uint16_t *up = nullptr;
  float limit = 0.0f;
  const float *nssq = nullptr;
  const uint16_t *norm_w = nullptr;
  float eps = 0.0f;
  float *res = nullptr;
  float *res_ssq = nullptr;
  // the attention prologue: x is the decode attention's split slots
  // [rows][attn_nkv][attn_nsplit][attn_g][128 + 2], combined in the prepare
  const float *attn_part = nullptr;
  int attn_nkv = 0, attn_g = 0, attn_nsplit = 0;
  // x holds prepared rows, one [rows][in] set per weight, stacked in the
  // weights' order (a producer formed each weight's prepare)
  bool stacked = false;
};
hipError_t launch_gemv_fused(const GemvLinear *ls, int count, const Format &f, const void *x,
                             int xdt, int ydt, int rows, int in, Scratch *sc, const GemvFuse &fz,
                             hipStream_t s);
// Largest in / 128 the RMSNorm prologue takes (one partial sum per lane).
constexpr int NORM_MAXBLK = 64;
// Whether a GEMV launch's rows fit one prepare batch (what the RMSNorm
// prologue needs).
bool gemv_one_batch(int in, int total_out, bool generic, int rows);
// xp = the prepare (with suh, the consumer linear's) of h = f16(silu(g) *
// u) over [rows][in], in one launch: the prepared rows a GEMV with
// GemvFuse.stacked reads (in a multiple of 128).
hipError_t launch_swiglu_prepare(const uint16_t *g, const uint16_t *u, const uint16_t *suh,
                                 uint16_t *xp, int rows, int in, float limit, hipStream_t s);
// The decode attention's combine (its split slots in part, as
// exl3d_attn_decode_rope with out NULL leaves them) into prepared rows xp
// [B][nq * 128] for the consumer linear with suh.
hipError_t launch_attn_combine_prepare(const float *part, int B, int nq, int nkv, int Tmax,
                                       const uint16_t *suh, uint16_t *xp, hipStream_t s);
// The RMSNorm of an f32 residual h [B][H] (exl3d_add_rmsnorm's arithmetic)
// prepared for `count` (<= 4) consumer linears: xp holds count stacked
// [B][H] sets, set c prepared with suh[c] (H a multiple of 512, <= 8192).
hipError_t launch_rmsnorm_prepare(const float *h, const uint16_t *w, int B, int H, float eps,
                                  const uint16_t *const *suh, int count, uint16_t *xp,
                                  hipStream_t s);
// h = f16(silu(g) * u) elementwise, the SwiGLU prologue's arithmetic.
hipError_t launch_swiglu(const uint16_t *g, const uint16_t *u, uint16_t *h, size_t n, float limit,
                         hipStream_t s);
// The down projection of a dense SwiGLU MLP: y = (silu(g) * u) @ W^T, the
// SwiGLU with the MoE mid step's arithmetic (clamped by limit > 0); g, u f16
// [rows, in].  Up to SWIGLU_PROLOGUE_ROWS rows the GEMV applies it as it
// prepares its rows (one launch); more rows go through h (f16 [rows, in],
// caller's scratch) first.
constexpr int SWIGLU_PROLOGUE_ROWS = 4;
hipError_t launch_gemv_swiglu(const GemvLinear &l, const Format &f, const uint16_t *g,
                              const uint16_t *u, uint16_t *h, float limit, int ydt, int rows,
                              int in, Scratch &sc, hipStream_t s);
// GEMM (any rows): the same contract through LDS-staged decode and MFMA.
// Grids of at most 128 tiles (small rows or outputs) split k: the
// splits store f32 planes (kpart, gemm_split's size, private to the
// stream) and a second launch adds them and finishes.
constexpr int GM_SPLIT_MAX = 32;
constexpr int GM_SPLIT_TILES = 128;  // grids above this many tiles run whole
struct GemmSplit {
  int splits = 1, tiles = 0;
  size_t part_floats = 0;
};
GemmSplit gemm_split(int rows, int in, int out);
// The split-K plane floats a launch_gemm call of `rows` rows needs (its row
// windows' largest; 0: no split).
size_t gemm_kpart_floats(int64_t rows, int in, int out);
hipError_t launch_gemm(const uint16_t *trellis, const Format &f, const uint16_t *xp,
                       const uint16_t *svh, void *y, int ydt, uint16_t *zout, int rows, int in,
                       int out, float *kpart, size_t kpart_floats, hipStream_t s);
// The split of one GEMV launch over weights of total output width
// total_out: a linear of width out needs ksplit * rows * out partial floats.
void gemv_multi_plan(int in, int total_out, bool generic, int rows, int *ksplit, int *tps);

// ------------------------------------------------------------------- MoE

struct MoeBank {
  const uint16_t *trellis;  // [E][in/16][out/16][n]
  const uint16_t *suh;      // [E][in]
  const uint16_t *svh;      // [E][out]
  Format f;
  int in, out;
};

// Routed SwiGLU over `rows` rows of x [rows, hidden] (ACT_*), experts
// inds [rows, topk] (i32 or u32: both read as u32, out-of-range slots
// contribute nothing), scores [rows, topk] (ACT_*); inds == nullptr: the
// dense SwiGLU of expert 0 (topk 1, score 1).  limit > 0 clamps gate and up.
// y [rows, hidden] in ydt.
// The most slots (rows x topk) one launch_moe call orders; the host runs
// larger calls as windows of whole rows.
constexpr int MOE_SLOTS_MAX = 65535;
struct MoeArgs {
  const void *x;
  int xdt;
  const uint32_t *inds;
  const void *scores;
  int sdt;
  int rows, topk, experts, hidden, inter;
  float limit;
  void *y;
  int ydt;
  // the decode chain (grouped GEMV items) at any row count
  // (exl3_swiglu_opts.verify_rows)
  bool verify_rows;
};
// Whether a routed call takes the grouped GEMM (prefill-sized expert
// batches: at least 32 slots per expert on average, integer rates, and not
// verify_rows) rather than the grouped GEMV's items of up to 4 slots.
bool moe_uses_gemm(const MoeArgs &a, bool gu_generic, bool d_generic);
// Staging bytes for a call, and (in *partial_floats) the partial-sum slots
// of its Scratch.
size_t moe_scratch_bytes(const MoeArgs &a, bool gu_generic, bool d_generic,
                         size_t *partial_floats);
// shared (optional): a shared expert's linears (each a bank of one), served
// inside the routed launches as expert index a.experts - 1, whose slots the
// caller's inds / scores hold (launch_moe_shared_route makes them); the GEMV
// path only (moe_uses_gemm false), of the banks' formats and widths.
struct MoeShared {
  MoeBank gate, up, down;
  // one row with its k routes given (routes_k = k > 0): a.inds / a.scores
  // are the caller's k routes (scores in a.sdt) and slot k the shared
  // expert, whose gate sigmoid(logit or x . gate_vec) (xdt) the combine
  // forms; no route launch (see moe_shared_direct)
  int routes_k = 0;
  const void *logit = nullptr, *gate_vec = nullptr;
};
// Whether launch_moe takes a one-row swiglu_shared call with given routes
// without the route launch (its launches are small enough for the mid step
// in the down GEMV's prepare).
bool moe_shared_direct(const MoeArgs &a, bool gu_generic, bool d_generic);
hipError_t launch_moe(const MoeArgs &a, const MoeBank &gate, const MoeBank &up,
                      const MoeBank &down, void *scratch, size_t scratch_bytes,
                      const Scratch &slots, hipStream_t s, const MoeShared *shared = nullptr);
// The routes of a swiglu with a shared expert, k + 1 slots per row into
// inds_out / scores_out (f32): the routed experts' as given (inds, scores in
// sdt) or, with logits [rows][E] (xdt), the softmax's top k (ties: the lower
// index) renormalized to sum 1; then the shared expert (index E) with score
// sigmoid(logit) rounded to xdt, the logit given per row (logit [rows], xdt)
// or the dot of x's row with gate_vec [hidden] (xdt), rounded to xdt.
hipError_t launch_moe_shared_route(const uint32_t *inds, const void *scores, int sdt,
                                   const void *logits, int experts, int k, const void *logit,
                                   const void *gate_vec, const void *x, int xdt, int rows,
                                   int hidden, uint32_t *inds_out, float *scores_out,
                                   hipStream_t s);

}  // namespace exl3
