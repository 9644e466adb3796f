// exl3_kern.h -- the rate-templated EXL3 kernels (GEMV, GEMM, grouped MoE
// GEMV) and their per-rate launchers, for MI355X (gfx950, wave64).
//
// Included by exl3_kernels.hip (dispatchers; it sees the launchers as
// extern instantiations) and by exl3_rate.hip, which the build compiles once
// per rate K with EXL3_INST_K = K to instantiate that rate's kernels, so the
// rates compile in parallel.  Paths in citations are relative to
// /root/reference/plugins/.
#pragma once

#include <algorithm>
#include <utility>

#include "exl3_device.h"
#include "exl3_kernels.h"

namespace exl3 {


template <int... Is, typename F>
__device__ __forceinline__ void static_for_impl(std::integer_sequence<int, Is...>, F &&f) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl(std::make_integer_sequence<int, N>{}, f);
}

// Agent-scope (all XCDs) loads and stores for the split-K hand-off, through
// the global address space (a flat access is also counted as an LDS
// operation, so a wait for LDS would wait for it too).
typedef __attribute__((address_space(1))) uint32_t gu32_t;
typedef __attribute__((address_space(1))) float gf32_t;
__device__ __forceinline__ void st_agent(float *p, float v) {
  __hip_atomic_store((gf32_t *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// An agent-scope load (sc1, the bit an agent-scope atomic load's
// global_load carries) through a buffer resource: the base in SGPRs, a
// per-lane byte offset and a uniform one, so many slots of one lane cost one
// VGPR of address between them.  Offsets stay below 2^31 (the hosts check
// the slot planes' size).  The empty asm with a memory clobber keeps a poll
// loop's load from being hoisted or merged: the load is re-issued on every
// call.
__device__ __forceinline__ float ld_agent_at(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                             uint32_t soff) {
  asm volatile("" ::: "memory");
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 16));
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(float *base) {
  return __builtin_amdgcn_make_buffer_rsrc(base, (short)0, 0x7FFFFFFF, 0x00020000);
}
// s_waitcnt vmcnt(0): this wave's outstanding vector-memory operations,
// stores included on gfx9-family parts, have completed.
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0x0F70); }
// Workgroup barrier that orders LDS only: the fences name the local address
// space, so the barrier waits for this wave's LDS operations (lgkmcnt) but
// not for its global loads in flight (a __syncthreads() fence also covers
// global memory and so waits for every outstanding load, prefetches
// included).  Global memory shared between waves is ordered explicitly.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ===================================================================== GEMV
//
// One launch per matmul of up to 16 rows, and one launch for up to four
// weights that read the same rows (q/k/v, gate/up: the reference's
// linearShared, sushi_ds41/src/sushi/exl3/linear.zig:34-60), their column
// groups side by side in the grid.  A workgroup (8 waves) owns one
// 128-column group (8 output tiles: one Hadamard block of the output) of one
// weight and one k-split of tps k-tile rows (whole input Hadamard blocks):
//  1. it prepares its rows' input slice in LDS (x * suh, Hadamard-128, f16:
//     the reference's prepare, run per split instead of as its own launch);
//  2. wave w takes tiles 2q, 2q+1 (q = w % 4) of the group over k-part w / 4
//     of the split; lane l = 16g + 8t + c takes chunk c of tile 2q+t in
//     k-tile row 4i+g of its part at step i, loads its K dwords (+ the
//     history dword of lane l-1 of its tile, by ds_bpermute), decodes its 32
//     codewords in registers into four 8 x f16 MFMA B operands (column a /
//     a+8, rows 0-7 / 8-15), and v_mfma_f32_16x16x32_f16 sums them against
//     the rows' activations (A operands from LDS) over the step's 4 k-tile
//     rows.  MFMA rows are the call's rows: 1..16 rows cost one decode;
//  3. the two k-parts add in LDS; the other splits' per-row sums go to
//     scratch slots, and the workgroup of the last split (the highest
//     workgroup index of the column group) adds the splits in split order,
//     rounds z to f16 and runs the finish (Hadamard-128, * svh) on its 128
//     columns.  Every sum is in a fixed order that does not depend on how
//     many rows share the call.
//  With mul1 at an integer rate the MFMAs take the codebook value before its
//  affine step (chunk_pair_mul1_h) and the step is applied to the sums.
//
//  Every memory round trip is on the critical path of a launch this small
//  (a q/o linear at K=4 is 8 MiB: about 1 us of HBM time), so the trellis
//  and activation pointers and the launch geometry are kernel arguments that
//  gfx950 preloads into SGPRs: a workgroup issues its weight and activation
//  loads at its first instructions, with no kernel-argument load before them.

constexpr int GEMV_THREADS = 512;
constexpr int GEMV_ROWS = 16;
constexpr int GEMV_TPS_MAX = 64;
// k-tile rows a GEMV workgroup takes at one or two rows (their prepare items
// fit the rows form's first pass)
constexpr int GEMV_TPS_ONE_ROW_MAX = 128;
static_assert(2 * (GEMV_TPS_ONE_ROW_MAX / 8) <= GEMV_THREADS / 16, "two rows in one pass");
constexpr int GEMV_KSPLIT_MAX = 64;
constexpr int GEMV_MAXW = 4;
// Prepare items (one row's 128-block) per wave per batch, and per batch of
// the workgroup.
constexpr int PREP_BATCH = 2;
constexpr int PREP_ITEMS = PREP_BATCH * (GEMV_THREADS / 64);

struct GemvRow {
  int in_off;   // element offset of the row's activations
  int out_off;  // element offset of the row's output
  int prow;     // row of the split-K partial buffer
  int pad;
};

// Per weight, read from the kernel-argument segment after the loads are out.
struct GemvWeight {
  const uint16_t *suh;  // [E][in]
  const uint16_t *svh;  // [E][out]
  void *y;              // finished output in ydt, or nullptr:
  uint16_t *zout;       // the inner product z (f16) instead
  float *partial;       // [ksplit][ptotal][out] slots, empty between calls
  size_t expert_words;  // trellis dwords per expert
  // routed launches with a shared expert: expert index GemvCfg::shared_expert
  // reads this linear (trellis, suh, svh) instead of the bank's
  const uint32_t *sh_tw;
  const uint16_t *sh_suh;
  const uint16_t *sh_svh;
};

struct GemvCfg {
  size_t ptotal;  // rows of the partial-sum slots
  // the word a split-K wait that gives up sets, and the wait's bound
  uint32_t *status;
  int poll_max;
  // failure-handling tests only (the host sets it on request): the splits
  // other than the last skip their partial-sum stores, so the last split's
  // wait gives up at its bound
  int drop_partials;
  int ydt;
  int ksplit;
  CbRow dec;            // window mask and table row
  int nw;               // trellis dwords per tile (n / 2)
  const uint16_t *x2;   // SwiGLU prologue: up (f16, the layout of x = gate)
  float limit;          // ... and its clamp (0: none)
  // RMSNorm prologue: x is the f32 residual h [rows][in]; nssq [rows][in /
  // 128] its sums of squares per 128 columns; x = f16(h * r * nw), r =
  // rsqrt(sum / in + eps)
  const float *nssq;
  const uint16_t *nw_norm;
  float eps;
  // residual finish (res set): res[row][col] += f32(y) instead of storing y,
  // and res_ssq[row][group] = the group's sum of squares of the new res
  float *res;
  float *res_ssq;
  int shared_expert;  // routed launches: the index of the shared expert (-1: none)
  int experts;        // routed launches without an item list: expert indices below this
  int routes_k;       // ... > 0: sorted holds k routes, slot k is the shared expert
  // attention prologue (set: on; the launch's x is then this pointer): the
  // decode attention's per-split slots [rows][attn_nkv][attn_nsplit]
  // [attn_g][128 + 2] (o values, then m, l)
  const float *attn_part;
  int attn_nkv, attn_g, attn_nsplit;
};

// Prologue forms of the GEMV prepare (compile time: they decide which loads
// a workgroup issues at its start).
constexpr int PRO_PLAIN = 0, PRO_SWIGLU = 1, PRO_RMSNORM = 2, PRO_ATTN = 3;


// The SwiGLU of one element pair of gate (g) and up (u), f16 bits: the MoE
// mid step's arithmetic: h = f16(silu(g) * u), silu(g) = g / (1 + e^-g) in
// f32, clamped first when limit > 0 (swiglu_clamp).
__device__ __forceinline__ float swiglu1(uint16_t gb, uint16_t ub, float limit) {
  float gv = h2f(gb), uv = h2f(ub);
  if (limit > 0.0f) swiglu_clamp(gv, uv, limit);
  return h2f(f2h(f32_value(gv / (1.0f + expf(-gv))) * uv));
}
__device__ __forceinline__ void swiglu_unpack(uint32_t g2, uint32_t u2, float limit, float &a,
                                              float &b) {
  a = swiglu1((uint16_t)(g2 & 0xFFFFu), (uint16_t)(u2 & 0xFFFFu), limit);
  b = swiglu1((uint16_t)(g2 >> 16), (uint16_t)(u2 >> 16), limit);
}

struct GemvArgs {
  GemvCfg c;
  GemvWeight w[GEMV_MAXW];
};

// Launch geometry in three words (preloaded SGPRs, so that no launch value
// costs a load; gridDim itself is a load from the implicit arguments):
//   g0 = cg1 | cg2 << 16     first column groups of weights 1, 2 (0: absent)
//   g1 = cg3 | cgend << 16   ... of weight 3, and the end of the last weight
//   g2 = in_tiles | tps << 16 | rows << 23 | xdt << 28 | prepared << 30 |
//        stacked << 31 (prepared rows: one [rows][in] set per weight, stacked)
struct GemvGeo {
  int cg1, cg2, cg3, cgend, in_tiles, tps, rows, xdt, prepared, stacked;
  __host__ __device__ static GemvGeo unpack(uint32_t g0, uint32_t g1, uint32_t g2) {
    GemvGeo g;
    g.cg1 = (int)(g0 & 0xFFFFu);
    g.cg2 = (int)(g0 >> 16);
    g.cg3 = (int)(g1 & 0xFFFFu);
    g.cgend = (int)(g1 >> 16);
    g.in_tiles = (int)(g2 & 0xFFFFu);
    g.tps = 8 * (int)((g2 >> 16) & 0x7Fu);  // stored in blocks of 8 tiles
    g.rows = (int)((g2 >> 23) & 0x1Fu);
    g.xdt = (int)((g2 >> 28) & 3u);
    g.prepared = (int)((g2 >> 30) & 1u);
    g.stacked = (int)(g2 >> 31);
    return g;
  }
};
// Fields: cg1, cg2, cg3, cgend, in_tiles 16 bits each; tps / 8 in 7 bits
// (tps a multiple of 8, at most 1016); rows 5, xdt 2, prepared 1, stacked 1.  False
// when a value does not fit its field (the launchers refuse the launch).
inline bool gemv_geo_pack(const GemvGeo &g, uint32_t *g0, uint32_t *g1, uint32_t *g2) {
  if (g.cg1 < 0 || g.cg1 > 0xFFFF || g.cg2 < 0 || g.cg2 > 0xFFFF || g.cg3 < 0 ||
      g.cg3 > 0xFFFF || g.cgend < 0 || g.cgend > 0xFFFF || g.in_tiles < 0 ||
      g.in_tiles > 0xFFFF || g.tps <= 0 || g.tps % 8 != 0 || g.tps / 8 > 0x7F || g.rows < 0 ||
      g.rows > 0x1F || g.xdt < 0 || g.xdt > 3)
    return false;
  *g0 = (uint32_t)g.cg1 | ((uint32_t)g.cg2 << 16);
  *g1 = (uint32_t)g.cg3 | ((uint32_t)g.cgend << 16);
  *g2 = (uint32_t)g.in_tiles | ((uint32_t)(g.tps / 8) << 16) | ((uint32_t)g.rows << 23) |
        ((uint32_t)g.xdt << 28) | ((uint32_t)(g.prepared & 1) << 30) |
        ((uint32_t)(g.stacked & 1) << 31);
  return true;
}

// Row b of a workgroup: its activations, output and partial-sum row.  A
// table in LDS (the MoE's slots) or, without one, row b of the call.
struct RowMap {
  const GemvRow *t;
  int in, out;
  __device__ __forceinline__ int in_off(int b) const { return t ? t[b].in_off : b * in; }
  __device__ __forceinline__ int out_off(int b) const { return t ? t[b].out_off : b * out; }
  __device__ __forceinline__ int prow(int b) const { return t ? t[b].prow : b; }
};

// Dynamic LDS of a GEMV workgroup: row table, prepared rows, the two
// k-parts' z tiles, the prepared rows' sums per 64 elements, and (generic
// rate) a word stage per wave.
__host__ __device__ constexpr size_t gemv_lds_bytes(int rows_alloc, int tps, bool generic) {
  return 256 + (size_t)rows_alloc * (tps * 16 + 8) * 2 +
         (size_t)2 * (rows_alloc > 2 ? rows_alloc : 2) * 128 * 4 +
         (size_t)rows_alloc * (tps / 4) * 4 +
         (generic ? (size_t)(GEMV_THREADS / 64) * 512 * 4 : 0);
}

// The rows' input slice [tk0*16, tk0*16 + ntk*16) prepared into xs (row
// stride kr halfs): one wave per (row, 128-block) item.  Loads and
// arithmetic are split so a workgroup issues its first items' loads with its
// weight loads.

// Batch j of a wave's prepare holds item base + 8 j + wave; an item past the
// last would only redo the last one (its index clamped), so the wave skips
// it and every later batch (the test is uniform within the wave).
__device__ __forceinline__ bool prep_item_live(int j, int base, int wave, int nitems) {
  return base + wave + j * (GEMV_THREADS / 64) < nitems;
}

// Raw bits as loaded (converted only when the rows are prepared, so the
// loads do not wait): x holds the two elements (one dword for f16/bf16, two
// for f32), su the two suh values.
struct PrepRegs {
  uint32_t x0[PREP_BATCH], x1[PREP_BATCH], su[PREP_BATCH];
  uint32_t nw[PREP_BATCH];  // RMSNorm: weights of the pair
  float nt[PREP_BATCH];     // ... and the row's partial sums of squares
};

// RMSNorm prologue: the item's norm-weight pair and the lane's share of its
// row's partial sums (nssq[row][lane], 0 past the row's groups).
__device__ __forceinline__ void gemv_prep_load_norm(const GemvCfg &a, const RowMap &rm,
                                                    int nitems, int nb, int tk0, int in, int base,
                                                    int wave, int lane, PrepRegs &r) {
  const uint16_t *nwp = a.nw_norm;
  const float *ssq = a.nssq;
  asm volatile("" : "+s"(nwp), "+s"(ssq)::"memory");
  const int ng = in >> 7;
#pragma unroll
  for (int j = 0; j < PREP_BATCH; ++j) {
    if (!prep_item_live(j, base, wave, nitems)) break;
    const int it = min(base + wave + j * (GEMV_THREADS / 64), nitems - 1);
    const int row = it / nb, blk = it - row * nb;
    const int k = tk0 * 16 + blk * 128 + 2 * lane;
    r.nw[j] = *(const __attribute__((address_space(1))) uint32_t *)(nwp + k);
    const float t = *(const __attribute__((address_space(1))) float *)(ssq + (size_t)row * ng +
                                                                          min(lane, ng - 1));
    r.nt[j] = lane < ng ? t : 0.0f;
  }
}
__device__ __forceinline__ float norm_scale(float part, int in, float eps) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) part += xor_lanes(part, m);
  return rsqrtf(part / (float)in + eps);
}

// Branch-free: all three readings are formed and one is selected, so no
// control flow joins while the weight loads are in flight.
__device__ __forceinline__ void prep_unpack(uint32_t x0, uint32_t x1, int dt, float &a, float &b) {
  const float fa = h2f((uint16_t)(x0 & 0xFFFFu)), fb = h2f((uint16_t)(x0 >> 16));
  const float ba = bits<float>(x0 << 16), bb = bits<float>(x0 & 0xFFFF0000u);
  const float sa = bits<float>(x0), sb = bits<float>(x1);
  a = dt == OUT_F32 ? sa : dt == OUT_BF16 ? ba : fa;
  b = dt == OUT_F32 ? sb : dt == OUT_BF16 ? bb : fb;
}

// Items past the last one load (and later store) the last item again: the
// same values to the same place.  Every lane issues the same loads whatever
// the dtype (f16/bf16 read their dword twice; prepared rows read x in place
// of suh), so the batch has no branches around its loads and the waits for
// them do not also wait for the weight loads in flight.  The activations
// need only preloaded arguments; suh needs its pointer from the argument
// segment, so it is a second call.
__device__ __forceinline__ void gemv_prep_load_x(const void *x, int xdt, int prepared,
                                                 const RowMap &rm, int nitems, int nb, int tk0,
                                                 int base, int wave, int lane, PrepRegs &r) {
  const int esz = (!prepared && xdt == OUT_F32) ? 4 : 2;
#pragma unroll
  for (int j = 0; j < PREP_BATCH; ++j) {
    if (!prep_item_live(j, base, wave, nitems)) break;
    const int it = min(base + wave + j * (GEMV_THREADS / 64), nitems - 1);
    const int row = it / nb, blk = it - row * nb;
    const int k = tk0 * 16 + blk * 128 + 2 * lane;
    const char *pa = (const char *)x + ((size_t)rm.in_off(row) + k) * esz;
    r.x0[j] = *reinterpret_cast<const uint32_t *>(pa);
    r.x1[j] = *reinterpret_cast<const uint32_t *>(pa + (esz - 2) * 2);
  }
}
// A load through the global address space (a pointer that passed through
// inline asm is otherwise generic, and a flat load is waited for as both a
// vector-memory and an LDS operation).
__device__ __forceinline__ uint32_t ld_global_u32(const void *p) {
  return *(const __attribute__((address_space(1))) uint32_t *)p;
}

__device__ __forceinline__ void gemv_prep_load_su(const void *x, int prepared, const uint16_t *suh,
                                                  int nitems, int nb, int tk0, int base, int wave,
                                                  int lane, PrepRegs &r) {
  const uint16_t *sup = prepared ? (const uint16_t *)x : suh;
#pragma unroll
  for (int j = 0; j < PREP_BATCH; ++j) {
    if (!prep_item_live(j, base, wave, nitems)) break;
    const int it = min(base + wave + j * (GEMV_THREADS / 64), nitems - 1);
    const int blk = it % nb;
    const int k = tk0 * 16 + blk * 128 + 2 * lane;
    r.su[j] = ld_global_u32(sup + k);
  }
}

// SwiGLU prologue: the up pair of every item into x1 (gate is x, loaded by
// gemv_prep_load_x as f16).
__device__ __forceinline__ void gemv_prep_load_up(const uint16_t *x2, const RowMap &rm,
                                                  int nitems, int nb, int tk0, int base, int wave,
                                                  int lane, PrepRegs &r) {
#pragma unroll
  for (int j = 0; j < PREP_BATCH; ++j) {
    if (!prep_item_live(j, base, wave, nitems)) break;
    const int it = min(base + wave + j * (GEMV_THREADS / 64), nitems - 1);
    const int row = it / nb, blk = it - row * nb;
    const int k = tk0 * 16 + blk * 128 + 2 * lane;
    r.x1[j] = ld_global_u32(x2 + (size_t)rm.in_off(row) + k);
  }
}

// Attention prologue: input element pair (2 lane, 2 lane + 1) of query head
// hq of batch row b, combined from the decode attention's split slots as
// its combine step does (decoder_ops.hip attn_combine_kernel): M = the
// largest m_s, f_s = e^(m_s - M) (0 for an empty split), out =
// f16(sum_s o_s f_s / sum_s l_s f_s), both sums in split order, the same
// f32 operations, so the values equal the combine's output bit for bit.
// Lane i holds m, l of split c0 + i of its 64-split chunk c0; a split's
// factor and l * f reach every lane by readlane, in split order.  The first
// round of loads (o of splits 0..31, m and l of splits 0..63) is issued by
// attn_load, early in the workgroup; attn_combine does the rest.
constexpr int ATTN_CH = 32;
typedef float attn_f2_t __attribute__((ext_vector_type(2)));
struct AttnLoads {
  attn_f2_t ov[ATTN_CH];
  float mv, lv;
};
struct AttnItem {
  const float *base;  // split 0's slot of this head
  size_t sst;         // floats between splits
  int ns;
};
__device__ __forceinline__ AttnItem attn_item(const float *part, const GemvCfg &a, int b, int hq) {
  constexpr int D = 128;
  const int kvh = hq / a.attn_g, g = hq - kvh * a.attn_g;
  const size_t sst = (size_t)a.attn_g * (D + 2);
  return AttnItem{part + ((size_t)b * a.attn_nkv + kvh) * a.attn_nsplit * sst + g * (D + 2), sst,
                  a.attn_nsplit};
}
__device__ __forceinline__ attn_f2_t attn_ld_o(const AttnItem &t, int s, int lane) {
  return *(const __attribute__((address_space(1))) attn_f2_t *)(t.base + (size_t)s * t.sst +
                                                                2 * lane);
}
__device__ __forceinline__ void attn_ld_ml(const AttnItem &t, int c0, int lane, float &m,
                                           float &l) {
  const int s = min(c0 + lane, t.ns - 1);
  const attn_f2_t v =
      *(const __attribute__((address_space(1))) attn_f2_t *)(t.base + (size_t)s * t.sst + 128);
  m = c0 + lane < t.ns ? v.x : -INFINITY;
  l = v.y;
}
__device__ __forceinline__ void attn_load(const AttnItem &t, int lane, AttnLoads &L) {
#pragma unroll
  for (int j = 0; j < ATTN_CH; ++j) L.ov[j] = attn_ld_o(t, min(j, t.ns - 1), lane);
  attn_ld_ml(t, 0, lane, L.mv, L.lv);
}
__device__ __forceinline__ uint32_t attn_combine(const AttnItem &t, int lane, AttnLoads &L) {
  const int ns = t.ns;
  float M = L.mv;
  for (int c0 = 64; c0 < ns; c0 += 64) {
    float m2, l2;
    attn_ld_ml(t, c0, lane, m2, l2);
    M = fmaxf(M, m2);
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) M = fmaxf(M, xor_lanes(M, m));
  float Ls = 0.0f, acc0 = 0.0f, acc1 = 0.0f;
  float mv = L.mv, lv = L.lv, fv = 0.0f, pv = 0.0f;
  for (int s0 = 0; s0 < ns; s0 += ATTN_CH) {
    if ((s0 & 63) == 0) {
      if (s0 > 0) attn_ld_ml(t, s0, lane, mv, lv);
      fv = mv == -INFINITY ? 0.0f : __expf(mv - M);
      pv = lv * fv;
    }
    if (s0 > 0) {
#pragma unroll
      for (int j = 0; j < ATTN_CH; ++j) L.ov[j] = attn_ld_o(t, min(s0 + j, ns - 1), lane);
    }
#pragma unroll
    for (int j = 0; j < ATTN_CH; ++j) {
      if (s0 + j < ns) {
        const int ln = (s0 + j) & 63;
        const float f = bits<float>((uint32_t)__builtin_amdgcn_readlane((int)bits<uint32_t>(fv), ln));
        const float p = bits<float>((uint32_t)__builtin_amdgcn_readlane((int)bits<uint32_t>(pv), ln));
        Ls += p;
        acc0 += L.ov[j].x * f;
        acc1 += L.ov[j].y * f;
      }
    }
  }
  return (uint32_t)f2h(acc0 / Ls) | ((uint32_t)f2h(acc1 / Ls) << 16);
}

// The attention prologue's input pairs of every item into x0 (f16 bits);
// the wave's first item's first round of loads was issued into L (when the
// item is live).
__device__ __forceinline__ void gemv_prep_attn(const float *part, const GemvCfg &a, int nitems,
                                               int nb, int tk0, int base, int wave, int lane,
                                               AttnLoads &L, PrepRegs &r) {
#pragma unroll
  for (int j = 0; j < PREP_BATCH; ++j) {
    if (!prep_item_live(j, base, wave, nitems)) break;
    const int it = min(base + wave + j * (GEMV_THREADS / 64), nitems - 1);
    const int row = it / nb, blk = it - row * nb;
    const AttnItem t = attn_item(part, a, row, tk0 / 8 + blk);
    if (j > 0) attn_load(t, lane, L);
    r.x0[j] = attn_combine(t, lane, L);
    r.x1[j] = 0u;
  }
}

// Element i of a 128-block sits in lane i/2, register i%2: the butterfly's
// stage on index bit 0 is in-register, bits 1..6 exchange across lanes; each
// stage is (lo + hi, lo - hi), in bit order, as the reference's kernels
// compute it (expert_exl3_kernels.zig:902-970).
__device__ __forceinline__ void had128_pair(float &v0, float &v1, int lane) {
  const float a = v0 + v1, b = v0 - v1;
  v0 = a;
  v1 = b;
#pragma unroll
  for (int bit = 1; bit <= 32; bit <<= 1) {
    const float p0 = xor_lanes(v0, bit), p1 = xor_lanes(v1, bit);
    const float sg = (lane & bit) == 0 ? 1.0f : -1.0f;
    v0 = butterfly(sg, v0, p0);
    v1 = butterfly(sg, v1, p1);
  }
}

// Stores the prepared pairs; with hsum (row stride nb * 2) also the sum of
// each 64 prepared elements (lanes 0-31 and 32-63 of an item), added in a
// fixed butterfly order.
template <int PRO = PRO_PLAIN>
__device__ __forceinline__ void gemv_prep_store(int xdt, int prepared, int nitems, int nb,
                                                int base, int wave, int lane, uint16_t *xs, int kr,
                                                const PrepRegs &r, float *hsum, float limit = 0.0f,
                                                int in = 0, float eps = 0.0f) {
#pragma unroll
  for (int j = 0; j < PREP_BATCH; ++j) {
    if (!prep_item_live(j, base, wave, nitems)) break;
    const int it = min(base + wave + j * (GEMV_THREADS / 64), nitems - 1);
    const int row = it / nb, blk = it - row * nb;
    uint32_t *dst = reinterpret_cast<uint32_t *>(xs + row * kr + blk * 128 + 2 * lane);
    // f16(x) * suh in f32, the butterfly, * 1/sqrt(128), f16
    // (expert_exl3.zig:490-501); prepared rows are taken as they are (the
    // rotation is formed regardless and not used: no branch)
    float x0, x1;
    if constexpr (PRO == PRO_SWIGLU) {
      swiglu_unpack(r.x0[j], r.x1[j], limit, x0, x1);  // x0: gate pair, x1: up pair
    } else if constexpr (PRO == PRO_RMSNORM) {
      // the residual pair (f32) normalized: f16(h * r * w)
      const float rs = norm_scale(r.nt[j], in, eps);
      x0 = h2f(f2h(bits<float>(r.x0[j]) * rs * h2f((uint16_t)(r.nw[j] & 0xFFFFu))));
      x1 = h2f(f2h(bits<float>(r.x1[j]) * rs * h2f((uint16_t)(r.nw[j] >> 16))));
    } else {
      prep_unpack(r.x0[j], r.x1[j], xdt, x0, x1);
    }
    float v0 = h2f(f2h(x0)) * h2f((uint16_t)(r.su[j] & 0xFFFFu));
    float v1 = h2f(f2h(x1)) * h2f((uint16_t)(r.su[j] >> 16));
    had128_pair(v0, v1, lane);
    const uint32_t rot = (uint32_t)f2h(v0 * HAD_SCALE) | ((uint32_t)f2h(v1 * HAD_SCALE) << 16);
    const uint32_t y = prepared ? r.x0[j] : rot;
    *dst = y;
    if (hsum != nullptr) {
      float s = h2f((uint16_t)(y & 0xFFFFu)) + h2f((uint16_t)(y >> 16));
#pragma unroll
      for (int m = 1; m < 32; m <<= 1) s = s + xor_lanes(s, m);
      if ((lane & 31) == 0) hsum[row * nb * 2 + blk * 2 + (lane >> 5)] = s;
    }
  }
}

// Prepare of many rows (more items than one batch): all of a workgroup's
// rows in one pass of loads.  A 128-block is held by 16 consecutive lanes, 8
// consecutive elements each: the butterfly's stages on index bits 0-2 are
// in-register, bits 3-6 exchange across the 16 lanes; every element sees the
// same f32 operations in the same order as in had128_pair, so a row's
// prepared values (and its 64-element sums, the same pairwise tree) do not
// depend on which path prepared it.  Group G = tid / 16 + 32 p of pass p
// takes block G of the workgroup (row G / nb, block G % nb); groups past the
// last block redo the last block (the same values to the same place).
constexpr int PREP_GROUPS = GEMV_THREADS / 16;
constexpr int PREP_PASSES = GEMV_ROWS * (GEMV_TPS_MAX / 8) / PREP_GROUPS;

// NP passes of the PREP_GROUPS groups cover nblk <= NP * PREP_GROUPS blocks
// (a launch takes the smallest NP in 1, 2, PREP_PASSES that covers its rows).
template <int NP>
struct RowsRegs {
  u4_t x[NP][2];  // 8 elements: one 16-byte piece (f16/bf16) or two (f32)
  u4_t su[NP];
};

template <int NP>
__device__ __forceinline__ void gemv_rows_load_x(const void *x, int xdt, int prepared,
                                                 const RowMap &rm, int nblk, int nb, int tk0,
                                                 RowsRegs<NP> &r) {
  const int esz = (!prepared && xdt == OUT_F32) ? 4 : 2;
  const int li = threadIdx.x & 15;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int G = min((int)(threadIdx.x >> 4) + PREP_GROUPS * p, nblk - 1);
    const int row = G / nb, blk = G - row * nb;
    const int k = tk0 * 16 + blk * 128 + 8 * li;
    const char *pa = (const char *)x + ((size_t)rm.in_off(row) + k) * esz;
    r.x[p][0] = *reinterpret_cast<const u4_t *>(pa);
    r.x[p][1] = *reinterpret_cast<const u4_t *>(pa + (esz - 2) * 8);
  }
}

template <int NP>
__device__ __forceinline__ void gemv_rows_load_su(const void *x, int prepared, const uint16_t *suh,
                                                  int nblk, int nb, int tk0, RowsRegs<NP> &r) {
  const uint16_t *sup = prepared ? (const uint16_t *)x : suh;
  const int li = threadIdx.x & 15;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int G = min((int)(threadIdx.x >> 4) + PREP_GROUPS * p, nblk - 1);
    const int blk = G % nb;
    r.su[p] = *(const __attribute__((address_space(1))) u4_t *)(sup + tk0 * 16 + blk * 128 + 8 * li);
  }
}

// SwiGLU prologue (rows form): the up pieces into x[p][1].
template <int NP>
__device__ __forceinline__ void gemv_rows_load_up(const uint16_t *x2, const RowMap &rm, int nblk,
                                                  int nb, int tk0, RowsRegs<NP> &r) {
  const int li = threadIdx.x & 15;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int G = min((int)(threadIdx.x >> 4) + PREP_GROUPS * p, nblk - 1);
    const int row = G / nb, blk = G - row * nb;
    r.x[p][1] = *(const __attribute__((address_space(1))) u4_t *)(x2 + (size_t)rm.in_off(row) +
                                                                  tk0 * 16 + blk * 128 + 8 * li);
  }
}

template <int PRO, int NP>
__device__ __forceinline__ void gemv_rows_store(int xdt, int prepared, int nblk, int nb,
                                                uint16_t *xs, int kr, const RowsRegs<NP> &r,
                                                float *hsum, float limit = 0.0f) {
  const int li = threadIdx.x & 15, lane = threadIdx.x & 63;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int G = min((int)(threadIdx.x >> 4) + PREP_GROUPS * p, nblk - 1);
    const int row = G / nb, blk = G - row * nb;
    uint32_t y[4];
    if (prepared) {
      // prepared rows (a producer formed the rotation): taken as they are,
      // the rotation's VALU work skipped (a uniform branch)
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = r.x[p][0][e];
    } else {
      float v[8];
      // f16(x) * suh: inputs that are f16 values already (f16 rows, the
      // SwiGLU's f16 results) skip the rounding, an identity for them (a
      // uniform branch on the dtype)
      auto unpack = [&](auto IS16) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float a, b;
          if constexpr (PRO == PRO_SWIGLU) {
            swiglu_unpack(r.x[p][0][e], r.x[p][1][e], limit, a, b);  // gate, up pieces
          } else if constexpr (decltype(IS16)::value) {
            a = h2f((uint16_t)(r.x[p][0][e] & 0xFFFFu));
            b = h2f((uint16_t)(r.x[p][0][e] >> 16));
          } else {
            prep_unpack(r.x[p][0][e], 0u, xdt, a, b);  // bf16 pair e
            const float fa = bits<float>(r.x[p][e >> 1][2 * (e & 1)]);
            const float fb = bits<float>(r.x[p][e >> 1][2 * (e & 1) + 1]);
            if (xdt == OUT_F32) {
              a = fa;
              b = fb;
            }
            a = h2f(f2h(a));
            b = h2f(f2h(b));
          }
          const uint32_t su = r.su[p][e];
          v[2 * e] = a * h2f((uint16_t)(su & 0xFFFFu));
          v[2 * e + 1] = b * h2f((uint16_t)(su >> 16));
        }
      };
      if (PRO == PRO_SWIGLU || xdt == OUT_F16)
        unpack(std::true_type{});
      else
        unpack(std::false_type{});
      // stages on bits 0, 1, 2 (in-register), then 3-6 (lanes xor 1, 2, 4, 8)
#pragma unroll
      for (int m = 1; m < 8; m <<= 1) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (e & m) continue;
          const float lo = v[e], hi = v[e + m];
          v[e] = lo + hi;
          v[e + m] = lo - hi;
        }
      }
#pragma unroll
      for (int m = 1; m < 16; m <<= 1) {
        const float sg = (li & m) == 0 ? 1.0f : -1.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = butterfly(sg, v[e], xor_lanes(v[e], m));
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t rot =
            (uint32_t)f2h(v[2 * e] * HAD_SCALE) | ((uint32_t)f2h(v[2 * e + 1] * HAD_SCALE) << 16);
        y[e] = rot;
      }
    }
    const u4_t yv = {y[0], y[1], y[2], y[3]};
    *reinterpret_cast<u4_t *>(xs + row * kr + blk * 128 + 8 * li) = yv;
    if (hsum != nullptr) {
      // the 64-element sum as the pairwise tree had128_pair's layout forms:
      // in-lane pairs, then pairs of pairs, ..., then across lanes
      float s2[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        s2[e] = h2f((uint16_t)(y[e] & 0xFFFFu)) + h2f((uint16_t)(y[e] >> 16));
      float s = (s2[0] + s2[1]) + (s2[2] + s2[3]);
#pragma unroll
      for (int m = 1; m < 8; m <<= 1) s = s + xor_lanes(s, m);
      if ((li & 7) == 0) hsum[row * nb * 2 + blk * 2 + (li >> 3)] = s;
    }
  }
  (void)lane;
}

__device__ __forceinline__ h8_t frag(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  const u4_t v = {a, b, c, d};
  return bits<h8_t>(v);
}

// Four MFMAs of one step: columns a (acc0) and a+8 (acc1), rows 0-7 then 8-15.
__device__ __forceinline__ void gemv_mfma(const uint32_t (&p)[16], h8_t alo, h8_t ahi, f4_t &acc0,
                                          f4_t &acc1) {
  acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, frag(p[0], p[4], p[8], p[12]), acc0, 0, 0, 0);
  acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, frag(p[2], p[6], p[10], p[14]), acc1, 0, 0, 0);
  acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, frag(p[1], p[5], p[9], p[13]), acc0, 0, 0, 0);
  acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, frag(p[3], p[7], p[11], p[15]), acc1, 0, 0, 0);
}

// Split-K hand-off over zf[nrows][128] (this workgroup's f32 sums): returns
// true in the workgroup of the last split, with z = f16(sum over splits, in
// split order) in zf.  Partial-sum slots hold PARTIAL_EMPTY (a NaN bit
// pattern no arithmetic produces) between calls.  The other splits store
// their sums and exit; the last split's workgroup reads their slots,
// re-reading all of those still empty together (one round trip per round,
// up to 16 slots a round) until every store has landed, then puts
// PARTIAL_EMPTY back.  It never waits on a workgroup that has not started: the last split
// has the highest workgroup index of its column group, and workgroups are
// dispatched in index order, so every slot it waits for belongs to a
// workgroup already running, whose stores land within a memory round trip.
// PARTIAL_POLL_MAX bounds the wait regardless: a slot still empty then makes
// the sum NaN, is left as it is (its store may still land), and sets the
// status word, which the host reads (and after which it refills the slots:
// exl3_stream_status).  Slots are agent-scope atomics, coherent across the
// XCDs' L2s, so no fence is needed.  (A device fence would write back and
// invalidate the L2 in every workgroup.)
constexpr uint32_t PARTIAL_EMPTY = 0xFFFFFFFFu;
constexpr int PARTIAL_POLL_MAX = 1 << 20;

// The pause between polls of the split-K hand-off (s_sleep units of 64 cycles).
#ifndef EXL3_POLL_SLEEP
#define EXL3_POLL_SLEEP 2
#endif

// The last split's sum of the other splits' slots for this thread's
// elements e = e0 + tid + GEMV_THREADS j (j < EM, e < E): rounds of KC splits,
// every element's slots of a round read at once; a slot still empty is read
// again in the same round (at most poll_max times), and each slot read is
// set back to the empty mark.  zf[e] = f16(sum_k v_k + zf[e]), the sum in
// split order.  Returns whether a wait gave up.
template <int EM, int KC>
__device__ __forceinline__ bool splitk_sum(float *zf, __amdgpu_buffer_rsrc_t pr, uint32_t sstride,
                                           float *partial, size_t stride, int E, int e0, int ks,
                                           const RowMap &rm, size_t out, int col0, int poll_max) {
  static_assert(EM * KC <= 32, "one pending bit per read");
  const float empty = bits<float>(PARTIAL_EMPTY);
  uint32_t po[EM];
  float s[EM];
  bool live[EM];
#pragma unroll
  for (int i = 0; i < EM; ++i) {
    const int e = e0 + threadIdx.x + GEMV_THREADS * i;
    live[i] = e < E;
    const int ec = live[i] ? e : 0;  // (a dead element's place is never read)
    po[i] = (uint32_t)(((size_t)rm.prow(ec >> 7) * out + col0 + (ec & 127)) * 4);
    s[i] = 0.0f;
  }
  bool gave_up = false;
  for (int k0 = 0; k0 < ks; k0 += KC) {
    const int nk = min(KC, ks - k0);
    float v[EM][KC];
    uint32_t pending = 0;
#pragma unroll
    for (int i = 0; i < EM; ++i)
#pragma unroll
      for (int j = 0; j < KC; ++j)
        if (live[i] && j < nk) v[i][j] = ld_agent_at(pr, po[i], (uint32_t)(k0 + j) * sstride);
#pragma unroll
    for (int i = 0; i < EM; ++i)
#pragma unroll
      for (int j = 0; j < KC; ++j)
        if (live[i] && j < nk && bits<uint32_t>(v[i][j]) == PARTIAL_EMPTY)
          pending |= 1u << (i * KC + j);
    for (int n = 0; pending != 0 && n < poll_max; ++n) {
      __builtin_amdgcn_s_sleep(EXL3_POLL_SLEEP);
#pragma unroll
      for (int i = 0; i < EM; ++i)
#pragma unroll
        for (int j = 0; j < KC; ++j)
          if (pending & (1u << (i * KC + j)))
            v[i][j] = ld_agent_at(pr, po[i], (uint32_t)(k0 + j) * sstride);
#pragma unroll
      for (int i = 0; i < EM; ++i)
#pragma unroll
        for (int j = 0; j < KC; ++j)
          if ((pending & (1u << (i * KC + j))) && bits<uint32_t>(v[i][j]) != PARTIAL_EMPTY)
            pending &= ~(1u << (i * KC + j));
    }
    gave_up |= pending != 0;
#pragma unroll
    for (int i = 0; i < EM; ++i) {
      if (!live[i]) continue;
#pragma unroll
      for (int j = 0; j < KC; ++j) {
        if (j >= nk) break;
        if (!(pending & (1u << (i * KC + j))))
          st_agent(partial + (po[i] >> 2) + (size_t)(k0 + j) * stride, empty);
        s[i] = s[i] + v[i][j];
      }
    }
  }
#pragma unroll
  for (int i = 0; i < EM; ++i) {
    const int e = e0 + threadIdx.x + GEMV_THREADS * i;
    if (live[i]) zf[e] = h2f(f2h(s[i] + zf[e]));
  }
  return gave_up;
}

template <bool MULTI>
__device__ __forceinline__ bool gemv_splitk_last(float *zf, const GemvCfg &a, float *partial,
                                                 int nrows, const RowMap &rm, int ks, size_t out,
                                                 int col0) {
  const int E = nrows * 128;
  if (a.ksplit == 1) {
    for (int e = threadIdx.x; e < E; e += GEMV_THREADS) zf[e] = h2f(f2h(zf[e]));
    lds_barrier();
    return true;
  }
  const size_t stride = a.ptotal * out;
  if (ks != a.ksplit - 1) {
    if (a.drop_partials) return false;
    for (int e = threadIdx.x; e < E; e += GEMV_THREADS) {
      const int b = e >> 7, col = e & 127;
      float v = zf[e];
      if (v != v) v = bits<float>(0x7FC00000u);  // never PARTIAL_EMPTY
      st_agent(partial + ks * stride + (size_t)rm.prow(b) * out + col0 + col, v);
    }
    return false;
  }
  const __amdgpu_buffer_rsrc_t pr = buffer_of(partial);
  const uint32_t sstride = (uint32_t)(stride * 4);  // bytes between splits' planes
  // a thread's elements e = tid + 512 j.  MULTI (the rows-form launches,
  // many rows): the elements share each round of slot reads (2 elements x 8
  // splits, or 4 x 4), so the rows beyond 4 cost few extra round trips;
  // else (launches of few rows, whose registers set their occupancy) one
  // element at a time, 16 splits a round
  bool gave_up = false;
  if constexpr (MULTI) {
    if (E <= 2 * GEMV_THREADS)
      gave_up = splitk_sum<2, 8>(zf, pr, sstride, partial, stride, E, 0, ks, rm, out, col0,
                                 a.poll_max);
    else
      gave_up = splitk_sum<4, 4>(zf, pr, sstride, partial, stride, E, 0, ks, rm, out, col0,
                                 a.poll_max);
  } else {
    for (int e0 = 0; e0 < E; e0 += GEMV_THREADS)
      gave_up |= splitk_sum<1, 16>(zf, pr, sstride, partial, stride, E, e0, ks, rm, out, col0,
                                   a.poll_max);
  }
  if (gave_up) atomicOr(a.status, 1u);
  lds_barrier();
  return true;
}

// Stores two consecutive finished f16 values in the output dtype.
__device__ __forceinline__ void store_out2(void *p, size_t i, uint16_t y0, uint16_t y1, int dt) {
  if (dt == OUT_F16) {
    *reinterpret_cast<uint32_t *>((uint16_t *)p + i) = (uint32_t)y0 | ((uint32_t)y1 << 16);
  } else if (dt == OUT_BF16) {
    *reinterpret_cast<uint32_t *>((uint16_t *)p + i) =
        (uint32_t)f2bf(h2f(y0)) | ((uint32_t)f2bf(h2f(y1)) << 16);
  } else {
    float2 v;
    v.x = h2f(y0);
    v.y = h2f(y1);
    *reinterpret_cast<float2 *>((float *)p + i) = v;
  }
}

// The finish over zf[nrows][128] (f32 holding f16 values): rotation,
// * 1/sqrt(128), * svh, f16, output dtype (one wave per row, element i in
// lane i/2); or z itself when y is null.  sv holds svh of this lane's two
// columns (2 lane, 2 lane + 1), loaded at the start.
__device__ __forceinline__ void gemv_finish(float *zf, int ydt, void *y, uint16_t *zout, int nrows,
                                            const RowMap &rm, uint32_t sv, int col0) {
  if (y == nullptr) {
    for (int e = threadIdx.x; e < nrows * 128; e += GEMV_THREADS) {
      const int b = e >> 7, col = e & 127;
      zout[(size_t)rm.out_off(b) + col0 + col] = f2h(zf[e]);
    }
    return;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float sv0 = h2f((uint16_t)(sv & 0xFFFFu)), sv1 = h2f((uint16_t)(sv >> 16));
  for (int b = wave; b < nrows; b += GEMV_THREADS / 64) {
    float v0 = zf[b * 128 + 2 * lane], v1 = zf[b * 128 + 2 * lane + 1];
    had128_pair(v0, v1, lane);
    const float s0 = v0 * HAD_SCALE, s1 = v1 * HAD_SCALE;
    store_out2(y, (size_t)rm.out_off(b) + col0 + 2 * lane, f2h(s0 * sv0), f2h(s1 * sv1), ydt);
  }
}

// The finish into a residual: y as gemv_finish forms it (f16), then
// res += f32(y) over the group's 128 columns of each row (the old values in
// resv, loaded at the start: rows wave and wave + 8), and the group's
// sum of squares of the new res (a fixed pairwise order) into
// res_ssq[row][cg], for the RMSNorm prologue of the next GEMV.
__device__ __forceinline__ void gemv_finish_res(float *zf, float *res, float *res_ssq, size_t out,
                                                int nrows, const RowMap &rm, uint32_t sv, int cg,
                                                const float2 (&resv)[2]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float sv0 = h2f((uint16_t)(sv & 0xFFFFu)), sv1 = h2f((uint16_t)(sv >> 16));
  const int ng = (int)(out >> 7);
#pragma unroll
  for (int r2 = 0; r2 < 2; ++r2) {
    const int b = wave + r2 * (GEMV_THREADS / 64);
    if (b >= nrows) break;
    float v0 = zf[b * 128 + 2 * lane], v1 = zf[b * 128 + 2 * lane + 1];
    had128_pair(v0, v1, lane);
    const float s0 = v0 * HAD_SCALE, s1 = v1 * HAD_SCALE;
    const float y0 = h2f(f2h(s0 * sv0)), y1 = h2f(f2h(s1 * sv1));
    float *hp = res + (size_t)rm.out_off(b) + cg * 128 + 2 * lane;
    const float2 h = resv[r2];  // loaded at the workgroup's start
    float2 hn;
    hn.x = h.x + y0;
    hn.y = h.y + y1;
    *reinterpret_cast<float2 *>(hp) = hn;
    float ss = hn.x * hn.x + hn.y * hn.y;
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) ss += xor_lanes(ss, m);
    if (lane == 0) res_ssq[(size_t)rm.prow(b) * ng + cg] = ss;
  }
}

// One workgroup of the GEMV: expert `expert` of the weight with trellis
// words `twe` (that expert's) and out_tiles output tiles, nrows <= 16 rows
// (row map rm), column group cg, split ks.  PREP 0: the rows' items fit one
// prepare batch (nrows * tps / 8 <= PREP_ITEMS); else the rows form in PREP
// passes (nrows * tps / 8 <= PREP * PREP_GROUPS).
template <int K, int CB, bool MASKED, int PREP, int PRO = PRO_PLAIN>
__device__ __forceinline__ void gemv_wg(const uint32_t *twe, int out_tiles, const void *x,
                                        const GemvGeo &geo, const GemvCfg &a,
                                        const GemvWeight &W, int expert, int nrows,
                                        const RowMap &rm, int cg, int ks, char *smem,
                                        int rows_alloc, const uint16_t *psuh = nullptr) {
  // PREP 0: the rows' items fit one prepare batch (one item per wave);
  // else the rows form in PREP passes
  constexpr bool ONEB = PREP == 0;
  constexpr int NP = ONEB ? 1 : PREP;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = wave & 3, kp = wave >> 2;
  const size_t out = (size_t)out_tiles * 16;
  const int tps = geo.tps, in_tiles = geo.in_tiles;
  const int in = in_tiles * 16;
  const int tk0 = ks * tps;
  const int ntk = min(tps, in_tiles - tk0);  // a multiple of 8
  const int kr = tps * 16 + 8;
  uint16_t *xs = reinterpret_cast<uint16_t *>(smem);
  const int zrows = rows_alloc > 2 ? rows_alloc : 2;
  float *zp = reinterpret_cast<float *>(smem + (size_t)rows_alloc * kr * 2);  // [2][zrows][128]
  // mul1 at an integer rate: the MFMAs take h (the codebook value before its
  // affine step, chunk_pair_mul1_h), and z = a * acc + b * (sum of the
  // k-part's prepared activations) afterwards, from the 64-element sums
  // hsum[row][ntk / 4] that the prepare leaves
  constexpr bool FOLD = K > 0 && CB == CB_MUL1;
  float *hsum = zp + 2 * zrows * 128;
  const int nw = K > 0 ? 8 * K : a.nw;  // trellis dwords per tile
  const int g = lane >> 4, t = (lane >> 3) & 1, c = lane & 7;
  const size_t tn = (size_t)cg * 8 + 2 * q + t;
  const int part = ntk >> 1;  // k-tile rows per k-part, a multiple of 4
  const int kb = tk0 + kp * part;
  const int iters = part >> 2;

  // Loads of the workgroup's start, all in flight at once, in the order
  // their data is needed (vector loads complete in issue order): the first
  // prepare items' activations, the first step's weights, suh of those items,
  // the next NBUF - 1 steps' weights (steps past the last reload the last one:
  // in bounds and unused, so no branches and the waits stay exact), svh for
  // the finish.
  constexpr int KB = K > 0 ? K : 1;
  // steps in flight per wave: as many as a few registers allow
  constexpr int NBUF = K <= 0 ? 1 : 3;
  uint32_t bw[NBUF][KB];
  const gu32_t *wp = (const gu32_t *)(twe + ((size_t)(kb + g) * out_tiles + tn) * nw + c * K);
  const size_t wstep = (size_t)4 * out_tiles * nw;  // dwords per step
  const int nb = ntk >> 3, nitems = nrows * nb;
  // ONEB: one item (row, 128-block) per wave and batch; else every row's
  // items in one pass (gemv_rows_*)
  PrepRegs pr;
  RowsRegs<NP> rr;
  static_assert(PRO != PRO_ATTN || ONEB, "the attention prologue is for rows in one prepare batch");
  if constexpr (ONEB) {
    if constexpr (PRO != PRO_ATTN)
      gemv_prep_load_x(x, geo.xdt, geo.prepared, rm, nitems, nb, tk0, 0, wave, lane, pr);
  } else {
    gemv_rows_load_x(x, geo.xdt, geo.prepared, rm, nitems, nb, tk0, rr);
  }
  // psuh (a preloaded argument, plain prologue): suh's loads go out right
  // after x's, and no load waits for the argument segment
  const bool early = PRO == PRO_PLAIN && psuh != nullptr;
  if (early) {
    if constexpr (ONEB)
      gemv_prep_load_su(x, geo.prepared, psuh + (size_t)expert * in, nitems, nb, tk0, 0, wave,
                        lane, pr);
    else
      gemv_rows_load_su(x, geo.prepared, psuh + (size_t)expert * in, nitems, nb, tk0, rr);
  }
  if constexpr (K > 0) {
#pragma unroll
    for (int i = 0; i < K; ++i) bw[0][i] = wp[i];
  }
  // attention prologue: the first round of the wave's first item (x is the
  // attention's split slots)
  AttnLoads al;
  if constexpr (PRO == PRO_ATTN) {
    if (prep_item_live(0, 0, wave, nitems)) {
      const int row = wave / nb, blk = wave - row * nb;
      attn_load(attn_item((const float *)x, a, row, tk0 / 8 + blk), lane, al);
    }
  }
  // The loads above use preloaded arguments only (the attention prologue's
  // also its geometry from the argument segment).  W.suh comes from the
  // argument segment (a scalar load issued at entry); passing it through an
  // empty asm statement that also orders memory keeps the wait for that
  // scalar load after the loads above are issued.
  if (!early) {
    const uint16_t *suh0 = W.suh;
    asm volatile("" : "+s"(suh0)::"memory");
    const uint16_t *suh = suh0 + (size_t)expert * in;
    if constexpr (ONEB)
      gemv_prep_load_su(x, geo.prepared, suh, nitems, nb, tk0, 0, wave, lane, pr);
    else
      gemv_rows_load_su(x, geo.prepared, suh, nitems, nb, tk0, rr);
  }
  if constexpr (PRO == PRO_SWIGLU) {
    // SwiGLU prologue: x is gate; up from the argument segment, like suh
    const uint16_t *up = a.x2;
    asm volatile("" : "+s"(up)::"memory");
    if constexpr (ONEB)
      gemv_prep_load_up(up, rm, nitems, nb, tk0, 0, wave, lane, pr);
    else
      gemv_rows_load_up(up, rm, nitems, nb, tk0, rr);
  }
  if constexpr (PRO == PRO_RMSNORM) {
    static_assert(ONEB, "the RMSNorm prologue is for rows that fit one prepare batch");
    gemv_prep_load_norm(a, rm, nitems, nb, tk0, in, 0, wave, lane, pr);
  }
  if constexpr (K > 0) {
#pragma unroll
    for (int b = 1; b < NBUF; ++b) {
      const gu32_t *pb = wp + (size_t)min(b, iters - 1) * wstep;
#pragma unroll
      for (int i = 0; i < K; ++i) bw[b][i] = pb[i];
    }
  }
  // svh of this lane's two columns (read whether or not the finish runs: a
  // load without a branch around it)
  const uint16_t *svp =
      W.svh != nullptr ? W.svh + (size_t)expert * out + cg * 128 : W.suh + (size_t)expert * in;
  const uint32_t sv = ld_global_u32(svp + 2 * lane);
  // residual finish: the column group's residual pairs of the rows this wave
  // finishes (rows wave, wave + 8), loaded now so the finish does not wait
  // on them (without a residual, 8 bytes of the group's 128 svh values: a
  // load in bounds and without a branch)
  static_assert(GEMV_ROWS <= 2 * (GEMV_THREADS / 64), "two finish rows per wave");
  typedef float f2v_t __attribute__((ext_vector_type(2)));
  float2 resv[2];
#pragma unroll
  for (int r2 = 0; r2 < 2; ++r2) {
    const int b = min(wave + r2 * (GEMV_THREADS / 64), nrows - 1);
    const float *rp = a.res != nullptr
                          ? a.res + (size_t)rm.out_off(b) + cg * 128 + 2 * lane
                          : reinterpret_cast<const float *>(svp + 4 * (lane >> 1));
    const f2v_t v = *(const __attribute__((address_space(1))) f2v_t *)rp;
    resv[r2].x = v.x;
    resv[r2].y = v.y;
  }
  if constexpr (PRO == PRO_ATTN)
    gemv_prep_attn((const float *)x, a, nitems, nb, tk0, 0, wave, lane, al, pr);
  if constexpr (ONEB)
    gemv_prep_store<PRO>(geo.xdt, geo.prepared, nitems, nb, 0, wave, lane, xs, kr, pr,
                         FOLD ? hsum : nullptr, a.limit, in, a.eps);
  else
    gemv_rows_store<PRO, NP>(geo.xdt, geo.prepared, nitems, nb, xs, kr, rr,
                             FOLD ? hsum : nullptr, a.limit);
  lds_barrier();

  const int arow = min(lane & 15, nrows - 1);
  const uint16_t *xa = xs + arow * kr + (kp * part + g) * 16;
  f4_t acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (K > 0) {
    const int src = ((lane & ~7) | ((lane + 7) & 7)) << 2;
    auto step = [&](uint32_t(&b)[KB], int it) {
      uint32_t wd[K + 1];
#pragma unroll
      for (int i = 0; i < K; ++i) wd[i + 1] = b[i];
      wd[0] = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)b[K - 1]);
      {
        // the buffer is free once copied: its next step's load goes out
        // before this step's decode
        const gu32_t *pn = wp + (size_t)min(it + NBUF, iters - 1) * wstep;
#pragma unroll
        for (int i = 0; i < K; ++i) b[i] = pn[i];
      }
      const h8_t alo = *reinterpret_cast<const h8_t *>(xa + it * 64);
      const h8_t ahi = *reinterpret_cast<const h8_t *>(xa + it * 64 + 8);
      // one B operand at a time (pairs f, f+4, f+8, f+12: rows 0-7 or 8-15 of
      // column a or a+8), each consumed by its MFMA before the next is made
      static_for<4>([&](auto F) {
        constexpr int f = decltype(F)::value;
        constexpr int p0 = (f == 0) ? 0 : (f == 1) ? 2 : (f == 2) ? 1 : 3;
        uint32_t qv[4];
        static_for<4>([&](auto J) {
          constexpr int pq = p0 + 4 * decltype(J)::value;
          if constexpr (FOLD)
            qv[J] = chunk_pair_mul1_h<MASKED, K, pq>(wd, a.dec.mask);
          else
            qv[J] = chunk_pair_cw<K, CB, MASKED, pq>(wd, a.dec);
        });
        const h8_t bf = frag(qv[0], qv[1], qv[2], qv[3]);
        if constexpr (f == 0) acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bf, acc0, 0, 0, 0);
        if constexpr (f == 1) acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bf, acc1, 0, 0, 0);
        if constexpr (f == 2) acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bf, acc0, 0, 0, 0);
        if constexpr (f == 3) acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bf, acc1, 0, 0, 0);
      });
    };
    int it = 0;
    for (; it + NBUF <= iters; it += NBUF)
      static_for<NBUF>([&](auto B) { step(bw[decltype(B)::value], it + decltype(B)::value); });
    static_for<NBUF - 1>([&](auto B) {
      if (it + decltype(B)::value < iters) step(bw[decltype(B)::value], it + decltype(B)::value);
    });
  } else {
    // any even n: the wave stages its 4 k-tile rows x 2 tiles of dwords
    uint32_t *stage = reinterpret_cast<uint32_t *>(smem + (size_t)rows_alloc * kr * 2 +
                                                   (size_t)2 * zrows * 128 * 4 +
                                                   (size_t)rows_alloc * (tps / 4) * 4) +
                      wave * 512;
    const int n = 2 * nw;
    for (int it = 0; it < iters; ++it) {
      for (int i = lane; i < 8 * nw; i += 64) {
        const int seg = i / (2 * nw), off = i - seg * 2 * nw;
        stage[i] = twe[((size_t)(kb + 4 * it + seg) * out_tiles + cg * 8 + 2 * q) * nw + off];
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const uint32_t *mine = stage + (g * 2 + t) * nw;
      const h8_t alo = *reinterpret_cast<const h8_t *>(xa + it * 64);
      const h8_t ahi = *reinterpret_cast<const h8_t *>(xa + it * 64 + 8);
      uint32_t p[16];
#pragma unroll
      for (int pq = 0; pq < 16; ++pq) {
        const uint32_t cw = 32u * c + 2u * pq;
        p[pq] = decode_pair<CB>(tile_window(mine, n, cw), tile_window(mine, n, cw + 1u), a.dec);
      }
      gemv_mfma(p, alo, ahi, acc0, acc1);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }

  // C of a 16x16 MFMA: lane l holds rows 4(l/16)+i, column l%16.
  const int col = (2 * q + t) * 16 + c;
  float *zk = zp + kp * zrows * 128;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = 4 * g + i;
    if (m < nrows) {
      float z0 = acc0[i], z1 = acc1[i];
      if constexpr (FOLD) {
        // the k-part's 64-element sums of row m, in k order
        const float *hs = hsum + m * nb * 2 + kp * (part >> 2);
        float sx = 0.0f;
        for (int h = 0; h < (part >> 2); ++h) sx = sx + hs[h];
        const float bx = MUL1_B * sx;
        z0 = MUL1_A * z0 + bx;
        z1 = MUL1_A * z1 + bx;
      }
      zk[m * 128 + col] = z0;
      zk[m * 128 + col + 8] = z1;
    }
  }
  lds_barrier();
  float *zf = zp;
  for (int e = tid; e < nrows * 128; e += GEMV_THREADS) zf[e] = zp[e] + zp[zrows * 128 + e];
  lds_barrier();
  if (!gemv_splitk_last<!ONEB>(zf, a, W.partial, nrows, rm, ks, out, cg * 128)) {
    return;
  }
  if (a.res != nullptr)
    gemv_finish_res(zf, a.res, a.res_ssq, out, nrows, rm, sv, cg, resv);
  else
    gemv_finish(zf, a.ydt, W.y, W.zout, nrows, rm, sv, cg * 128);
}

// The weight of grid column group `gx` (weights' groups side by side) and
// its first and end column groups.
struct WeightSpan {
  int wi, c0, c1;
};
__device__ __forceinline__ WeightSpan gemv_weight_of(int gx, int cg1, int cg2, int cg3, int gend) {
  const int wi = (cg1 > 0 && gx >= cg1) + (cg2 > 0 && gx >= cg2) + (cg3 > 0 && gx >= cg3);
  const int c0 = wi == 0 ? 0 : wi == 1 ? cg1 : wi == 2 ? cg2 : cg3;
  const int n1 = wi == 0 ? cg1 : wi == 1 ? cg2 : wi == 2 ? cg3 : 0;
  return WeightSpan{wi, c0, n1 > 0 ? n1 : gend};
}

// Dense GEMV over up to four weights: the trellis pointers, the activations
// and the geometry are the first kernel arguments (preloaded SGPRs).
template <int K, int CB, bool MASKED, int PREP, int PRO>
__global__ __launch_bounds__(GEMV_THREADS) void gemv_kernel(
    const uint32_t *tw0, const uint32_t *tw1, const uint32_t *tw2, const uint32_t *tw3,
    const void *x, uint32_t g0, uint32_t g1, uint32_t g2, GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const GemvGeo geo = GemvGeo::unpack(g0, g1, g2);
  const WeightSpan ws = gemv_weight_of(blockIdx.x, geo.cg1, geo.cg2, geo.cg3, geo.cgend);
  const uint32_t *tw = ws.wi == 0 ? tw0 : ws.wi == 1 ? tw1 : ws.wi == 2 ? tw2 : tw3;
  const int out_tiles = 8 * (ws.c1 - ws.c0);
  const RowMap rm{nullptr, geo.in_tiles * 16, out_tiles * 16};
  // launches of fewer than four weights carry suh pointers in the unused
  // trellis arguments (gemv_multi puts them there): one weight tw1; two tw2,
  // tw3; three tw3 for weight 0
  const int nwt = 1 + (geo.cg1 > 0) + (geo.cg2 > 0) + (geo.cg3 > 0);
  const uint16_t *psuh =
      nwt == 1   ? (const uint16_t *)tw1
      : nwt == 2 ? (const uint16_t *)(ws.wi == 0 ? tw2 : tw3)
      : nwt == 3 && ws.wi == 0 ? (const uint16_t *)tw3
                               : nullptr;
  // stacked prepared rows: weight wi's set follows the sets of weights < wi
  const void *xw = geo.stacked ? (const void *)((const uint16_t *)x + (size_t)ws.wi * geo.rows *
                                                                          geo.in_tiles * 16)
                               : x;
  gemv_wg<K, CB, MASKED, PREP, PRO>(tw, out_tiles, xw, geo, a.c, a.w[ws.wi], 0, geo.rows, rm,
                               blockIdx.x - ws.c0, blockIdx.y, smem + 256, geo.rows, psuh);
}

// ===================================================================== GEMM
//
// Workgroup tile 256 rows x 128 columns (one Hadamard block of the output),
// stages of 64 k (four k-tile rows).  The operands meet in LDS in MFMA
// layout; within a stage, MFMA step kk contracts k = 32 h + 8 kk + e over
// lane half h and element e, the same order for both operands.  The MFMAs
// take the weights as their first operand, so the accumulators hold z^T: a
// lane holds one row of z and 16 of its columns.  That is the operand layout
// of a second MFMA, which applies the finish's Hadamard stages on column
// bits 0-4 (H_32, +-1 entries: exact products, f32 sums) to f16(z); the
// 128-column block spans two waves, so stages 5 and 6 go through LDS, then
// * 1/sqrt(128) * svh.  Each decoded weight serves 256 rows.  Tiles of 128
// columns keep the grid a multiple of the 256 CUs at the Qwen3-8B shapes
// (M = 2048: 256 tiles for 4096 outputs, 768 for 12288).

constexpr int GM_BM = 256, GM_BN = 128, GM_BK = 64;
constexpr int GM_LD = GM_BK + 8;         // halfs per LDS row of A / column of B^T
constexpr int GM_BTILE = GM_BN * GM_LD;  // halfs of B^T per stage buffer
// finish exchange: 64 rows of the 128 columns after the H_32 step (f32),
// rows padded to 132 floats (33 KiB)
constexpr int GM_FLD = 132;

// Pair place in fragment order: fragment f (0: column a, rows 0-7; 1: column
// a+8, rows 0-7; 2: column a, rows 8-15; 3: column a+8, rows 8-15) holds
// pairs p0(f) + 4J, J = 0..3.
__host__ __device__ constexpr int gm_pair(int f, int J) {
  return ((f == 0) ? 0 : (f == 1) ? 2 : (f == 2) ? 1 : 3) + 4 * J;
}

// Word sets of the decode waves' packed-word ring: the words of stage x are
// loaded gm_wl stages ahead (a few registers each, so deep: the history
// exchange of stage x, two stages before its use, then never waits on HBM
// latency).
template <int K>
constexpr int gm_wl() { return K <= 4 ? 6 : 3; }  // word sets (divides the 6-stage trip)

// The end of a GEMM tile, by all THREADS threads of the workgroup (mw: this
// wave holds accumulators, wave tile (wm, wc); the others take part in the
// barriers and the butterflies).  Split k: the f32 sums go to their plane.
// Else z^T is stored (y null) or finished: the Hadamard-128 on the
// accumulators, * 1/sqrt(128) * svh, the output dtype.
template <int THREADS>
__device__ __forceinline__ void gemm_tile_end(f16v_t (&acc)[2][2], uint16_t *lds, bool mw, int wm,
                                              int wc, int m0, int cg, int M, size_t out, int S,
                                              int ks, const uint16_t *__restrict__ svh,
                                              void *__restrict__ y, int ydt,
                                              uint16_t *__restrict__ zout,
                                              float *__restrict__ kpart,
                                              const uint32_t *__restrict__ rowmap = nullptr) {
  // output row of tile row m (< M): m, or rowmap[m] (a routed item's slots)
  auto orow = [&](int m) -> size_t { return rowmap ? (size_t)rowmap[m] : (size_t)m; };
  // acc[i][j] = z^T for columns 64 wc + 32 j .. and rows 64 wm + 32 i .. of
  // the tile: lane l holds row (l & 31), register r column
  // 8 (r / 4) + 4 (l / 32) + r % 4 (the 32 x 32 MFMA result layout).
  const int lane = threadIdx.x & 63, tid = threadIdx.x;
  const int rb = m0 + 64 * wm + (lane & 31);
  if (S > 1) {
    if (!mw) return;
    // split-K: this split's sums of rows < M go to its plane of
    // kpart [S][M][out] (f32, row-major; four consecutive columns per
    // store); gemm_splitk_finish_kernel adds the planes and finishes
    float *plane = kpart + (size_t)ks * M * out;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (rb + 32 * i >= M) continue;
      float *pr = plane + (size_t)(rb + 32 * i) * out + cg * 128 + 64 * wc + 4 * (lane >> 5);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const float4 v = make_float4(acc[i][j][4 * q4], acc[i][j][4 * q4 + 1],
                                       acc[i][j][4 * q4 + 2], acc[i][j][4 * q4 + 3]);
          *reinterpret_cast<float4 *>(pr + 32 * j + 8 * q4) = v;
        }
    }
    return;
  }
  if (y == nullptr) {
    if (!mw) return;
    static_for<2>([&](auto I) {
      constexpr int i = decltype(I)::value;
      if (rb + 32 * i < M) {
        uint16_t *zr = zout + orow(rb + 32 * i) * out + cg * 128 + 64 * wc + 4 * (lane >> 5);
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) zr[32 * j + 8 * (r >> 2) + (r & 3)] = f2h(acc[i][j][r]);
      }
    });
    return;
  }
  // H_32 as the second operand: element e of fragment kk pairs with column
  // 16 kk + 8 (e / 4) + 4 (l / 32) + e % 4 of a 32-column block (the
  // registers 8 kk + e above), output column (l & 31).
  h8_t hb[2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int nl = 16 * kk + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
      hb[kk][e] = (__builtin_popcount(nl & lane & 31) & 1) ? -1.0f16 : 1.0f16;
    }
  // The stage buffers are free now: the H_32 outputs go through them as f32
  // [64 rows][GM_FLD], in four passes of 64 rows (row block i of the waves
  // with wm / 2 == g), so the butterflies across the four 32-column blocks
  // (two waves) can pair them.
  float *fx = reinterpret_cast<float *>(lds);
  static_for<4>([&](auto P) {
    constexpr int i = decltype(P)::value & 1, g = decltype(P)::value >> 1;
    lds_barrier();  // the previous use of the buffers is done
    if (mw && (wm >> 1) == g) {
      // D2_j = f16(z block j) H_32: lane l holds output column (l & 31) of
      // block 2 wc + j, register r row 8 (r / 4) + 4 (l / 32) + r % 4 of the
      // wave's rows 32 i ..
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        h8_t a0, a1;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          a0[e] = bits<_Float16>(f2h(acc[i][j][e]));
          a1[e] = bits<_Float16>(f2h(acc[i][j][8 + e]));
        }
        f16v_t zero = {};
        f16v_t d2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, hb[0], zero, 0, 0, 0);
        d2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, hb[1], d2, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = 32 * (wm & 1) + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          fx[row * GM_FLD + 32 * (2 * wc + j) + (lane & 31)] = d2[r];
        }
      }
    }
    lds_barrier();
    // butterflies on column bits 5 and 6, in that order (lo + hi, lo - hi),
    // then * 1/sqrt(128) * svh
    for (int e = tid; e < 64 * 32; e += THREADS) {
      const int row = e >> 5, cl = e & 31;
      const float *fr = fx + row * GM_FLD + cl;
      const float t0 = fr[0] + fr[32], t1 = fr[0] - fr[32];
      const float t2 = fr[64] + fr[96], t3 = fr[64] - fr[96];
      const float u[4] = {t0 + t2, t1 + t3, t0 - t2, t1 - t3};
      const int m = m0 + 64 * (2 * g + (row >> 5)) + 32 * i + (row & 31);
      if (m < M) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          store_out(y, orow(m) * out + cg * 128 + 32 * j + cl,
                    f2h((u[j] * HAD_SCALE) * h2f(svh[cg * 128 + 32 * j + cl])), ydt);
      }
    }
  });
}

// ================================================ GEMM, specialised waves
//
// gemm_ws_kernel: the tile above (256 rows x 128 columns, 64-k stages), with
// the work split by wave.  Waves 0-7 (the MFMA
// waves, wave tile 64 x 64) issue the MFMAs and bring the activations into
// LDS with direct global-to-LDS loads (no registers; three A buffers, the
// loads of stage x issued during stage x - 2).  Waves 8-15 (the decode
// waves) decode the next stage's packed words into the other B buffer: the
// 256 chunks of a stage, half a chunk per thread (waves 8-11 rows 0-7 of
// each chunk's columns, waves 12-15 rows 8-15).  Four waves per SIMD: the
// decode's VALU work issues beside the other waves' MFMAs.  One barrier per
// stage.
//
// A buffer (unpadded, 128 bytes a row): 16-byte piece q of row R sits at
// piece place q ^ ((R / 2) % 8), so a fragment read (rows R0 .. R0 + 15 of
// one piece, R0 % 32 == 0) touches 16 distinct 16-byte bank groups, and
// a load instruction fills 1 KiB (8 rows) contiguously.
constexpr int GW_THREADS = 1024;
constexpr int GW_BBUF = GM_BTILE * 2;         // bytes of a B buffer ([128][72] halfs)
constexpr int GW_ABUF = GM_BM * GM_BK * 2;    // bytes of an A buffer
constexpr int GW_A0 = 2 * GW_BBUF;            // the A buffers follow the two B buffers
constexpr int GW_LDS_BYTES = GW_A0 + 3 * GW_ABUF;  // 132 KiB
static_assert(64 * GM_FLD * 4 <= GW_A0, "finish exchange reaches the A buffers");

// 16 bytes per lane from global memory (base + voff) straight into LDS at
// address lds + 16 * lane.  M0 carries the LDS address (the compiler uses
// M0 for nothing in these kernels); an LDS DMA that reads M0 right after it
// is written needs wait states between them (the compiler's hazard check
// does not see into asm), hence the s_nop.  vmcnt counts the load until its
// bytes are in LDS.
__device__ __forceinline__ void lds_dma16(const void *base, uint32_t voff, uint32_t lds) {
  // M0 is not named as clobbered: the AMDGPU backend reserves it and ignores
  // (with a warning) such a clobber; no other instruction in the kernels that
  // call this reads M0 (their gfx950 code sets it only here).
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 1\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds),
               "v"(voff), "s"(base)
               : "memory");
}

// The MFMA waves' main loop.  ax[kk]: byte address of the wave's A fragment
// kk in A buffer 0 (row block i adds 4 KiB, buffer a adds a * GW_ABUF);
// brd: half index of its B fragment 0 in B buffer 0; voff[u]: its
// activation pieces (rows 32 w + 8 u + l / 8); dma0: LDS address of its
// first load in A buffer 0.
__device__ __forceinline__ void gw_mfma_main(f16v_t (&acc)[2][2], uint16_t *lds, const char *xpb,
                                             const uint32_t (&voff)[4], uint32_t dma0,
                                             const uint32_t (&ax)[4], int brd, int NS) {
  const char *L = reinterpret_cast<const char *>(lds);
  h8_t af[2][2], bf[2][2];
  auto dma = [&](int st, int a, int u) {
    lds_dma16(xpb + (size_t)st * (GM_BK * 2), voff[u], dma0 + a * GW_ABUF + u * 1024);
  };
  auto read_af = [&](int q, int a, int kk, int i) {
    af[q][i] = *reinterpret_cast<const h8_t *>(L + ax[kk] + a * GW_ABUF + i * 32 * 128);
  };
  auto read_bf = [&](int q, int b, int kk, int j) {
    bf[q][j] = *reinterpret_cast<const h8_t *>(lds + b * GM_BTILE + brd + j * 32 * GM_LD + 8 * kk);
  };
  auto stage = [&](auto PH, int st) {
    constexpr int ph = decltype(PH)::value;
    constexpr int a = ph % 3, b = ph & 1;                  // this stage's buffers
    constexpr int an = (ph + 1) % 3, bn = (ph + 1) & 1;    // the next stage's
    constexpr int a2 = (ph + 2) % 3;                       // stage st + 2's A buffer
    const int st2 = min(st + 2, NS - 1);  // past the end: a free buffer, drained below
    static_for<16>([&](auto SL) {
      constexpr int s = decltype(SL)::value;
      constexpr int kk = s >> 2, i = (s >> 1) & 1, j = s & 1;
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[kk & 1][j], af[kk & 1][i], acc[i][j],
                                                          0, 0, 0);
      if constexpr (kk < 2) {
        constexpr int qn = (kk + 1) & 1;
        if constexpr ((s & 3) < 2) read_af(qn, a, kk + 1, s & 1);
        if constexpr ((s & 3) >= 2) read_bf(qn, b, kk + 1, s & 1);
      }
      if constexpr (s == 8) {
        read_af(1, a, 3, 0);
        read_af(1, a, 3, 1);
      }
      if constexpr (s == 9) {
        read_bf(1, b, 3, 0);
        read_bf(1, b, 3, 1);
      }
      if constexpr (s < 4) dma(st2, a2, s);
      // stage st + 1's activations (loaded during stage st - 1) and B
      // (decoded during stage st) are in, this stage's buffers are read
      if constexpr (s == 10) asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if constexpr (s == 12) {
        read_af(0, an, 0, 0);
        read_af(0, an, 0, 1);
      }
      if constexpr (s == 13) {
        read_bf(0, bn, 0, 0);
        read_bf(0, bn, 0, 1);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  // prologue: stages 0 and 1 in flight, wait for stage 0 (and its B)
  for (int u = 0; u < 4; ++u) dma(0, 0, u);
  for (int u = 0; u < 4; ++u) dma(1, 1, u);
  asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  read_af(0, 0, 0, 0);
  read_af(0, 0, 0, 1);
  read_bf(0, 0, 0, 0);
  read_bf(0, 0, 0, 1);
  int st = 0;
  for (; st + 6 <= NS; st += 6) {
    static_for<6>([&](auto PH) { stage(PH, st + decltype(PH)::value); });
  }
  if (st < NS) {  // NS is even: 2 or 4 stages left
    stage(std::integral_constant<int, 0>{}, st);
    stage(std::integral_constant<int, 1>{}, st + 1);
    if (st + 2 < NS) {
      stage(std::integral_constant<int, 2>{}, st + 2);
      stage(std::integral_constant<int, 3>{}, st + 3);
    }
  }
  // no load may still write this workgroup's LDS when it ends
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// The decode waves' main loop: the thread decodes fragments 2 HALF and
// 2 HALF + 1 of chunk c of output tile tnl of k-tile row tkl of every stage
// (twc: its words in stage 0), stage st + 1 during stage st, into B buffer
// (st + 1) % 2 at bst.
template <int K, int CB, bool MASKED, int HALF>
__device__ __forceinline__ void gw_decode_main(uint16_t *lds, const uint32_t *twc, size_t wstage,
                                               int src, int bst, int NS, CbRow mask) {
  constexpr int WL = gm_wl<K>();
  uint32_t wn[WL][K];
  uint32_t hist[2];
  auto load_w = [&](auto S, int st) {
    constexpr int q = decltype(S)::value;
    const uint32_t *p = twc + (size_t)min(st, NS - 1) * wstage;
#pragma unroll
    for (int j = 0; j < K; ++j) wn[q][j] = p[j];
  };
  auto bperm = [&](auto S, auto HS) {
    constexpr int q = decltype(S)::value, hq = decltype(HS)::value;
    hist[hq] = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)wn[q][K - 1]);
  };
  // the thread's half of the chunk of word set S (history HS) into B
  // buffer b: two fragments
  auto decode = [&](auto S, auto HS, int b) {
    constexpr int q = decltype(S)::value, hq = decltype(HS)::value;
    uint32_t wd[K + 1];
    wd[0] = hist[hq];
#pragma unroll
    for (int j = 0; j < K; ++j) wd[j + 1] = wn[q][j];
    static_for<2>([&](auto F) {
      constexpr int f = 2 * HALF + decltype(F)::value;
      uint32_t v[4];
      static_for<4>([&](auto J) {
        v[J] = chunk_pair_cw<K, CB, MASKED, gm_pair(f, decltype(J)::value)>(wd, mask);
      });
      const u4_t u = {v[0], v[1], v[2], v[3]};
      *reinterpret_cast<u4_t *>(lds + b * GM_BTILE + bst + 8 * (f & 1) * GM_LD + 8 * (f >> 1)) = u;
    });
  };
  using IC0 = std::integral_constant<int, 0>;
  using IC1 = std::integral_constant<int, 1>;
  auto stage = [&](auto PH, int st) {
    constexpr int ph = decltype(PH)::value;
    using W0 = std::integral_constant<int, ph % WL>;
    using W1 = std::integral_constant<int, (ph + 1) % WL>;
    using W2 = std::integral_constant<int, (ph + 2) % WL>;
    using H1 = std::integral_constant<int, (ph + 1) & 1>;
    using H2 = std::integral_constant<int, ph & 1>;
    if (st + 1 < NS) decode(W1{}, H1{}, (ph + 1) & 1);
    load_w(W0{}, st + WL);
    bperm(W2{}, H2{});
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };
  static_for<WL>([&](auto W) { load_w(W, decltype(W)::value); });
  bperm(IC0{}, IC0{});
  decode(IC0{}, IC0{}, 0);
  bperm(IC1{}, IC1{});
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  int st = 0;
  for (; st + 6 <= NS; st += 6) {
    static_for<6>([&](auto PH) { stage(PH, st + decltype(PH)::value); });
  }
  if (st < NS) {
    stage(std::integral_constant<int, 0>{}, st);
    stage(std::integral_constant<int, 1>{}, st + 1);
    if (st + 2 < NS) {
      stage(std::integral_constant<int, 2>{}, st + 2);
      stage(std::integral_constant<int, 3>{}, st + 3);
    }
  }
}

// ------------------------------------------------ half-integer rates
//
// At n = 8 FR halfwords a tile (FR odd: K = FR / 2 = 1.5, 2.5, exllamav3's
// half-integer rates; turboexl3_ds41/src/bank/frac.zig:1-21), chunk c of a
// tile (codewords 32 c .. 32 c + 31) is stream halfwords c FR .. c FR + FR - 1
// (bitEnd(32 c) = 2 n c: a halfword boundary, not a dword one).  A decode
// thread loads the LW = NB + 1 dwords holding that chunk and the halfword
// before it (the tile's last for c = 0: the ring wraps), starting at dword b;
// one v_alignbit_b32 per dword by sh (16 when that history halfword is the
// low half of dword b, else 0 with b one dword earlier) leaves NB dwords
// [history | chunk], MSB first, in which codeword i's window ends at bit
// 16 + floor((i + 1) FR / 2): compile-time positions, as chunk_cw's.
template <int FR>
constexpr int gf_nb() {
  return (FR + 1) / 2;
}

template <int FR, int I>
__device__ __forceinline__ uint32_t chunk_cw_frac(const uint32_t (&w)[gf_nb<FR>()]) {
  constexpr int E = 16 + ((I + 1) * FR) / 2;
  constexpr int J0 = (E - 16) >> 5, J1 = (E - 1) >> 5;
  static_assert(J1 < gf_nb<FR>(), "window outside the chunk buffer");
  if constexpr (J0 == J1)
    return __builtin_amdgcn_ubfe(w[J0], 31 - ((E - 1) & 31), 16);
  else
    return __builtin_amdgcn_alignbit(w[J0], w[J1], 31 - ((E - 1) & 31)) & 0xFFFFu;
}

// The decode waves' main loop at a half-integer rate: gw_decode_main's
// schedule and barriers (stage st + 1 decoded during stage st into B buffer
// (st + 1) % 2) with each thread's chunk loaded whole (off: its LW dword
// offsets in the tile, twt: its tile in stage 0).
template <int FR, int CB, bool MASKED, int HALF>
__device__ __forceinline__ void gw_decode_frac(uint16_t *lds, const uint32_t *twt, size_t wstage,
                                               const int (&off)[gf_nb<FR>() + 1], uint32_t sh,
                                               int bst, int NS, CbRow mask) {
  constexpr int NB = gf_nb<FR>(), LW = NB + 1;
  constexpr int WL = 6;
  uint32_t wn[WL][LW];
  auto load_w = [&](auto S, int st) {
    constexpr int q = decltype(S)::value;
    const uint32_t *p = twt + (size_t)min(st, NS - 1) * wstage;
#pragma unroll
    for (int j = 0; j < LW; ++j) wn[q][j] = p[off[j]];
  };
  auto decode = [&](auto S, int b) {
    constexpr int q = decltype(S)::value;
    uint32_t wd[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) wd[j] = __builtin_amdgcn_alignbit(wn[q][j], wn[q][j + 1], sh);
    static_for<2>([&](auto F) {
      constexpr int f = 2 * HALF + decltype(F)::value;
      uint32_t v[4];
      static_for<4>([&](auto J) {
        constexpr int pr = gm_pair(f, decltype(J)::value);
        v[J] = decode_pair_cw<CB, MASKED>(chunk_cw_frac<FR, 2 * pr>(wd),
                                          chunk_cw_frac<FR, 2 * pr + 1>(wd), mask);
      });
      const u4_t u = {v[0], v[1], v[2], v[3]};
      *reinterpret_cast<u4_t *>(lds + b * GM_BTILE + bst + 8 * (f & 1) * GM_LD + 8 * (f >> 1)) = u;
    });
  };
  auto stage = [&](auto PH, int st) {
    constexpr int ph = decltype(PH)::value;
    using W0 = std::integral_constant<int, ph % WL>;
    using W1 = std::integral_constant<int, (ph + 1) % WL>;
    if (st + 1 < NS) decode(W1{}, (ph + 1) & 1);
    load_w(W0{}, st + WL);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };
  static_for<WL>([&](auto W) { load_w(W, decltype(W)::value); });
  decode(std::integral_constant<int, 0>{}, 0);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  int st = 0;
  for (; st + 6 <= NS; st += 6) {
    static_for<6>([&](auto PH) { stage(PH, st + decltype(PH)::value); });
  }
  if (st < NS) {
    stage(std::integral_constant<int, 0>{}, st);
    stage(std::integral_constant<int, 1>{}, st + 1);
    if (st + 2 < NS) {
      stage(std::integral_constant<int, 2>{}, st + 2);
      stage(std::integral_constant<int, 3>{}, st + 3);
    }
  }
}

// FR = 0: an integer rate K; FR odd: the half-integer rate n = 8 FR (K unused).
template <int K, int CB, bool MASKED, int FR = 0>
__global__ __launch_bounds__(GW_THREADS, 1) void gemm_ws_kernel(
    const uint32_t *__restrict__ tw, const uint16_t *__restrict__ xp,
    const uint16_t *__restrict__ svh, void *__restrict__ y, int ydt, uint16_t *__restrict__ zout,
    int M, int in_tiles, int out_tiles, CbRow mask, float *__restrict__ kpart) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[GW_LDS_BYTES / 2];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool mw = wave < 8;
  const int wm = (wave & 7) >> 1, wc = wave & 1;
  // Workgroup n runs on XCD n % 8 (the dispatcher's round robin); taking the
  // row block as n % (row blocks) gives each XCD a few row blocks of the
  // activations to keep in its L2.  (Only the speed depends on this.)
  const int mblocks = gridDim.y;
  const int lin = blockIdx.x + gridDim.x * blockIdx.y;
  const int cg = lin / mblocks;
  const int m0 = (lin % mblocks) * GM_BM;
  const int in = in_tiles * 16;
  const size_t out = (size_t)out_tiles * 16;
  constexpr int NW = FR > 0 ? 4 * FR : 8 * K;
  const int NS = in_tiles / 4;
  const int S = gridDim.z, ks = blockIdx.z;
  const int P = NS / 2;
  const int st0 = 2 * (P * ks / S), st1 = 2 * (P * (ks + 1) / S);

  f16v_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  if (mw) {
    // activation loads: rows 32 w + 8 u + l / 8 of the tile, the piece
    // (l % 8) ^ ((row / 2) % 8) of them (rows past M read row M - 1)
    uint32_t voff[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int R = 32 * wave + 8 * u + (lane >> 3);
      const int q = (lane & 7) ^ ((R >> 1) & 7);
      voff[u] = (uint32_t)(((size_t)min(m0 + R, M - 1) * in + 8 * q) * 2);
    }
    const uint32_t dma0 =
        (uint32_t)(uintptr_t)lds + GW_A0 + (uint32_t)(32 * wave) * 128;  // 4 KiB per wave
    // fragment reads: A row 64 wm + 32 i + (l & 31), k 32 h + 8 kk (piece
    // 4 h + kk); B column 64 wc + 32 j + (l & 31)
    const int h = lane >> 5;
    uint32_t ax[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      ax[kk] = GW_A0 + (64 * wm + (lane & 31)) * 128 + 16 * ((4 * h + kk) ^ ((lane >> 1) & 7));
    const int brd = (64 * wc + (lane & 31)) * GM_LD + 32 * h;
    gw_mfma_main(acc, lds, reinterpret_cast<const char *>(xp + (size_t)st0 * GM_BK), voff, dma0,
                 ax, brd, st1 - st0);
  } else {
    // chunk c of output tile tnl of k-tile row tkl (threads dt and dt + 256
    // take the same chunk); the 8 chunks of a tile sit in 8 consecutive lanes
    const int dt = (tid - 512) & 255;
    const int tkl = dt >> 6, tnl = (dt >> 3) & 7, c = dt & 7;
    const size_t wstage = (size_t)4 * out_tiles * NW;
    const int bst = (tnl * 16 + c) * GM_LD + tkl * 16;
    if constexpr (FR > 0) {
      // the chunk's history halfword hs (stream order: halfword s is the high
      // half of dword s / 2 when s is even, the low half when odd)
      constexpr int LW = gf_nb<FR>() + 1;
      const int hs = (c * FR - 1 + 8 * FR) % (8 * FR);
      const bool low = (hs & 1) != 0;
      const int b0 = (hs >> 1) - (low ? 0 : 1);
      int off[LW];
#pragma unroll
      for (int j = 0; j < LW; ++j) off[j] = (b0 + j) % NW;
      const uint32_t *twt =
          tw + ((size_t)tkl * out_tiles + cg * 8 + tnl) * NW + (size_t)st0 * wstage;
      if (wave < 12)
        gw_decode_frac<FR, CB, MASKED, 0>(lds, twt, wstage, off, low ? 16u : 0u, bst, st1 - st0,
                                          mask);
      else
        gw_decode_frac<FR, CB, MASKED, 1>(lds, twt, wstage, off, low ? 16u : 0u, bst, st1 - st0,
                                          mask);
    } else {
      const uint32_t *twc = tw + ((size_t)tkl * out_tiles + cg * 8 + tnl) * NW + c * K;
      const int src = ((lane & ~7) | ((lane + 7) & 7)) << 2;
      twc += (size_t)st0 * wstage;
      if (wave < 12)
        gw_decode_main<K, CB, MASKED, 0>(lds, twc, wstage, src, bst, st1 - st0, mask);
      else
        gw_decode_main<K, CB, MASKED, 1>(lds, twc, wstage, src, bst, st1 - st0, mask);
    }
  }
  gemm_tile_end<GW_THREADS>(acc, lds, mw, wm, wc, m0, cg, M, out, S, ks, svh, y, ydt, zout,
                            kpart);
}

// ==================================================== grouped MoE GEMV

// A work item of the routed MoE: up to GEMV_ROWS slots of one expert.
struct MoeItem {
  uint32_t expert, start, count, pad;
};

// Work items of up to 4 slots over splits of up to 256 k-tiles: an item's
// rows fill at most the rows form's passes (4 rows x 32 blocks), and a
// workgroup streams up to four times the weights of a dense split for its
// fixed costs (row gathering, prepare, split-K hand-off).  DeepSeek-V3's
// gate+up at 16 rows: 2 splits of 28 blocks over items of up to 4 slots,
// 9 % faster a layer than 4 splits of up to 16 blocks over items of up to 8
// (an expert's slots beyond 4 form another item that reads its weights
// again: at 64 rows, where the shared expert holds every row, 2-5 % faster).
constexpr int MOE_ITEM_ROWS = 4;
constexpr int MOE_TPS_MAX = 256;
static_assert(MOE_ITEM_ROWS * (MOE_TPS_MAX / 8) <= PREP_PASSES * PREP_GROUPS,
              "a work item's prepare exceeds the rows form");
// One-row items (no item list) take splits of up to 160 k-tiles: their rows
// form is one pass, and one row of LDS keeps three workgroups a CU.
constexpr int MOE_DIRECT_TPS_MAX = 160;
static_assert(MOE_DIRECT_TPS_MAX / 8 <= PREP_GROUPS, "a one-row item's prepare exceeds one pass");

// Grouped GEMV: blockIdx.z = work item, blockIdx.x = column group over the
// launch's weights (gate and up side by side, or down).  Raw inputs are rows
// slot / topk of x; prepared inputs are rows slot.  Without an item list
// (items null: one row's slots) item z is slot z alone, its expert
// sorted[z] (the routes; with a.c.routes_k = k > 0 slot k is the shared
// expert), skipped when not below a.c.experts.  PRO_SWIGLU (down): x is
// the slots' gate rows and a.c.x2 their up rows (topk 1: row slot), the
// mid step's SwiGLU and rotation formed in the prepare.
template <int K, int CB, bool MASKED, int PRO>
__global__ __launch_bounds__(GEMV_THREADS) void moe_gemv_kernel(
    const uint32_t *tw0, const uint32_t *tw1, const void *x, uint32_t g0, uint32_t g1,
    uint32_t g2, int topk, const uint32_t *__restrict__ sorted,
    const MoeItem *__restrict__ items, const uint32_t *__restrict__ n_items, GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int item = blockIdx.z;
  MoeItem it;
  if (items != nullptr) {
    if ((uint32_t)item >= *n_items) return;
    it = items[item];
  } else {
    if ((size_t)item >= a.c.ptotal) return;
    // uniform across the workgroup; readfirstlane keeps it in a scalar
    // register for the address arithmetic that follows
    const uint32_t e = (uint32_t)__builtin_amdgcn_readfirstlane(
        a.c.routes_k > 0 && item >= a.c.routes_k ? a.c.shared_expert : (int)sorted[item]);
    if (e >= (uint32_t)a.c.experts) return;
    it = MoeItem{e, (uint32_t)item, 1u, 0u};
  }
  const GemvGeo geo = GemvGeo::unpack(g0, g1, g2);
  const WeightSpan ws = gemv_weight_of(blockIdx.x, geo.cg1, 0, 0, geo.cgend);
  const uint32_t *tw = ws.wi == 0 ? tw0 : tw1;
  const int out_tiles = 8 * (ws.c1 - ws.c0);
  const GemvWeight &W = a.w[ws.wi];
  GemvRow *ri = reinterpret_cast<GemvRow *>(smem);
  if (threadIdx.x < GEMV_ROWS) {
    const int b = min((int)threadIdx.x, (int)it.count - 1);
    const int slot = items != nullptr ? (int)sorted[it.start + b] : item;
    const int in = geo.in_tiles * 16, out = out_tiles * 16;
    ri[threadIdx.x] = GemvRow{(geo.prepared ? slot : slot / topk) * in, slot * out, slot, 0};
  }
  lds_barrier();
  const RowMap rm{ri, 0, 0};
  // the prepare form the item's rows need (most items hold a few slots: one
  // batch or one pass instead of the passes 16 rows take)
  // the shared expert (an index past the bank's) reads its own linear
  const bool sh = (int)it.expert == a.c.shared_expert;
  GemvWeight Wx = W;
  if (sh) {
    Wx.suh = W.sh_suh;
    Wx.svh = W.sh_svh;
  }
  const uint32_t *twe = sh ? W.sh_tw : tw + (size_t)it.expert * W.expert_words;
  auto run = [&](auto P) {
    gemv_wg<K, CB, MASKED, decltype(P)::value, PRO>(twe, out_tiles, x, geo, a.c, Wx,
                                               sh ? 0 : (int)it.expert, (int)it.count, rm,
                                               blockIdx.x - ws.c0, blockIdx.y, smem + 256,
                                               items != nullptr ? MOE_ITEM_ROWS : 1);
  };
  const int items_n = (int)it.count * (geo.tps / 8);
  if (items_n <= PREP_ITEMS)
    run(std::integral_constant<int, 0>{});
  else if (items_n <= PREP_GROUPS)
    run(std::integral_constant<int, 1>{});
  else if (items_n <= 2 * PREP_GROUPS)
    run(std::integral_constant<int, 2>{});
  else
    run(std::integral_constant<int, PREP_PASSES>{});
}

// Grouped GEMM over routed work items (prefill-sized expert batches): the
// specialised-wave GEMM with workgroup (column group cg, item) taking item
// `blockIdx.y` = (expert e, up to 256 slots sorted[start ..]): activation
// rows gathered by slot (x holds one prepared row per slot), expert e's
// trellis words and svh, outputs scattered to the slots' rows.  No split k.
struct GemmGroup {
  const uint32_t *sorted;
  const MoeItem *items;
  const uint32_t *n_items;
  size_t expert_words;  // trellis dwords per expert
  // groups > 0: a grouped linear's items, formed from blockIdx.y without an
  // item list: group g = y / T, tile t = y % T (T = ceil(rows / 256)), rows
  // t 256 .. of the group, whose slots are row * groups + g
  int groups;
  int rows;
};

template <int K, int CB, bool MASKED>
__global__ __launch_bounds__(GW_THREADS, 1) void gemm_grouped_kernel(
    const uint32_t *__restrict__ tw, const uint16_t *__restrict__ xp,
    const uint16_t *__restrict__ svh, void *__restrict__ y, int ydt, int in_tiles, int out_tiles,
    CbRow mask, GemmGroup gg) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[GW_LDS_BYTES / 2];
  __shared__ uint32_t rows[GM_BM];
  MoeItem item;
  if (gg.groups > 0) {
    const int tpg = (gg.rows + GM_BM - 1) / GM_BM;
    const int g = (int)blockIdx.y / tpg, t = (int)blockIdx.y - g * tpg;
    item = MoeItem{(uint32_t)g, (uint32_t)(t * GM_BM), (uint32_t)min(GM_BM, gg.rows - t * GM_BM), 0u};
  } else {
    if (blockIdx.y >= *gg.n_items) return;  // the whole workgroup, before any barrier
    item = gg.items[blockIdx.y];
  }
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool mw = wave < 8;
  const int wm = (wave & 7) >> 1, wc = wave & 1;
  const int cg = blockIdx.x;
  const int M = (int)item.count;  // 1 .. GM_BM
  const int in = in_tiles * 16;
  const size_t out = (size_t)out_tiles * 16;
  constexpr int NW = 8 * K;
  const int NS = in_tiles / 4;
  if (tid < GM_BM)
    rows[tid] = gg.groups > 0 ? (item.start + min(tid, M - 1)) * (uint32_t)gg.groups + item.expert
                              : gg.sorted[item.start + min(tid, M - 1)];
  lds_barrier();

  f16v_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const uint32_t *twe = tw + (size_t)item.expert * gg.expert_words;
  if (mw) {
    uint32_t voff[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int R = 32 * wave + 8 * u + (lane >> 3);
      const int q = (lane & 7) ^ ((R >> 1) & 7);
      voff[u] = (uint32_t)(((size_t)rows[R] * in + 8 * q) * 2);
    }
    const uint32_t dma0 = (uint32_t)(uintptr_t)lds + GW_A0 + (uint32_t)(32 * wave) * 128;
    const int h = lane >> 5;
    uint32_t ax[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      ax[kk] = GW_A0 + (64 * wm + (lane & 31)) * 128 + 16 * ((4 * h + kk) ^ ((lane >> 1) & 7));
    const int brd = (64 * wc + (lane & 31)) * GM_LD + 32 * h;
    gw_mfma_main(acc, lds, reinterpret_cast<const char *>(xp), voff, dma0, ax, brd, NS);
  } else {
    const int dt = (tid - 512) & 255;
    const int tkl = dt >> 6, tnl = (dt >> 3) & 7, c = dt & 7;
    const uint32_t *twc = twe + ((size_t)tkl * out_tiles + cg * 8 + tnl) * NW + c * K;
    const size_t wstage = (size_t)4 * out_tiles * NW;
    const int src = ((lane & ~7) | ((lane + 7) & 7)) << 2;
    const int bst = (tnl * 16 + c) * GM_LD + tkl * 16;
    if (wave < 12)
      gw_decode_main<K, CB, MASKED, 0>(lds, twc, wstage, src, bst, NS, mask);
    else
      gw_decode_main<K, CB, MASKED, 1>(lds, twc, wstage, src, bst, NS, mask);
  }
  gemm_tile_end<GW_THREADS>(acc, lds, mw, wm, wc, 0, cg, M, out, 1, 0,
                            svh + (size_t)item.expert * out, y, ydt, nullptr, nullptr, rows);
}

// Calls go(codebook, masked) with both as compile-time constants for the
// weight's codebook form and window.  pair1 exists at n = 24..64 (its table's
// rows) and only at the full window (the table admits its own window alone),
// so it has forms at K = 2, 3, 4 and the run-time rate (K = 0) only.
template <int K, typename G>
inline void cb_dispatch(const Format &f, G &&go) {
  using T = std::true_type;
  using F = std::false_type;
  const bool masked = f.window < 16;
  switch (f.codebook) {
    case CB_MCG:
      masked ? go(std::integral_constant<int, CB_MCG>{}, T{})
             : go(std::integral_constant<int, CB_MCG>{}, F{});
      break;
    case CB_HASH:
      masked ? go(std::integral_constant<int, CB_HASH>{}, T{})
             : go(std::integral_constant<int, CB_HASH>{}, F{});
      break;
    case CB_PAIR1:
      if constexpr (K == 0 || (K >= 2 && K <= 4)) go(std::integral_constant<int, CB_PAIR1>{}, F{});
      break;
    default:
      masked ? go(std::integral_constant<int, CB_MUL1>{}, T{})
             : go(std::integral_constant<int, CB_MUL1>{}, F{});
  }
}

template <int K>
void gemm_grouped_go(const Format &f, dim3 grid, hipStream_t s, const uint32_t *tw,
                     const uint16_t *xp, const uint16_t *svh, void *y, int ydt, int in_tiles,
                     int out_tiles, const GemmGroup &gg) {
  static_assert(K > 0, "the GEMM serves integer rates");
  const CbRow m = f.dec();
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(GW_THREADS), 0, s, tw, xp, svh, y, ydt, in_tiles,
                       out_tiles, m, gg);
  };
  cb_dispatch<K>(f, [&](auto CBC, auto MC) {
    go(gemm_grouped_kernel<K, decltype(CBC)::value, decltype(MC)::value>);
  });
}

// ====================================================== per-rate launchers
//
// K = 1..8: an integer rate (n = 16K) with compile-time windows; K = 0: any
// even n (GEMV only).

// Dense GEMV over up to four weights (tw[i] their trellis words).
template <int K>
void gemv_go(const Format &f, int prep, dim3 grid, size_t lds, hipStream_t s,
             const uint32_t *const *tw, const void *x, uint32_t g0, uint32_t g1, uint32_t g2,
             const GemvArgs &a) {
  const dim3 blk(GEMV_THREADS);
  // a.c.x2 set: the SwiGLU prologue (x is gate, x2 up); a.c.nssq set: the
  // RMSNorm prologue (x is the f32 residual; rows in one prepare batch);
  // a.c.attn_part set: the attention prologue (x is the split slots; one
  // batch)
  auto go2 = [&](auto CBC, auto MC, auto PC) {
    constexpr int CB = decltype(CBC)::value;
    constexpr bool M = decltype(MC)::value;
    constexpr int O = decltype(PC)::value;
    if (a.c.x2 != nullptr) {
      hipLaunchKernelGGL((gemv_kernel<K, CB, M, O, PRO_SWIGLU>), grid, blk, lds, s, tw[0], tw[1],
                         tw[2], tw[3], x, g0, g1, g2, a);
      return;
    }
    if constexpr (O == 0) {
      if (a.c.nssq != nullptr) {
        hipLaunchKernelGGL((gemv_kernel<K, CB, M, O, PRO_RMSNORM>), grid, blk, lds, s, tw[0],
                           tw[1], tw[2], tw[3], x, g0, g1, g2, a);
        return;
      }
      if (a.c.attn_part != nullptr) {
        hipLaunchKernelGGL((gemv_kernel<K, CB, M, O, PRO_ATTN>), grid, blk, lds, s, tw[0],
                           tw[1], tw[2], tw[3], x, g0, g1, g2, a);
        return;
      }
    }
    hipLaunchKernelGGL((gemv_kernel<K, CB, M, O, PRO_PLAIN>), grid, blk, lds, s, tw[0], tw[1],
                       tw[2], tw[3], x, g0, g1, g2, a);
  };
  // prep: 0 (one prepare batch) or the rows form's passes (1, 2, PREP_PASSES)
  auto go = [&](auto CBC, auto MC) {
    switch (prep) {
      case 0: go2(CBC, MC, std::integral_constant<int, 0>{}); break;
      case 1: go2(CBC, MC, std::integral_constant<int, 1>{}); break;
      case 2: go2(CBC, MC, std::integral_constant<int, 2>{}); break;
      default: go2(CBC, MC, std::integral_constant<int, PREP_PASSES>{});
    }
  };
  cb_dispatch<K>(f, go);
}

// The prepare form of a GEMV launch: 0 when its rows' items fit one batch,
// else the fewest passes of the rows form that cover them.
inline int gemv_prep_form(int rows, int tps) {
  const int items = rows * (tps / 8);
  if (items <= PREP_ITEMS) return 0;
  return items <= PREP_GROUPS ? 1 : items <= 2 * PREP_GROUPS ? 2 : PREP_PASSES;
}

template <int K>
void moe_gemv_go(const Format &f, int pro, dim3 grid, size_t lds, hipStream_t s,
                 const uint32_t *tw0, const uint32_t *tw1, const void *x, uint32_t g0,
                 uint32_t g1, uint32_t g2, int topk, const uint32_t *sorted, const MoeItem *items,
                 const uint32_t *n_items, const GemvArgs &a) {
  const dim3 blk(GEMV_THREADS);
  cb_dispatch<K>(f, [&](auto CBC, auto MC) {
    constexpr int CB = decltype(CBC)::value;
    constexpr bool M = decltype(MC)::value;
    if (pro == PRO_SWIGLU)
      hipLaunchKernelGGL((moe_gemv_kernel<K, CB, M, PRO_SWIGLU>), grid, blk, lds, s, tw0, tw1, x,
                         g0, g1, g2, topk, sorted, items, n_items, a);
    else
      hipLaunchKernelGGL((moe_gemv_kernel<K, CB, M, PRO_PLAIN>), grid, blk, lds, s, tw0, tw1, x,
                         g0, g1, g2, topk, sorted, items, n_items, a);
  });
}


template <int K>
void gemm_go(const Format &f, dim3 grid, hipStream_t s, const uint32_t *tw, const uint16_t *xp,
             const uint16_t *svh, void *y, int ydt, uint16_t *zout, int M, int in_tiles,
             int out_tiles, float *kpart) {
  static_assert(K > 0, "the GEMM serves integer rates");
  const CbRow m = f.dec();
  cb_dispatch<K>(f, [&](auto CBC, auto MC) {
    hipLaunchKernelGGL((gemm_ws_kernel<K, decltype(CBC)::value, decltype(MC)::value>), grid,
                       dim3(GW_THREADS), 0, s, tw, xp, svh, y, ydt, zout, M, in_tiles, out_tiles, m,
                       kpart);
  });
}

// The prefill GEMM at a half-integer rate n = 8 FR (the specialised-wave
// kernel; activations addressed with 32-bit offsets, checked by the caller).
template <int FR>
void gemm_frac_go(const Format &f, dim3 grid, hipStream_t s, const uint32_t *tw,
                  const uint16_t *xp, const uint16_t *svh, void *y, int ydt, uint16_t *zout, int M,
                  int in_tiles, int out_tiles, float *kpart) {
  static_assert(FR % 2 == 1, "a half-integer rate");
  const CbRow m = f.dec();
  cb_dispatch<0>(f, [&](auto CBC, auto MC) {
    hipLaunchKernelGGL((gemm_ws_kernel<1, decltype(CBC)::value, decltype(MC)::value, FR>), grid,
                       dim3(GW_THREADS), 0, s, tw, xp, svh, y, ydt, zout, M, in_tiles, out_tiles,
                       m, kpart);
  });
}

// Declarations of one rate's launcher instantiations.
#define EXL3_GEMV_GO(KK)                                                                 \
  void gemv_go<KK>(const Format &, int, dim3, size_t, hipStream_t, const uint32_t *const *, \
                   const void *, uint32_t, uint32_t, uint32_t, const GemvArgs &)
#define EXL3_MOE_GEMV_GO(KK)                                                                    \
  void moe_gemv_go<KK>(const Format &, int, dim3, size_t, hipStream_t, const uint32_t *,       \
                       const uint32_t *, const void *, uint32_t, uint32_t, uint32_t, int,       \
                       const uint32_t *, const MoeItem *, const uint32_t *, const GemvArgs &)
#define EXL3_GEMM_GROUPED_GO(KK)                                                             \
  void gemm_grouped_go<KK>(const Format &, dim3, hipStream_t, const uint32_t *, const uint16_t *, \
                           const uint16_t *, void *, int, int, int, const GemmGroup &)
#define EXL3_GEMM_GO(KK)                                                                    \
  void gemm_go<KK>(const Format &, dim3, hipStream_t, const uint32_t *, const uint16_t *, \
                   const uint16_t *, void *, int, uint16_t *, int, int, int, float *)
#define EXL3_GEMM_FRAC_GO(FR)                                                                    \
  void gemm_frac_go<FR>(const Format &, dim3, hipStream_t, const uint32_t *, const uint16_t *, \
                        const uint16_t *, void *, int, uint16_t *, int, int, int, float *)

#ifndef EXL3_INST_K
// instantiated in the per-rate units only
#define EXL3_EXTERN_RATE(KK)            \
  extern template EXL3_GEMV_GO(KK);     \
  extern template EXL3_MOE_GEMV_GO(KK);
EXL3_EXTERN_RATE(0)
EXL3_EXTERN_RATE(1)
EXL3_EXTERN_RATE(2)
EXL3_EXTERN_RATE(3)
EXL3_EXTERN_RATE(4)
EXL3_EXTERN_RATE(5)
EXL3_EXTERN_RATE(6)
EXL3_EXTERN_RATE(7)
EXL3_EXTERN_RATE(8)
#undef EXL3_EXTERN_RATE
extern template EXL3_GEMM_GO(1);
extern template EXL3_GEMM_GROUPED_GO(1);
extern template EXL3_GEMM_GO(2);
extern template EXL3_GEMM_GROUPED_GO(2);
extern template EXL3_GEMM_GO(3);
extern template EXL3_GEMM_GROUPED_GO(3);
extern template EXL3_GEMM_GO(4);
extern template EXL3_GEMM_GROUPED_GO(4);
extern template EXL3_GEMM_GO(5);
extern template EXL3_GEMM_GROUPED_GO(5);
extern template EXL3_GEMM_GO(6);
extern template EXL3_GEMM_GROUPED_GO(6);
extern template EXL3_GEMM_GO(7);
extern template EXL3_GEMM_GROUPED_GO(7);
extern template EXL3_GEMM_GO(8);
extern template EXL3_GEMM_GROUPED_GO(8);
extern template EXL3_GEMM_FRAC_GO(3);
extern template EXL3_GEMM_FRAC_GO(5);
#endif

}  // namespace exl3
