// exl3_host.cpp -- the C ABI of include/exl3_mi355x.h: the quant plugin
// table's entries (claims, validate, bill, open, close, load_tensor,
// load_bank, release, matmul, moe, swiglu) over the HIP kernels.
//
// Reference entries (paths relative to /root/reference/plugins/):
//   turboexl3_ds41/config.zig:43-61   claims / validate / bill
//   turboexl3_ds41/plugin.zig:52-287  open .. swiglu
//   turboexl3_qwen38/config.zig:86-105 turboexl3's block rules (named refusals)
// Errors are returned as named refusals; nothing falls back to another path.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <string>
#include <utility>
#include <vector>

#include "../../include/exl3_decoder.h"
#include "../../include/exl3_mi355x.h"
#include "exl3_codebooks.h"
#include "exl3_dense.h"
#include "exl3_json.h"
#include "exl3_kernels.h"
#include "exl3_selfcheck.h"

using exl3::CodebookTable;
using exl3::Format;
using exl3::Json;
using exl3::PACK_MCG;
using exl3::PACK_PAIR1;
using exl3::PACK_SPEC1;
using exl3::pack_codebook_of;
using exl3::resolve_codebook_table;
using exl3::codebook_row;

namespace {

const char *const kName = "turboexl3_mi355x";
const char *const kNameQwen38 = "turboexl3_mi355x_qwen38";

exl3_verdict ok() { return exl3_verdict{EXL3_OK, ""}; }
exl3_verdict refuse(int32_t code, const char *why) { return exl3_verdict{code, why}; }

// --------------------------------------------------------------- blocks

// A parsed EXL3 quantization block: the codebook and window the pack's
// search used (a bank's rate comes from each tensor's packed dim).
struct Block {
  bool exl3 = false;
  int codebook = 0;  // PackCodebook (0 mul1, 1 mcg, 2 spec1, 3 pair1, 4 std1), -1 other
  int window = 16;   // -1: not an integer in 8..16
  bool has_k = false;
  double k = 0.0;
  // spec1, std1, pair1: the table the block names, or why it names none
  const CodebookTable *table = nullptr;
  const char *table_refusal = nullptr;
};

Block parse_block(const Json &b) {
  Block out;
  if (!b.is_object()) return out;
  const Json *qm = b.get("quant_method");
  const Json *fm = b.get("format");
  out.exl3 = (qm && qm->is_string("exl3")) || (fm && fm->is_string("exl3"));
  if (const Json *cb = b.get("codebook"))
    out.codebook = cb->kind == Json::STRING ? pack_codebook_of(cb->str.c_str()) : -1;
  if (const Json *w = b.get("window")) {
    if (w->kind == Json::NUMBER && w->integral && w->num >= 8 && w->num <= 16)
      out.window = (int)w->num;
    else
      out.window = -1;
  }
  if (out.codebook >= PACK_SPEC1 && out.window >= 0)
    out.table_refusal = resolve_codebook_table(b, out.codebook, out.window, &out.table);
  if (const Json *k = b.get("k")) {
    out.has_k = true;
    out.k = k->kind == Json::NUMBER ? k->num : -1.0;
  }
  return out;
}

Json parse(exl3_str s) { return Json::parse(s.ptr, s.len); }

// 16k halfwords per tile must be an even integer in 16..128
// (turboexl3_qwen38/config.zig:95-103).
bool rate_ok(double k) {
  const double scaled = k * 16.0;
  const double n = std::round(scaled);
  return std::fabs(scaled - n) <= 1e-6 && n >= 16 && n <= 128 && std::fmod(n, 2.0) == 0.0;
}

bool n_ok(int64_t n) { return n >= 16 && n <= 128 && n % 2 == 0; }

// ------------------------------------------------------------- weights

// A group of un-rotated resident matrices joined side by side:
// [in, cols] in the activation dtype `act` (mlx code), member m's columns
// starting at its `col`.
struct WeightPriv;
struct Joined {
  void *data = nullptr;
  int act = 0;
  int64_t in = 0, cols = 0;
  int device = 0;
  std::vector<WeightPriv *> members;
};

// A linear's resident state (QuantTable.resident, quant.zig:96-107):
// admitted by exl3_resident; its decoded matrix W_inner f16 [in, out] held
// from its first prefill call on, or, once un-rotated, its columns of a
// joined public matrix.
struct ResidentState {
  bool admitted = false;
  uint16_t *inner = nullptr;
  std::shared_ptr<Joined> joined;
  int64_t col = 0;
};

struct WeightPriv {
  Format f;
  int64_t in = 0, out = 0, experts = 0;  // experts = 0: a single linear
  int64_t groups = 0;  // a grouped linear: `experts` banks, x [..., groups, in]
  int device = 0;
  bool borrowed = false;
  ResidentState res;
};

WeightPriv *priv_of(const exl3_weight *w) {
  return w ? static_cast<WeightPriv *>(w->priv) : nullptr;
}

// The weight's private part when it is one linear (not a bank or a group).
const WeightPriv *single_linear(const exl3_weight *w) {
  const WeightPriv *pv = priv_of(w);
  return pv && pv->experts == 0 && pv->groups == 0 ? pv : nullptr;
}

int64_t numel(const exl3_array &a) {
  int64_t n = 1;
  for (int i = 0; i < a.ndim; ++i) n *= a.shape[i];
  return n;
}

size_t dt_size(int dt) {
  switch (dt) {
    case EXL3_DT_BOOL:
    case EXL3_DT_U8:
    case EXL3_DT_I8: return 1;
    case EXL3_DT_U16:
    case EXL3_DT_I16:
    case EXL3_DT_F16:
    case EXL3_DT_BF16: return 2;
    case EXL3_DT_U32:
    case EXL3_DT_I32:
    case EXL3_DT_F32: return 4;
    default: return 8;
  }
}

// mlx dtype -> kernel activation type (-1: not an activation dtype)
int act_of(int dt) {
  if (dt == EXL3_DT_F16) return exl3::ACT_F16;
  if (dt == EXL3_DT_BF16) return exl3::ACT_BF16;
  if (dt == EXL3_DT_F32) return exl3::ACT_F32;
  return -1;
}

exl3_array make_array(void *data, int dt, std::initializer_list<int64_t> shape, bool owned) {
  exl3_array a{};
  a.data = data;
  a.dtype = dt;
  a.ndim = (int32_t)shape.size();
  int i = 0;
  for (int64_t s : shape) a.shape[i++] = s;
  a.owned = owned ? 1u : 0u;
  return a;
}

// -------------------------------------------------------------- scratch

// Device scratch per (device, stream): prepared rows, GEMM split-K planes,
// the GEMV/MoE slot buffer (a header with the split-K status word, then the
// partial-sum slots, all-ones bytes when made and left so by every call), MoE
// staging.  Calls on one
// stream take its lock; calls on different streams or devices run
// independently.  A buffer that must grow is replaced by a larger one (at
// least twice the size) and the old one is kept, not freed, until
// exl3_scratch_release: a HIP graph captured earlier on the stream may still
// point at it.  Growing while the stream is being captured is refused (the
// allocation and its fill cannot be captured): run the call once outside the
// capture first.
struct StreamScratch {
  std::mutex mu;
  void *xp = nullptr;
  size_t xp_bytes = 0;
  void *kpart = nullptr;
  size_t kpart_bytes = 0;
  void *slots = nullptr;
  size_t slot_bytes = 0;
  void *moe = nullptr;
  size_t moe_bytes = 0;
  void *aux = nullptr;  // a grouped linear's gathered rows and outputs; swiglu_shared's routes
  size_t aux_bytes = 0;
  std::vector<void *> retired;  // superseded buffers, freed by exl3_scratch_release
  // superseded slot buffers (each with its own status word and slots)
  std::vector<std::pair<void *, size_t>> retired_slots;
  // fixed: the buffers above are given (exl3_matmul_noalloc's array) and are
  // never replaced; a call that needs more is refused, not grown
  bool fixed = false;
};

std::mutex g_scratch_mu;
std::map<std::pair<int, hipStream_t>, StreamScratch> g_scratch;

bool capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(s, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

hipError_t grow(StreamScratch *ss, void **p, size_t *have, size_t need, hipStream_t s) {
  if (*have >= need && *p != nullptr) return hipSuccess;
  if (ss->fixed) return hipErrorOutOfMemory;
  if (capturing(s)) return hipErrorStreamCaptureUnsupported;
  const size_t bytes = std::max<size_t>({need, 2 * *have, 256});
  void *fresh = nullptr;
  hipError_t e = hipMalloc(&fresh, bytes);
  if (e != hipSuccess) return e;
  if (*p != nullptr) ss->retired.push_back(*p);
  *p = fresh;
  *have = bytes;
  return hipSuccess;
}

// The stream's slot buffer with room for `pf` partial-sum floats, as one
// exl3::Scratch: a header with the status word (zero when made), then the
// slots (the empty mark, all-ones bytes, when made).
hipError_t slots_for(StreamScratch *ss, size_t pf, hipStream_t s, exl3::Scratch *out) {
  const size_t have = ss->slots ? (ss->slot_bytes - exl3::SLOT_HEADER_BYTES) / 4 : 0;
  if (ss->slots == nullptr || pf > have) {
    if (ss->fixed) return hipErrorOutOfMemory;
    if (capturing(s)) return hipErrorStreamCaptureUnsupported;
    const size_t p2 = std::max<size_t>({pf, 2 * have, 64});
    const size_t bytes = exl3::SLOT_HEADER_BYTES + p2 * 4;
    void *fresh = nullptr;
    hipError_t e = hipMalloc(&fresh, bytes);
    if (e != hipSuccess) return e;
    e = hipMemsetAsync(fresh, 0, exl3::SLOT_HEADER_BYTES, s);
    if (e == hipSuccess)
      e = hipMemsetAsync((char *)fresh + exl3::SLOT_HEADER_BYTES, 0xFF, p2 * 4, s);
    if (e != hipSuccess) {
      (void)hipFree(fresh);
      return e;
    }
    if (ss->slots != nullptr) ss->retired_slots.push_back({ss->slots, ss->slot_bytes});
    ss->slots = fresh;
    ss->slot_bytes = bytes;
  }
  out->status = (uint32_t *)ss->slots;
  out->partial = (float *)((char *)ss->slots + exl3::SLOT_HEADER_BYTES);
  out->partial_floats = (ss->slot_bytes - exl3::SLOT_HEADER_BYTES) / 4;
  return hipSuccess;
}

StreamScratch *scratch_for(int device, hipStream_t s) {
  std::lock_guard<std::mutex> g(g_scratch_mu);
  return &g_scratch[{device, s}];
}

exl3_verdict hip_failed(hipError_t e) {
  if (e == hipErrorStreamCaptureUnsupported)
    return refuse(EXL3_FAILED,
                  "turboexl3_mi355x: scratch must grow while the stream is being captured; run the "
                  "call once outside the capture first");
  if (e == hipErrorOutOfMemory) return refuse(EXL3_TOO_LARGE, "turboexl3_mi355x: out of device memory");
  return refuse(EXL3_FAILED, "turboexl3_mi355x: a HIP call failed");
}

// Reads <base>.<part> from the source.
bool source_tensor(const exl3_load_ctx *ctx, const std::string &name, exl3_host_tensor *t) {
  if (!ctx->source || !ctx->source->tensor) return false;
  exl3_str s{name.data(), name.size()};
  std::memset(t, 0, sizeof(*t));
  return ctx->source->tensor(ctx->source->self, s, t) != 0 && t->data != nullptr;
}

struct Parts {
  exl3_host_tensor t, u, v;
};

// trellis [in/16, out/16, n] (i16 or u16), suh f16 [in], svh f16 [out]
// (turboexl3_ds41/plugin.zig:96-103); in_dim 0 = any.
bool shaped(const Parts &p, uint32_t in_dim) {
  if (p.t.ndim != 3 || p.u.ndim != 1 || p.v.ndim != 1) return false;
  if (p.t.dtype != EXL3_DT_I16 && p.t.dtype != EXL3_DT_U16) return false;
  if (p.u.shape[0] != p.t.shape[0] * 16 || p.v.shape[0] != p.t.shape[1] * 16) return false;
  if (in_dim != 0 && p.u.shape[0] != (int64_t)in_dim) return false;
  return p.u.dtype == EXL3_DT_F16 && p.v.dtype == EXL3_DT_F16;
}

int parts_of(const exl3_load_ctx *ctx, const std::string &base, Parts *p) {
  if (!source_tensor(ctx, base + ".trellis", &p->t)) return 0;
  if (!source_tensor(ctx, base + ".suh", &p->u)) return 0;
  if (!source_tensor(ctx, base + ".svh", &p->v)) return 0;
  return 1;
}

const exl3_verdict kNotShaped = {
    EXL3_UNSUPPORTED,
    "turboexl3_mi355x: not an EXL3 linear of the expected input width (trellis [in/16, out/16, "
    "n], suh f16 [in], svh f16 [out])"};
const exl3_verdict kMissing = {EXL3_FAILED, "MissingWeight"};
const exl3_verdict kRate = {EXL3_UNSUPPORTED, "turboexl3_mi355x: Exl3RateUnsupported"};
const exl3_verdict kShape = {EXL3_UNSUPPORTED, "turboexl3_mi355x: BadExl3Shape"};
const exl3_verdict kDtype = {EXL3_UNSUPPORTED, "turboexl3_mi355x: BadExl3Dtype"};

struct OpenState {
  int codebook = 0;
  int window = 16;
};

}  // namespace

// ================================================================ entries

extern "C" {

// turboexl3_ds41/config.zig:43-47: exllamav3's block (`quant_method`
// exl3) on a DeepSeek-V4.1 pack (config `model_type` deepseek_v41).
exl3_claim exl3_claims(exl3_str block_json, exl3_str config_json) {
  const Json b = parse(block_json);
  if (!b.is_object()) return EXL3_CLAIM_NO;
  const Json *qm = b.get("quant_method");
  if (!qm || !qm->is_string("exl3")) return EXL3_CLAIM_NO;
  const Json c = parse(config_json);
  const Json *mt = c.is_object() ? c.get("model_type") : nullptr;
  return mt && mt->is_string("deepseek_v41") ? EXL3_CLAIM_BY_MARKER : EXL3_CLAIM_NO;
}

// turboexl3_qwen38/config.zig:18-32 as a quant table's claim: a Qwen3.8 pack
// (config `model_type` qwen4_exp or qwen4_exp_text, src/direct/config.zig:12)
// whose config names a non-null `trunk_quant` block; the block itself is
// validate's to refuse by name.
exl3_claim exl3_claims_qwen38(exl3_str block_json, exl3_str config_json) {
  (void)block_json;
  const Json c = parse(config_json);
  if (!c.is_object()) return EXL3_CLAIM_NO;
  const Json *mt = c.get("model_type");
  if (!mt || !(mt->is_string("qwen4_exp") || mt->is_string("qwen4_exp_text"))) return EXL3_CLAIM_NO;
  const Json *t = c.get("trunk_quant");
  return t && t->kind != Json::NUL ? EXL3_CLAIM_BY_MARKER : EXL3_CLAIM_NO;
}

exl3_verdict exl3_validate(exl3_str block_json, exl3_str config_json, const exl3_pack_dir *dir) {
  (void)dir;
  const Json b = parse(block_json);
  const Block blk = parse_block(b);
  if (!blk.exl3) return refuse(EXL3_UNSUPPORTED, "turboexl3_mi355x: NotExl3");
  // turboexl3's codebooks: mul1 and mcg (the table codebooks serve through
  // exl3_weight_wrap)
  if (blk.codebook < 0 || blk.codebook > PACK_MCG)
    return refuse(EXL3_UNSUPPORTED, "turboexl3_mi355x: Exl3CodebookUnsupported");
  if (blk.window < 0) return refuse(EXL3_UNSUPPORTED, "turboexl3_mi355x: Exl3WindowUnsupported");
  if (blk.has_k && !rate_ok(blk.k)) return kRate;
  const Json c = parse(config_json);
  if (c.is_object()) {
    const Json *text = c.get("text_config");
    const Json *root = (text && text->is_object()) ? text : &c;
    const Json *k = root->get("num_experts_per_tok");
    if (k && k->kind == Json::NUMBER && k->integral && k->num > 32)
      return refuse(EXL3_UNSUPPORTED, "turboexl3_mi355x: Exl3TopKExceedsReduceBank");
  }
  return ok();
}

uint64_t exl3_bill(exl3_str block_json, exl3_str model_dir, uint64_t stored) {
  (void)block_json;
  (void)model_dir;
  return stored;
}

exl3_verdict exl3_open(exl3_load_ctx *ctx) {
  if (!ctx) return refuse(EXL3_FAILED, "turboexl3_mi355x: no load context");
  const Block blk = parse_block(parse(ctx->block_json));
  if (!blk.exl3 || blk.codebook < 0 || blk.codebook > PACK_MCG || blk.window < 0)
    return refuse(EXL3_UNSUPPORTED, "turboexl3_mi355x: not an exllamav3 mul1 or mcg block");
  // the self-check's host part first (it needs no device)
  exl3_verdict v = exl3::self_check(-1, 0, nullptr);
  if (v.code != EXL3_OK) return v;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
    return refuse(EXL3_UNSUPPORTED, "turboexl3_mi355x: no HIP device");
  if (ctx->device < 0 || ctx->device >= count)
    return refuse(EXL3_UNSUPPORTED, "turboexl3_mi355x: no such device");
  if (hipSetDevice(ctx->device) != hipSuccess) return hip_failed(hipErrorInvalidDevice);
  // the kernels must decode the golden planes and the codebook's states
  // exactly on this device before a pack is accepted (turboexl3_ds41/src/
  // exl3/quant.zig:469-503)
  v = exl3::self_check(ctx->device,
                       blk.codebook == PACK_MCG ? exl3::CB_FORM_MCG : exl3::CB_FORM_MUL1,
                       (hipStream_t)ctx->stream);
  if (v.code != EXL3_OK) return v;
  OpenState *st = new OpenState{blk.codebook, blk.window};
  ctx->state = st;
  return ok();
}

void exl3_close(exl3_load_ctx *ctx) {
  if (ctx && ctx->state) {
    delete static_cast<OpenState *>(ctx->state);
    ctx->state = nullptr;
  }
}

static exl3_verdict upload(const exl3_load_ctx *ctx, const std::vector<const exl3_host_tensor *> &parts,
                           size_t each_bytes, void **dst) {
  hipStream_t s = (hipStream_t)ctx->stream;
  hipError_t e = hipMalloc(dst, std::max<size_t>(each_bytes * parts.size(), 256));
  if (e != hipSuccess) return refuse(EXL3_TOO_LARGE, "turboexl3_mi355x: out of device memory");
  for (size_t i = 0; i < parts.size(); ++i) {
    e = hipMemcpyAsync((char *)*dst + i * each_bytes, parts[i]->data, each_bytes,
                       hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return hip_failed(e);
  }
  e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_failed(e);
  return ok();
}

static void free_weight_arrays(exl3_weight *w) {
  for (exl3_array *a : {&w->w, &w->scales, &w->biases, &w->side})
    if (a->owned && a->data) {
      (void)hipFree(a->data);
      a->data = nullptr;
    }
}

// Builds a weight from a stack of E linears (E = 0: one linear, rank 3).
static exl3_verdict load_parts(const exl3_load_ctx *ctx, const std::vector<Parts> &ps, bool bank,
                               exl3_weight *out) {
  const OpenState *st = static_cast<const OpenState *>(ctx->state);
  if (!st) return refuse(EXL3_FAILED, "turboexl3_mi355x: load before open");
  const Parts &p0 = ps[0];
  const int64_t it = p0.t.shape[0], ot = p0.t.shape[1], n = p0.t.shape[2];
  if (!n_ok(n)) return kRate;
  const int64_t in = it * 16, outf = ot * 16;
  if (in % 128 != 0 || outf % 128 != 0) return kNotShaped;
  for (const Parts &p : ps)
    if (p.t.shape[0] != it || p.t.shape[1] != ot || p.t.shape[2] != n) return kNotShaped;
  if (hipSetDevice(ctx->device) != hipSuccess) return hip_failed(hipErrorInvalidDevice);
  std::vector<const exl3_host_tensor *> tv, uv, vv;
  for (const Parts &p : ps) {
    tv.push_back(&p.t);
    uv.push_back(&p.u);
    vv.push_back(&p.v);
  }
  exl3_weight w{};
  void *dt = nullptr, *du = nullptr, *dv = nullptr;
  exl3_verdict v = upload(ctx, tv, (size_t)(it * ot * n) * 2, &dt);
  if (v.code == EXL3_OK) v = upload(ctx, uv, (size_t)in * 2, &du);
  if (v.code == EXL3_OK) v = upload(ctx, vv, (size_t)outf * 2, &dv);
  if (v.code != EXL3_OK) {
    for (void *d : {dt, du, dv})
      if (d) (void)hipFree(d);
    return v;
  }
  const int64_t E = (int64_t)ps.size();
  if (bank) {
    w.w = make_array(dt, EXL3_DT_U16, {E, it, ot, n}, true);
    w.scales = make_array(du, EXL3_DT_F16, {E, in}, true);
    w.biases = make_array(dv, EXL3_DT_F16, {E, outf}, true);
  } else {
    w.w = make_array(dt, EXL3_DT_U16, {it, ot, n}, true);
    w.scales = make_array(du, EXL3_DT_F16, {in}, true);
    w.biases = make_array(dv, EXL3_DT_F16, {outf}, true);
  }
  WeightPriv *pv = new WeightPriv;
  pv->f.n = (int)n;
  pv->f.codebook = st->codebook;
  pv->f.window = st->window;
  pv->in = in;
  pv->out = outf;
  pv->experts = bank ? E : 0;
  pv->device = ctx->device;
  w.priv = pv;
  *out = w;
  return ok();
}

exl3_verdict exl3_load_tensor(const exl3_load_ctx *ctx, exl3_str name, uint32_t in_dim,
                              exl3_weight *out) {
  if (!ctx || !out) return refuse(EXL3_FAILED, "turboexl3_mi355x: null argument");
  const std::string base(name.ptr ? name.ptr : "", name.len);
  std::vector<Parts> ps(1);
  if (parts_of(ctx, base, &ps[0])) {
    if (!shaped(ps[0], in_dim)) return kNotShaped;
    return load_parts(ctx, ps, false, out);
  }
  // a grouped linear: <base>.slice.<g> for g = 0, 1, .. as one G-bank
  // (turboexl3_ds41/plugin.zig:108-125)
  ps.clear();
  for (int g = 0;; ++g) {
    Parts p;
    if (!parts_of(ctx, base + ".slice." + std::to_string(g), &p)) break;
    if (!shaped(p, in_dim)) return kNotShaped;
    ps.push_back(p);
  }
  if (ps.empty()) return kMissing;
  exl3_verdict v = load_parts(ctx, ps, true, out);
  if (v.code != EXL3_OK) return v;
  static_cast<WeightPriv *>(out->priv)->groups = (int64_t)ps.size();
  out->flags = EXL3_WEIGHT_GROUPED;
  return ok();
}

exl3_verdict exl3_load_bank(const exl3_load_ctx *ctx, exl3_str name, uint32_t in_dim,
                            exl3_weight *out) {
  if (!ctx || !out) return refuse(EXL3_FAILED, "turboexl3_mi355x: null argument");
  const std::string full(name.ptr ? name.ptr : "", name.len);
  const size_t dot = full.rfind('.');
  if (dot == std::string::npos) return kMissing;
  const std::string prefix = full.substr(0, dot), suffix = full.substr(dot);
  std::vector<Parts> ps;
  for (int e = 0;; ++e) {
    Parts p;
    if (!parts_of(ctx, prefix + "." + std::to_string(e) + suffix, &p)) break;
    if (!shaped(p, in_dim)) return kNotShaped;
    ps.push_back(p);
  }
  if (ps.empty()) return kMissing;
  // Every expert the layer's router scores (<layer>.gate.weight [experts,
  // hidden]) must be in the bank (turboexl3_ds41/plugin.zig:132-151).
  const std::string tail = ".experts";
  if (prefix.size() > tail.size() && prefix.compare(prefix.size() - tail.size(), tail.size(), tail) == 0) {
    exl3_host_tensor g;
    const std::string router = prefix.substr(0, prefix.size() - tail.size()) + ".gate.weight";
    if (!source_tensor(ctx, router, &g) || g.ndim != 2 || g.shape[0] != (int64_t)ps.size())
      return refuse(EXL3_UNSUPPORTED,
                    "turboexl3_mi355x: the bank holds another count of experts than its router scores");
  }
  return load_parts(ctx, ps, true, out);
}

// ------------------------------------------------------ resident matrices

// The weights exl3_resident admitted (quant.zig:96-107: `resident`,
// `resident_pending`, `unrotate`, `linear_joined`).  Memory for speed at
// prefill widths, where it buys speed: a held W_inner f16 makes the matmul a
// prepare, a dense f16 GEMM (hipBLASLt) and the finish -- held only at the
// rates without the prefill GEMM (those run 16-row GEMV passes otherwise);
// at the GEMM's rates the fused decode GEMM is faster than the held path
// (prepare, dense GEMM, z round trip, finish), so the admission reserves the
// bytes (pending) and holds nothing until `unrotate`.  An un-rotated group's
// public matrix makes the matmul one dense GEMM in the activation dtype, at
// every rate.  Decode widths keep the EXL3 GEMV, which reads 2 to 8 times
// fewer bytes.
static std::mutex g_res_mu;
static std::set<WeightPriv *> g_resident;

// Whether an admitted weight holds its W_inner for prefill matmuls.
static bool holds_inner(const WeightPriv *pv) { return !pv->f.gemm_rate(); }

static uint64_t resident_bytes(const WeightPriv *pv) { return (uint64_t)pv->in * pv->out * 2; }

// Frees what pv holds (its decoded matrix; its place in a joined group, the
// group's matrix with its last member).  The device finishes its queued work
// first: a kept matrix may be read by any stream.  Caller holds g_res_mu.
static void resident_drop(WeightPriv *pv) {
  ResidentState &r = pv->res;
  if (r.inner || r.joined) {
    (void)hipSetDevice(pv->device);
    (void)hipDeviceSynchronize();
  }
  if (r.inner) (void)hipFree(r.inner);
  r.inner = nullptr;
  if (r.joined) {
    auto &m = r.joined->members;
    m.erase(std::remove(m.begin(), m.end(), pv), m.end());
    if (m.empty() && r.joined->data) {
      (void)hipFree(r.joined->data);
      r.joined->data = nullptr;
    }
    r.joined.reset();
  }
  r.col = 0;
  r.admitted = false;
}

// Holds pv's decoded matrix (decode_matrix into a new buffer on s).  Not
// under graph capture (the allocation cannot be captured).
static hipError_t resident_hold(const exl3_weight *w, WeightPriv *pv, hipStream_t s) {
  if (pv->res.inner) return hipSuccess;
  if (capturing(s)) return hipErrorStreamCaptureUnsupported;
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, resident_bytes(pv));
  if (e != hipSuccess) return e;
  e = exl3::launch_decode_matrix((const uint16_t *)w->w.data, pv->f, (int)pv->in, (int)pv->out,
                                 (uint16_t *)p, s);
  if (e != hipSuccess) {
    (void)hipFree(p);
    return e;
  }
  pv->res.inner = (uint16_t *)p;
  return hipSuccess;
}

// The matmul of an admitted weight at prefill widths through its resident
// matrix.  *taken false: the EXL3 kernels serve the call (not admitted, or
// an un-rotated matrix in another dtype than x's, or the first call under
// graph capture).
static hipError_t resident_matmul(const exl3_weight *w, WeightPriv *pv, const exl3_array &x,
                                  int xdt, int64_t rows, void *y, StreamScratch *ss, hipStream_t s,
                                  bool *taken) {
  *taken = false;
  std::lock_guard<std::mutex> g(g_res_mu);
  ResidentState &r = pv->res;
  if (!r.admitted) return hipSuccess;
  if (r.joined) {
    if (r.joined->act != x.dtype) return hipSuccess;
    *taken = true;
    const char *wj = (const char *)r.joined->data + (size_t)r.col * dt_size(x.dtype);
    return exl3::dense_gemm(x.data, xdt, wj, r.joined->cols, y, xdt, rows, pv->in, pv->out, s);
  }
  if (!holds_inner(pv)) return hipSuccess;  // the prefill GEMM is the faster path
  hipError_t e = resident_hold(w, pv, s);
  if (e == hipErrorStreamCaptureUnsupported) return hipSuccess;
  if (e != hipSuccess) return e;
  *taken = true;
  const size_t xp_bytes = ((size_t)rows * pv->in * 2 + 255) & ~(size_t)255;
  e = grow(ss, &ss->xp, &ss->xp_bytes, xp_bytes + (size_t)rows * pv->out * 2, s);
  if (e != hipSuccess) return e;
  uint16_t *xp = (uint16_t *)ss->xp;
  uint16_t *z = (uint16_t *)((char *)ss->xp + xp_bytes);
  const size_t xsz = dt_size(x.dtype);
  for (int64_t r0 = 0; r0 < rows && e == hipSuccess; r0 += 65535) {
    const int n = (int)std::min<int64_t>(65535, rows - r0);
    e = exl3::launch_prepare((const char *)x.data + (size_t)r0 * pv->in * xsz, xdt,
                             (const uint16_t *)w->scales.data, xp + (size_t)r0 * pv->in, n,
                             (int)pv->in, s);
  }
  if (e == hipSuccess)
    e = exl3::dense_gemm(xp, exl3::DENSE_F16, r.inner, pv->out, z, exl3::DENSE_F16, rows, pv->in,
                         pv->out, s);
  for (int64_t r0 = 0; r0 < rows && e == hipSuccess; r0 += 65535) {
    const int n = (int)std::min<int64_t>(65535, rows - r0);
    e = exl3::launch_finish(z + (size_t)r0 * pv->out, (const uint16_t *)w->biases.data,
                            (char *)y + (size_t)r0 * pv->out * xsz, xdt, n, (int)pv->out, s);
  }
  return e;
}

void exl3_release(exl3_weight *w) {
  if (!w) return;
  WeightPriv *pv = priv_of(w);
  if (pv) {
    std::lock_guard<std::mutex> g(g_res_mu);
    if (g_resident.erase(pv)) resident_drop(pv);
  }
  if (pv && !pv->borrowed) free_weight_arrays(w);
  delete pv;
  std::memset(w, 0, sizeof(*w));
}

static bool out_release(void *p);  // the output pool (below)

void exl3_array_free(exl3_array *a) {
  if (a && a->owned && a->data) {
    if (!out_release(a->data)) (void)hipFree(a->data);
    a->data = nullptr;
    a->owned = 0;
  }
}

exl3_verdict exl3_weight_wrap(exl3_array trellis, exl3_array suh, exl3_array svh,
                              exl3_str block_json, int32_t device, exl3_weight *out) {
  if (!out) return refuse(EXL3_FAILED, "turboexl3_mi355x: null argument");
  Block blk;
  if (block_json.ptr && block_json.len) {
    blk = parse_block(parse(block_json));
    if (blk.codebook < 0) return refuse(EXL3_UNSUPPORTED, "turboexl3_mi355x: Exl3CodebookUnsupported");
    if (blk.window < 0) return refuse(EXL3_UNSUPPORTED, "turboexl3_mi355x: Exl3WindowUnsupported");
    if (blk.table_refusal) return refuse(EXL3_UNSUPPORTED, blk.table_refusal);
  }
  const bool bank = trellis.ndim == 4;
  if (!(trellis.ndim == 3 || bank) || !trellis.data || !suh.data || !svh.data) return kShape;
  if (trellis.dtype != EXL3_DT_U16 && trellis.dtype != EXL3_DT_I16) return kDtype;
  if (suh.dtype != EXL3_DT_F16 || svh.dtype != EXL3_DT_F16) return kDtype;
  const int o = bank ? 1 : 0;
  const int64_t it = trellis.shape[o], ot = trellis.shape[o + 1], n = trellis.shape[o + 2];
  if (!n_ok(n)) return kRate;
  uint32_t row[4] = {0, 0, 0, 0};
  if (blk.table && !codebook_row(*blk.table, (int)n, row))
    return refuse(EXL3_UNSUPPORTED, "turboexl3_mi355x: Exl3CodebookTableRateMissing");
  const int64_t E = bank ? trellis.shape[0] : 0;
  if (bank) {
    if (suh.ndim != 2 || svh.ndim != 2 || suh.shape[0] != E || svh.shape[0] != E) return kShape;
    if (suh.shape[1] != it * 16 || svh.shape[1] != ot * 16) return kShape;
  } else {
    if (suh.ndim != 1 || svh.ndim != 1 || suh.shape[0] != it * 16 || svh.shape[0] != ot * 16)
      return kShape;
  }
  if ((it * 16) % 128 != 0 || (ot * 16) % 128 != 0) return kShape;
  exl3_weight w{};
  w.w = trellis;
  w.w.owned = 0;
  w.scales = suh;
  w.scales.owned = 0;
  w.biases = svh;
  w.biases.owned = 0;
  WeightPriv *pv = new WeightPriv;
  pv->f.n = (int)n;
  pv->f.codebook = blk.codebook == PACK_MCG     ? exl3::CB_FORM_MCG
                   : blk.codebook == PACK_PAIR1 ? exl3::CB_FORM_PAIR1
                   : blk.codebook >= PACK_SPEC1 ? exl3::CB_FORM_HASH
                                                : exl3::CB_FORM_MUL1;
  std::memcpy(pv->f.row, row, sizeof(row));
  pv->f.window = blk.window;
  pv->in = it * 16;
  pv->out = ot * 16;
  pv->experts = E;
  pv->device = device;
  pv->borrowed = true;
  w.priv = pv;
  *out = w;
  return ok();
}

// Allocates the output array when the caller passed none; checks it otherwise.
// ------------------------------------------------------- output arrays
//
// The reference's entries hand back a new array the caller owns
// (quant.zig:41-50); here exl3_array_free gives its memory to a pool of the
// (device, stream) the array was made for, and the next call on that
// stream that makes an array of a size the pool holds (up to twice the
// request) takes it without hipMalloc.  Work on the stream is ordered, so a
// reused block's earlier readers on it have run; a caller that read the
// array on another stream synchronizes before freeing it (as with a
// stream-ordered allocator).  Each stream's pool holds at most
// OUT_POOL_BYTES (beyond it the oldest blocks go back to the driver);
// exl3_scratch_release empties the stream's pool.
struct OutBlock {
  void *p;
  size_t bytes;
};
struct OutPool {
  std::vector<OutBlock> free;  // oldest first
  size_t held = 0;
};
constexpr size_t OUT_POOL_BYTES = (size_t)1 << 30;
std::mutex g_out_mu;
std::map<std::pair<int, hipStream_t>, OutPool> g_out_pools;
struct OutLive {
  int device;
  hipStream_t s;
  size_t bytes;
};
std::map<void *, OutLive> g_out_live;  // arrays handed out, not freed yet

static void *out_alloc(int device, hipStream_t s, size_t bytes) {
  bytes = (std::max<size_t>(bytes, 256) + 255) & ~(size_t)255;
  {
    std::lock_guard<std::mutex> g(g_out_mu);
    OutPool &pool = g_out_pools[{device, s}];
    size_t best = pool.free.size();
    for (size_t i = 0; i < pool.free.size(); ++i) {
      const size_t b = pool.free[i].bytes;
      if (b >= bytes && b <= 2 * bytes && (best == pool.free.size() || b < pool.free[best].bytes))
        best = i;
    }
    if (best < pool.free.size()) {
      const OutBlock blk = pool.free[best];
      pool.free.erase(pool.free.begin() + (std::ptrdiff_t)best);
      pool.held -= blk.bytes;
      g_out_live[blk.p] = OutLive{device, s, blk.bytes};
      return blk.p;
    }
  }
  void *p = nullptr;
  if (hipMalloc(&p, bytes) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> g(g_out_mu);
  g_out_live[p] = OutLive{device, s, bytes};
  return p;
}

// Returns p to its stream's pool; false if p is not an array of the pool's.
static bool out_release(void *p) {
  std::vector<void *> drop;
  {
    std::lock_guard<std::mutex> g(g_out_mu);
    auto it = g_out_live.find(p);
    if (it == g_out_live.end()) return false;
    const OutLive l = it->second;
    g_out_live.erase(it);
    OutPool &pool = g_out_pools[{l.device, l.s}];
    pool.free.push_back(OutBlock{p, l.bytes});
    pool.held += l.bytes;
    while (pool.held > OUT_POOL_BYTES && !pool.free.empty()) {
      drop.push_back(pool.free.front().p);
      pool.held -= pool.free.front().bytes;
      pool.free.erase(pool.free.begin());
    }
  }
  for (void *q : drop) (void)hipFree(q);
  return true;
}

// Empties (device, stream)'s pool (the caller has synchronized the stream).
static void out_pool_drop(int device, hipStream_t s) {
  std::vector<OutBlock> blocks;
  {
    std::lock_guard<std::mutex> g(g_out_mu);
    auto it = g_out_pools.find({device, s});
    if (it == g_out_pools.end()) return;
    blocks.swap(it->second.free);
    g_out_pools.erase(it);
  }
  for (const OutBlock &b : blocks) (void)hipFree(b.p);
}

static exl3_verdict output_for(exl3_array *out, const exl3_array &x, int64_t last,
                               int64_t rows, int device, hipStream_t s) {
  if (out->data == nullptr) {
    void *p = out_alloc(device, s, (size_t)(rows * last) * dt_size(x.dtype));
    if (p == nullptr) return refuse(EXL3_TOO_LARGE, "turboexl3_mi355x: out of device memory");
    exl3_array a = x;
    a.data = p;
    a.shape[a.ndim - 1] = last;
    a.owned = 1;
    *out = a;
    return ok();
  }
  if (out->dtype != x.dtype || out->ndim < 1 || out->shape[out->ndim - 1] != last ||
      numel(*out) != rows * last)
    return kShape;
  return ok();
}

// The partial-sum floats one GEMV launch over linears of widths outs[] needs.
static size_t gemv_slot_need(const int *outs, int count, int in, int rows, bool generic) {
  int total = 0;
  for (int i = 0; i < count; ++i) total += outs[i];
  int ksplit, tps;
  exl3::gemv_multi_plan(in, total, generic, rows, &ksplit, &tps);
  return (size_t)ksplit * rows * total;
}

// The scratch of one GEMV launch over `count` linears, carved from a slot
// buffer with room for gemv_slot_need: its status word, and partial sums
// split per linear.
static void gemv_carve(const exl3::Scratch &slots, const int *outs, int count, int in, int rows,
                       bool generic, exl3::Scratch *sc) {
  int total = 0;
  for (int i = 0; i < count; ++i) total += outs[i];
  int ksplit, tps;
  exl3::gemv_multi_plan(in, total, generic, rows, &ksplit, &tps);
  size_t po = 0;
  for (int i = 0; i < count; ++i) {
    sc[i].partial = slots.partial + po;
    sc[i].partial_floats = (size_t)ksplit * rows * outs[i];
    sc[i].status = slots.status;
    po += sc[i].partial_floats;
  }
}

static hipError_t gemv_scratch(StreamScratch *ss, const int *outs, int count, int in, int rows,
                               bool generic, exl3::Scratch *sc, hipStream_t s) {
  exl3::Scratch slots;
  hipError_t e = slots_for(ss, gemv_slot_need(outs, count, in, rows, generic), s, &slots);
  if (e != hipSuccess) return e;
  gemv_carve(slots, outs, count, in, rows, generic, sc);
  return hipSuccess;
}

// Linears ws[0..count) over `rows` rows of the same input: x raw (xdt,
// prepared in the kernels) or already prepared (f16), to finished outputs
// ys[i] (ydt) or, with ys null, inner products zs[i] (f16).  Up to 16 rows
// take the GEMV, one launch per 16 rows for all the linears; wider calls of
// an integer rate take the GEMM per linear after one prepare launch (other
// rates take the GEMV 16 rows at a time).
static hipError_t run_linears(const exl3_weight *const *ws, const WeightPriv *const *pvs, int count,
                              const void *x, int xdt, bool prepared, void *const *ys, int ydt,
                              uint16_t *const *zs, int64_t rows, StreamScratch *ss, hipStream_t s) {
  const WeightPriv *p0 = pvs[0];
  const int in = (int)p0->in;
  const size_t xsz = prepared ? 2 : (xdt == exl3::ACT_F32 ? 4 : 2);
  const size_t ysz = ydt == exl3::ACT_F32 ? 4 : 2;
  if (rows > exl3::GEMV_ROWS_MAX && p0->f.gemm_rate()) {
    for (int i = 0; i < count; ++i) {
      const uint16_t *xp = (const uint16_t *)x;
      if (!prepared) {
        hipError_t e = grow(ss, &ss->xp, &ss->xp_bytes, (size_t)rows * in * 2, s);
        if (e != hipSuccess) return e;
        for (int64_t r0 = 0; r0 < rows; r0 += 65535) {
          const int r = (int)std::min<int64_t>(65535, rows - r0);
          e = exl3::launch_prepare((const char *)x + (size_t)r0 * in * xsz, xdt,
                                   (const uint16_t *)ws[i]->scales.data,
                                   (uint16_t *)ss->xp + (size_t)r0 * in, r, in, s);
          if (e != hipSuccess) return e;
        }
        xp = (const uint16_t *)ss->xp;
      }
      const size_t kpf = exl3::gemm_kpart_floats(rows, in, (int)pvs[i]->out);
      if (kpf > 0) {
        hipError_t e = grow(ss, &ss->kpart, &ss->kpart_bytes, kpf * 4, s);
        if (e != hipSuccess) return e;
      }
      hipError_t e = exl3::launch_gemm(
          (const uint16_t *)ws[i]->w.data, pvs[i]->f, xp, (const uint16_t *)ws[i]->biases.data,
          ys ? ys[i] : nullptr, ydt, zs ? zs[i] : nullptr, (int)rows, in, (int)pvs[i]->out,
          (float *)ss->kpart, ss->kpart_bytes / 4, s);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  int outs[4];
  for (int i = 0; i < count; ++i) outs[i] = (int)pvs[i]->out;
  for (int64_t r0 = 0; r0 < rows; r0 += exl3::GEMV_ROWS_MAX) {
    const int r = (int)std::min<int64_t>(exl3::GEMV_ROWS_MAX, rows - r0);
    exl3::Scratch sc[4];
    hipError_t e = gemv_scratch(ss, outs, count, in, r, !p0->f.integer_rate(), sc, s);
    if (e != hipSuccess) return e;
    exl3::GemvLinear ls[4];
    for (int i = 0; i < count; ++i) {
      ls[i].trellis = (const uint16_t *)ws[i]->w.data;
      ls[i].suh = (const uint16_t *)ws[i]->scales.data;
      ls[i].svh = (const uint16_t *)ws[i]->biases.data;
      ls[i].y = ys ? (char *)ys[i] + (size_t)r0 * outs[i] * ysz : nullptr;
      ls[i].zout = zs ? zs[i] + (size_t)r0 * outs[i] : nullptr;
      ls[i].out = outs[i];
    }
    e = exl3::launch_gemv_multi(ls, count, p0->f, (const char *)x + (size_t)r0 * in * xsz, xdt,
                                prepared, ydt, r, in, sc, s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

static hipError_t run_linear(const exl3_weight *w, const WeightPriv *pv, const void *x, int xdt,
                             bool prepared, void *y, int ydt, uint16_t *zout, int64_t rows,
                             StreamScratch *ss, hipStream_t s) {
  void *ys[1] = {y};
  uint16_t *zs[1] = {zout};
  return run_linears(&w, &pv, 1, x, xdt, prepared, y ? ys : nullptr, ydt, zout ? zs : nullptr, rows,
                     ss, s);
}

// A grouped linear (G linears stored as a G-bank): x [..., G, in] ->
// y [..., G, out], x[..., g, :] through linear g (turboexl3_ds41/plugin.zig:
// 252-261; sushi_ds41/src/sushi/exl3/linear.zig:24-36).  Prompt rows (above
// 16, integer rates): x read in place, one prepare launch for every group
// (row r g of the flattened [rows G, in] takes group g's suh), one grouped
// GEMM launch over every group's 256-row tiles with the finish fused, y
// written in place (turboexl3_ds41/src/woa_join.zig:1-5: one prepare and
// one finish launch for all groups).  Otherwise per group: its rows gathered
// into scratch by a strided 2-D copy, the linear's kernels (GEMV or GEMM by
// the row count, as exl3_matmul), the result copied into y's group columns.
static exl3_verdict grouped_matmul(const exl3_weight *w, const WeightPriv *pv, exl3_array x,
                                   hipStream_t s, exl3_array *out) {
  const int xdt = act_of(x.dtype);
  if (xdt < 0) return kDtype;
  const int64_t G = pv->groups, in = pv->in, outf = pv->out;
  if (x.ndim < 2 || !x.data || x.shape[x.ndim - 1] != in || x.shape[x.ndim - 2] != G) return kShape;
  const int64_t rows = numel(x) / (G * in);
  if (rows <= 0 || rows > (int64_t)1 << 24) return kShape;
  if (hipSetDevice(pv->device) != hipSuccess) return hip_failed(hipErrorInvalidDevice);
  exl3_verdict v = output_for(out, x, outf, rows * G, pv->device, s);
  if (v.code != EXL3_OK) return v;
  const size_t esz = dt_size(x.dtype);
  StreamScratch *ss = scratch_for(pv->device, s);
  std::lock_guard<std::mutex> lk(ss->mu);
  const int64_t slots = rows * G;
  if (rows > exl3::GEMV_ROWS_MAX && pv->f.integer_rate() &&
      (uint64_t)slots * in * 2 <= 0xFFFFFFFFull && G * ((rows + 255) / 256) <= 65535) {
    hipError_t e = grow(ss, &ss->xp, &ss->xp_bytes, (size_t)slots * in * 2, s);
    const int64_t chunk = 65535 - 65535 % G;  // prepare windows of whole rows
    for (int64_t r0 = 0; r0 < slots && e == hipSuccess; r0 += chunk)
      e = exl3::launch_prepare((const char *)x.data + (size_t)r0 * in * esz, xdt,
                               (const uint16_t *)w->scales.data, (uint16_t *)ss->xp + (size_t)r0 * in,
                               (int)std::min<int64_t>(chunk, slots - r0), (int)in, s, (int)G);
    if (e == hipSuccess)
      e = exl3::launch_gemm_groups((const uint16_t *)w->w.data, pv->f, (const uint16_t *)ss->xp,
                                   (const uint16_t *)w->biases.data, out->data, xdt, (int)rows,
                                   (int)G, (int)in, (int)outf, s);
    return e == hipSuccess ? ok() : hip_failed(e);
  }
  const size_t xg_bytes = ((size_t)rows * in * esz + 255) & ~(size_t)255;
  hipError_t e = grow(ss, &ss->aux, &ss->aux_bytes, xg_bytes + (size_t)rows * outf * esz, s);
  if (e != hipSuccess) return hip_failed(e);
  char *xg = (char *)ss->aux, *yg = xg + xg_bytes;
  const size_t per = (size_t)(in / 16) * (outf / 16) * pv->f.n;  // trellis halfwords per linear
  WeightPriv pg = *pv;
  pg.experts = 0;
  pg.groups = 0;
  for (int64_t g = 0; g < G && e == hipSuccess; ++g) {
    exl3_weight wg = *w;
    wg.w.data = (uint16_t *)w->w.data + g * per;
    wg.scales.data = (uint16_t *)w->scales.data + g * in;
    wg.biases.data = (uint16_t *)w->biases.data + g * outf;
    wg.flags = 0;
    wg.priv = &pg;
    e = hipMemcpy2DAsync(xg, in * esz, (const char *)x.data + g * in * esz, G * in * esz, in * esz,
                         rows, hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess) e = run_linear(&wg, &pg, xg, xdt, false, yg, xdt, nullptr, rows, ss, s);
    if (e == hipSuccess)
      e = hipMemcpy2DAsync((char *)out->data + g * outf * esz, G * outf * esz, yg, outf * esz,
                           outf * esz, rows, hipMemcpyDeviceToDevice, s);
  }
  return e == hipSuccess ? ok() : hip_failed(e);
}

exl3_verdict exl3_matmul(const exl3_weight *w, exl3_array x, exl3_stream stream,
                         exl3_array *out) {
  const WeightPriv *pv = priv_of(w);
  if (!pv || !out) return refuse(EXL3_FAILED, "turboexl3_mi355x: null argument");
  if (pv->groups != 0) return grouped_matmul(w, pv, x, (hipStream_t)stream, out);
  if (pv->experts != 0) return refuse(EXL3_UNSUPPORTED, "turboexl3_mi355x: matmul of an expert bank");
  const int xdt = act_of(x.dtype);
  if (xdt < 0) return kDtype;
  if (x.ndim < 1 || x.ndim > EXL3_MAX_DIMS || !x.data || x.shape[x.ndim - 1] != pv->in) return kShape;
  const int64_t rows = numel(x) / pv->in;
  if (rows <= 0 || rows > (int64_t)1 << 24) return kShape;
  hipStream_t s = (hipStream_t)stream;
  if (hipSetDevice(pv->device) != hipSuccess) return hip_failed(hipErrorInvalidDevice);
  exl3_verdict v = output_for(out, x, pv->out, rows, pv->device, s);
  if (v.code != EXL3_OK) return v;
  StreamScratch *ss = scratch_for(pv->device, s);
  std::lock_guard<std::mutex> g(ss->mu);
  if (rows > exl3::GEMV_ROWS_MAX && pv->res.admitted) {
    bool taken = false;
    hipError_t e = resident_matmul(w, const_cast<WeightPriv *>(pv), x, xdt, rows, out->data, ss,
                                   s, &taken);
    if (e != hipSuccess) return hip_failed(e);
    if (taken) return ok();
  }
  hipError_t e = run_linear(w, pv, x.data, xdt, false, out->data, xdt, nullptr, rows, ss, s);
  if (e != hipSuccess) return hip_failed(e);
  return ok();
}

// exl3_matmul's kernels over exl3_matmul_noalloc's per-device array: the
// call's needs are checked against the array's regions first, and the
// fixed scratch refuses (never allocates) if a launch asked for more.
static std::mutex g_noalloc_mu;

exl3_verdict exl3_matmul_noalloc(const exl3_weight *w, exl3_array x, exl3_stream stream,
                                 exl3_array out) {
  const WeightPriv *pv = priv_of(w);
  if (!pv) return refuse(EXL3_FAILED, "turboexl3_mi355x: null argument");
  if (pv->groups != 0)
    return refuse(EXL3_UNSUPPORTED, "turboexl3_mi355x: a grouped linear takes exl3_matmul");
  if (pv->experts != 0) return refuse(EXL3_UNSUPPORTED, "turboexl3_mi355x: matmul of an expert bank");
  const int xdt = act_of(x.dtype);
  if (xdt < 0) return kDtype;
  if (x.ndim < 1 || x.ndim > EXL3_MAX_DIMS || !x.data || x.shape[x.ndim - 1] != pv->in) return kShape;
  const int64_t rows = numel(x) / pv->in;
  if (rows <= 0 || rows > (int64_t)1 << 24) return kShape;
  if (out.data == nullptr)
    return refuse(EXL3_FAILED,
                  "turboexl3_mi355x: the no-alloc matmul writes into the caller's output (out.data "
                  "is NULL)");
  if (out.dtype != x.dtype || out.ndim < 1 || out.shape[out.ndim - 1] != pv->out ||
      numel(out) != rows * pv->out)
    return kShape;
  // what run_linears will ask of the scratch
  const bool gemm = rows > exl3::GEMV_ROWS_MAX && pv->f.gemm_rate();
  size_t slot_floats = 0, xp_bytes = 0, kpart_bytes = 0;
  if (gemm) {
    xp_bytes = ((size_t)rows * pv->in * 2 + 255) & ~(size_t)255;
    kpart_bytes = exl3::gemm_kpart_floats(rows, (int)pv->in, (int)pv->out) * 4;
  } else {
    const int outs[1] = {(int)pv->out};
    slot_floats = gemv_slot_need(outs, 1, (int)pv->in,
                                 (int)std::min<int64_t>(rows, exl3::GEMV_ROWS_MAX),
                                 !pv->f.integer_rate());
  }
  if (exl3::SLOT_HEADER_BYTES + slot_floats * 4 > exl3::NOALLOC_SLOT_BYTES ||
      xp_bytes + kpart_bytes > exl3::NOALLOC_BYTES - exl3::NOALLOC_SLOT_BYTES)
    return refuse(EXL3_TOO_LARGE,
                  "turboexl3_mi355x: the call needs more scratch than the no-alloc matmul's 64 MiB "
                  "per device (8 MiB of split-K slots, 56 MiB of prepared rows and split-K "
                  "planes); exl3_matmul serves it");
  hipStream_t s = (hipStream_t)stream;
  if (hipSetDevice(pv->device) != hipSuccess) return hip_failed(hipErrorInvalidDevice);
  std::lock_guard<std::mutex> g(g_noalloc_mu);
  void *base = nullptr;
  hipError_t e = exl3::noalloc_scratch(pv->device, s, &base);
  if (e == hipErrorStreamCaptureUnsupported)
    return refuse(EXL3_FAILED,
                  "turboexl3_mi355x: the no-alloc matmul's first call on a device sets up its "
                  "array and must run outside graph capture");
  if (e != hipSuccess) return hip_failed(e);
  StreamScratch ss;
  ss.fixed = true;
  ss.slots = base;
  ss.slot_bytes = exl3::NOALLOC_SLOT_BYTES;
  char *staging = (char *)base + exl3::NOALLOC_SLOT_BYTES;
  ss.xp = staging;
  ss.xp_bytes = xp_bytes;
  ss.kpart = staging + xp_bytes;
  ss.kpart_bytes = exl3::NOALLOC_BYTES - exl3::NOALLOC_SLOT_BYTES - xp_bytes;
  e = run_linear(w, pv, x.data, xdt, false, out.data, xdt, nullptr, rows, &ss, s);
  if (e == hipErrorOutOfMemory)
    return refuse(EXL3_TOO_LARGE, "turboexl3_mi355x: the no-alloc matmul's scratch is too small");
  if (e != hipSuccess) return hip_failed(e);
  return ok();
}

exl3_verdict exl3_matmul_shared(const exl3_weight *const *ws, uint32_t count, exl3_array x,
                                exl3_stream stream, exl3_array *outs) {
  if (!ws || !outs || count < 1 || count > 4) return refuse(EXL3_FAILED, "turboexl3_mi355x: null argument");
  const WeightPriv *pvs[4];
  for (uint32_t i = 0; i < count; ++i) {
    pvs[i] = priv_of(ws[i]);
    if (!pvs[i]) return refuse(EXL3_FAILED, "turboexl3_mi355x: null argument");
    if (pvs[i]->experts != 0) return refuse(EXL3_UNSUPPORTED, "turboexl3_mi355x: matmul of an expert bank");
    if (pvs[i]->in != pvs[0]->in || pvs[i]->f.n != pvs[0]->f.n ||
        !pvs[i]->f.same_decode(pvs[0]->f) || pvs[i]->device != pvs[0]->device)
      return refuse(EXL3_UNSUPPORTED, "turboexl3_mi355x: shared linears differ in input, rate or codebook");
  }
  const int xdt = act_of(x.dtype);
  if (xdt < 0) return kDtype;
  const int64_t in = pvs[0]->in;
  if (x.ndim < 1 || x.ndim > EXL3_MAX_DIMS || !x.data || x.shape[x.ndim - 1] != in) return kShape;
  const int64_t rows = numel(x) / in;
  if (rows <= 0 || rows > (int64_t)1 << 24) return kShape;
  hipStream_t s = (hipStream_t)stream;
  if (hipSetDevice(pvs[0]->device) != hipSuccess) return hip_failed(hipErrorInvalidDevice);
  void *ys[4];
  for (uint32_t i = 0; i < count; ++i) {
    exl3_verdict v = output_for(&outs[i], x, pvs[i]->out, rows, pvs[0]->device, s);
    if (v.code != EXL3_OK) return v;
    ys[i] = outs[i].data;
  }
  StreamScratch *ss = scratch_for(pvs[0]->device, s);
  std::lock_guard<std::mutex> g(ss->mu);
  hipError_t e = run_linears(ws, pvs, (int)count, x.data, xdt, false, ys, xdt, nullptr, rows, ss, s);
  if (e != hipSuccess) return hip_failed(e);
  return ok();
}

exl3_verdict exl3_moe(const exl3_weight *bank, exl3_array x, exl3_array lhs, exl3_array rhs,
                      bool sorted, exl3_stream s, exl3_array *out) {
  (void)bank;
  (void)x;
  (void)lhs;
  (void)rhs;
  (void)sorted;
  (void)s;
  (void)out;
  return refuse(EXL3_UNSUPPORTED, "turboexl3_mi355x: routed experts run through swiglu");
}

exl3_verdict exl3_swiglu(const exl3_weight *gate, const exl3_weight *up, const exl3_weight *down,
                         exl3_array x, exl3_array inds, exl3_array scores,
                         const exl3_swiglu_opts *opts, exl3_stream stream, exl3_array *out) {
  const WeightPriv *pg = priv_of(gate), *pu = priv_of(up), *pd = priv_of(down);
  if (!pg || !pu || !pd || !out || !opts) return refuse(EXL3_FAILED, "turboexl3_mi355x: null argument");
  const int xdt = act_of(x.dtype);
  if (xdt < 0) return kDtype;
  if (x.ndim < 1 || !x.data) return kShape;
  const int64_t hidden = x.shape[x.ndim - 1];
  const int64_t rows = numel(x) / std::max<int64_t>(hidden, 1);
  if (opts->limit < 0 || opts->limit > 128)
    return refuse(EXL3_UNSUPPORTED, "turboexl3_mi355x: InvalidExl3Clamp");
  if (pg->in != hidden || pu->in != hidden || pd->out != hidden || pg->out != pu->out ||
      pd->in != pg->out)
    return kShape;
  if (pg->experts != pu->experts || pg->experts != pd->experts) return kShape;
  if (pg->groups || pu->groups || pd->groups)
    return refuse(EXL3_UNSUPPORTED, "turboexl3_mi355x: a grouped linear is not an expert bank");
  hipStream_t s = (hipStream_t)stream;
  if (hipSetDevice(pg->device) != hipSuccess) return hip_failed(hipErrorInvalidDevice);
  exl3::MoeArgs a{};
  a.x = x.data;
  a.xdt = xdt;
  a.rows = (int)rows;
  a.hidden = (int)hidden;
  a.inter = (int)pg->out;
  a.limit = (float)opts->limit;
  a.verify_rows = opts->verify_rows;
  a.experts = (int)std::max<int64_t>(pg->experts, 1);
  if (inds.data == nullptr) {
    // No routes: the dense SwiGLU MLP of single-linear weights
    // (turboexl3_ds41/plugin.zig:270-276): one expert, score 1.
    if (pg->experts != 0) return kShape;
    a.inds = nullptr;
    a.scores = nullptr;
    a.topk = 1;
  } else {
    if (pg->experts == 0) return kShape;
    if (inds.dtype != EXL3_DT_I32 && inds.dtype != EXL3_DT_U32) return kDtype;
    const int sdt = act_of(scores.dtype);
    if (sdt < 0 || !scores.data) return kDtype;
    if (inds.ndim < 1 || scores.ndim != inds.ndim) return kShape;
    for (int i = 0; i < inds.ndim; ++i)
      if (inds.shape[i] != scores.shape[i]) return kShape;
    const int64_t topk = inds.shape[inds.ndim - 1];
    if (topk <= 0 || topk > 32 || numel(inds) != rows * topk) return kShape;
    a.inds = (const uint32_t *)inds.data;
    a.scores = scores.data;
    a.sdt = sdt;
    a.topk = (int)topk;
  }
  if (pg->f.n != pu->f.n) return kRate;
  exl3_verdict v = output_for(out, x, hidden, rows, pg->device, s);
  if (v.code != EXL3_OK) return v;
  if (inds.data == nullptr && rows <= exl3::GEMV_ROWS_MAX && pg->f.same_decode(pu->f)) {
    // Dense MLP at decode sizes: gate and up in one GEMV launch (f16), then
    // the down GEMV with the SwiGLU applied as it prepares its rows (the MoE
    // path's mid step, bit for bit): two launches (above 4 rows the SwiGLU
    // runs once on its own first).
    StreamScratch *ss = scratch_for(pg->device, s);
    std::lock_guard<std::mutex> g(ss->mu);
    const size_t nel = (size_t)rows * pg->out;
    hipError_t e = grow(ss, &ss->moe, &ss->moe_bytes, nel * 3 * sizeof(uint16_t), s);
    if (e != hipSuccess) return hip_failed(e);
    uint16_t *gu = (uint16_t *)ss->moe;
    const exl3_weight *ws2[2] = {gate, up};
    const WeightPriv *pv2[2] = {pg, pu};
    void *ys[2] = {gu, gu + nel};
    e = run_linears(ws2, pv2, 2, x.data, xdt, false, ys, exl3::ACT_F16, nullptr, rows, ss, s);
    if (e != hipSuccess) return hip_failed(e);
    const int outs[1] = {(int)hidden};
    exl3::Scratch sc;
    e = gemv_scratch(ss, outs, 1, (int)pd->in, (int)rows, !pd->f.integer_rate(), &sc, s);
    if (e != hipSuccess) return hip_failed(e);
    const exl3::GemvLinear l{(const uint16_t *)down->w.data, (const uint16_t *)down->scales.data,
                             (const uint16_t *)down->biases.data, out->data, nullptr, (int)hidden};
    e = exl3::launch_gemv_swiglu(l, pd->f, gu, gu + nel, gu + 2 * nel, (float)opts->limit, xdt,
                                 (int)rows, (int)pd->in, sc, s);
    if (e != hipSuccess) {
      if (e == hipErrorInvalidValue) return kShape;
      return hip_failed(e);
    }
    return ok();
  }
  if (inds.data == nullptr && pg->f.gemm_rate() && pu->f.gemm_rate() && pd->f.gemm_rate()) {
    // Dense MLP of more rows (prefill, a shared expert at large batches):
    // gate and up through the GEMM (f16), the SwiGLU once (the MoE path's mid
    // step, bit for bit), the down projection through the GEMM.
    StreamScratch *ss = scratch_for(pg->device, s);
    std::lock_guard<std::mutex> g(ss->mu);
    const size_t nel = (size_t)rows * pg->out;
    hipError_t e = grow(ss, &ss->moe, &ss->moe_bytes, nel * 3 * sizeof(uint16_t), s);
    if (e != hipSuccess) return hip_failed(e);
    uint16_t *gu = (uint16_t *)ss->moe;
    const exl3_weight *ws2[2] = {gate, up};
    const WeightPriv *pv2[2] = {pg, pu};
    void *ys[2] = {gu, gu + nel};
    e = run_linears(ws2, pv2, 2, x.data, xdt, false, ys, exl3::ACT_F16, nullptr, rows, ss, s);
    if (e == hipSuccess) e = exl3::launch_swiglu(gu, gu + nel, gu + 2 * nel, nel, (float)opts->limit, s);
    const exl3_weight *wd[1] = {down};
    const WeightPriv *pvd[1] = {pd};
    void *yd[1] = {out->data};
    if (e == hipSuccess)
      e = run_linears(wd, pvd, 1, gu + 2 * nel, exl3::ACT_F16, false, yd, xdt, nullptr, rows, ss, s);
    if (e != hipSuccess) {
      if (e == hipErrorInvalidValue) return kShape;
      return hip_failed(e);
    }
    return ok();
  }
  a.y = out->data;
  a.ydt = xdt;
  exl3::MoeBank bg{(const uint16_t *)gate->w.data, (const uint16_t *)gate->scales.data,
                   (const uint16_t *)gate->biases.data, pg->f, (int)pg->in, (int)pg->out};
  exl3::MoeBank bu{(const uint16_t *)up->w.data, (const uint16_t *)up->scales.data,
                   (const uint16_t *)up->biases.data, pu->f, (int)pu->in, (int)pu->out};
  exl3::MoeBank bd{(const uint16_t *)down->w.data, (const uint16_t *)down->scales.data,
                   (const uint16_t *)down->biases.data, pd->f, (int)pd->in, (int)pd->out};
  StreamScratch *ss = scratch_for(pg->device, s);
  std::lock_guard<std::mutex> g(ss->mu);
  // A launch orders at most MOE_SLOTS_MAX slots (rows x topk): a larger call
  // (a long prompt's prefill) runs as windows of whole rows, one launch
  // sequence each, in row order on the stream over the same scratch.  Rows
  // are independent, so the windows' results are the rows' results.
  const int64_t wrows = std::max<int64_t>(1, exl3::MOE_SLOTS_MAX / a.topk);
  exl3::MoeArgs wa = a;
  wa.rows = (int)std::min<int64_t>(rows, wrows);
  size_t pf = 0;
  const size_t need =
      exl3::moe_scratch_bytes(wa, !pg->f.integer_rate(), !pd->f.integer_rate(), &pf);
  hipError_t e = grow(ss, &ss->moe, &ss->moe_bytes, need, s);
  if (e != hipSuccess) return hip_failed(e);
  exl3::Scratch slots;
  e = slots_for(ss, pf, s, &slots);
  if (e != hipSuccess) return hip_failed(e);
  const size_t xsz = xdt == exl3::ACT_F32 ? 4 : 2;
  const size_t ssz = a.inds ? (a.sdt == exl3::ACT_F32 ? 4 : 2) : 0;
  for (int64_t r0 = 0; r0 < rows && e == hipSuccess; r0 += wrows) {
    wa.rows = (int)std::min<int64_t>(rows - r0, wrows);
    wa.x = (const char *)a.x + (size_t)r0 * hidden * xsz;
    wa.y = (char *)a.y + (size_t)r0 * hidden * xsz;
    if (a.inds) {
      wa.inds = a.inds + (size_t)r0 * a.topk;
      wa.scores = (const char *)a.scores + (size_t)r0 * a.topk * ssz;
    }
    e = exl3::launch_moe(wa, bg, bu, bd, ss->moe, ss->moe_bytes, slots, s);
  }
  if (e != hipSuccess) {
    if (e == hipErrorInvalidValue) return kShape;
    return hip_failed(e);
  }
  return ok();
}

// The routed experts and the gated shared expert in the same launches: the
// routes gain a slot per row for the shared expert (an index past the bank's,
// score sigmoid(logit)), which the routed GEMV launches, the mid step and the
// weighted sum serve like any expert (quant.zig:94-97,183-197).
exl3_verdict exl3_swiglu_shared(const exl3_weight *gate, const exl3_weight *up,
                                const exl3_weight *down, exl3_array x, exl3_array inds,
                                exl3_array scores, const exl3_shared_swiglu *opts,
                                exl3_stream stream, exl3_array *out) {
  const WeightPriv *pg = priv_of(gate), *pu = priv_of(up), *pd = priv_of(down);
  if (!pg || !pu || !pd || !out || !opts) return refuse(EXL3_FAILED, "turboexl3_mi355x: null argument");
  if (opts->size < (uint32_t)sizeof(exl3_shared_swiglu))
    return refuse(EXL3_FAILED, "turboexl3_mi355x: SharedSwiglu older than this library's");
  const WeightPriv *sg = single_linear(opts->gate), *su = single_linear(opts->up),
                   *sd = single_linear(opts->down);
  if (!sg || !su || !sd)
    return refuse(EXL3_FAILED, "turboexl3_mi355x: the shared expert's linears are missing");
  const int xdt = act_of(x.dtype);
  if (xdt < 0) return kDtype;
  if (x.ndim < 1 || !x.data) return kShape;
  const int64_t hidden = x.shape[x.ndim - 1];
  const int64_t rows = numel(x) / std::max<int64_t>(hidden, 1);
  if (rows <= 0) return kShape;
  if (pg->experts == 0 || pg->experts != pu->experts || pg->experts != pd->experts ||
      pg->groups || pu->groups || pd->groups)
    return kShape;
  if (pg->in != hidden || pu->in != hidden || pd->out != hidden || pg->out != pu->out ||
      pd->in != pg->out)
    return kShape;
  auto same = [](const WeightPriv *a, const WeightPriv *b) {
    return a->in == b->in && a->out == b->out && a->f.n == b->f.n &&
           a->f.same_decode(b->f) && a->device == b->device;
  };
  if (!same(sg, pg) || !same(su, pu) || !same(sd, pd) || pg->f.n != pu->f.n ||
      !pg->f.same_decode(pu->f))
    return refuse(EXL3_UNSUPPORTED,
                  "turboexl3_mi355x: the shared expert differs from the routed experts in width, "
                  "rate or codebook (the host runs its chain)");
  const int64_t E = pg->experts;
  // routes: given, or from the router's logits
  int64_t k = 0;
  int sdt = exl3::ACT_F32;
  const bool from_logits = opts->logits.data != nullptr;
  if (from_logits) {
    if (inds.data || scores.data) return kShape;
    k = opts->k;
    if (opts->logits.dtype != x.dtype) return kDtype;
    if (k <= 0 || k > 31 || k > E || opts->logits.ndim < 1 ||
        opts->logits.shape[opts->logits.ndim - 1] != E || numel(opts->logits) != rows * E)
      return kShape;
  } else {
    if (!inds.data || !scores.data) return kShape;
    if (inds.dtype != EXL3_DT_I32 && inds.dtype != EXL3_DT_U32) return kDtype;
    sdt = act_of(scores.dtype);
    if (sdt < 0) return kDtype;
    k = inds.shape[inds.ndim - 1];
    if (k <= 0 || k > 31 || numel(inds) != rows * k || numel(scores) != rows * k) return kShape;
  }
  // the shared gate's logit: given per row, or the dot with gate_vec
  if (opts->logit.data) {
    if (opts->logit.dtype != x.dtype || numel(opts->logit) != rows) return kShape;
  } else if (opts->gate_vec.data) {
    if (opts->gate_vec.dtype != x.dtype || numel(opts->gate_vec) != hidden) return kShape;
  } else {
    return refuse(EXL3_FAILED, "turboexl3_mi355x: the shared gate needs logit or gate_vec");
  }
  hipStream_t s = (hipStream_t)stream;
  if (hipSetDevice(pg->device) != hipSuccess) return hip_failed(hipErrorInvalidDevice);
  exl3::MoeArgs a{};
  a.x = x.data;
  a.xdt = xdt;
  a.rows = (int)rows;
  a.hidden = (int)hidden;
  a.inter = (int)pg->out;
  a.limit = 0.0f;  // the table SwiGLU, unclamped (turboexl3_qwen38/src/direct/moe.zig:215-220)
  a.experts = (int)E + 1;
  a.topk = (int)k + 1;
  a.sdt = exl3::ACT_F32;
  StreamScratch *ss = scratch_for(pg->device, s);
  std::lock_guard<std::mutex> g(ss->mu);
  // the routes with the shared slot, k + 1 per row
  const size_t routes = ((size_t)rows * (k + 1) * 4 + 255) & ~(size_t)255;
  hipError_t e = grow(ss, &ss->aux, &ss->aux_bytes, 2 * routes, s);
  if (e != hipSuccess) return hip_failed(e);
  uint32_t *r_inds = (uint32_t *)ss->aux;
  float *r_scores = (float *)((char *)ss->aux + routes);
  a.inds = r_inds;
  a.scores = r_scores;
  if (exl3::moe_uses_gemm(a, !pg->f.integer_rate(), !pd->f.integer_rate()))
    return refuse(EXL3_UNSUPPORTED,
                  "turboexl3_mi355x: the shared expert rides the routed GEMV launches; at "
                  "prefill-sized batches the host runs swiglu and its shared expert's chain");
  exl3_verdict v = output_for(out, x, hidden, rows, pg->device, s);
  if (v.code != EXL3_OK) return v;
  a.y = out->data;
  a.ydt = xdt;
  size_t pf = 0;
  const size_t need =
      exl3::moe_scratch_bytes(a, !pg->f.integer_rate(), !pd->f.integer_rate(), &pf);
  e = grow(ss, &ss->moe, &ss->moe_bytes, need, s);
  if (e != hipSuccess) return hip_failed(e);
  // one row with its routes given: the routed launches read the k routes
  // and take slot k as the shared expert, the combine forms the gate; else
  // the route launch writes the (k + 1)-wide routes first
  const bool direct = !opts->logits.data &&
                      exl3::moe_shared_direct(a, !pg->f.integer_rate(), !pd->f.integer_rate());
  if (direct) {
    a.inds = (const uint32_t *)inds.data;
    a.scores = scores.data;
    a.sdt = sdt;
  } else {
    e = exl3::launch_moe_shared_route(
        (const uint32_t *)inds.data, scores.data, sdt, opts->logits.data, (int)E, (int)k,
        opts->logit.data, opts->gate_vec.data, x.data, xdt, (int)rows, (int)hidden, r_inds,
        r_scores, s);
    if (e != hipSuccess) return e == hipErrorInvalidValue ? kShape : hip_failed(e);
  }
  exl3::Scratch slots;
  e = slots_for(ss, pf, s, &slots);
  if (e != hipSuccess) return hip_failed(e);
  auto bank = [](const exl3_weight *w, const WeightPriv *p) {
    return exl3::MoeBank{(const uint16_t *)w->w.data, (const uint16_t *)w->scales.data,
                         (const uint16_t *)w->biases.data, p->f, (int)p->in, (int)p->out};
  };
  exl3::MoeShared sh{bank(opts->gate, sg), bank(opts->up, su), bank(opts->down, sd)};
  if (direct) {
    sh.routes_k = (int)k;
    sh.logit = opts->logit.data;
    sh.gate_vec = opts->gate_vec.data;
  }
  e = exl3::launch_moe(a, bank(gate, pg), bank(up, pu), bank(down, pd), ss->moe, ss->moe_bytes,
                       slots, s, &sh);
  if (e != hipSuccess) return e == hipErrorInvalidValue ? kShape : hip_failed(e);
  return ok();
}

exl3_verdict exl3_decode_matrix(const exl3_weight *w, int32_t expert, exl3_array out,
                                exl3_stream stream) {
  const WeightPriv *pv = priv_of(w);
  if (!pv) return refuse(EXL3_FAILED, "turboexl3_mi355x: null argument");
  if (out.dtype != EXL3_DT_F16 || !out.data || numel(out) != pv->in * pv->out) return kShape;
  const int64_t E = std::max<int64_t>(pv->experts, 1);
  if (expert < 0 || expert >= E) return kShape;
  if (hipSetDevice(pv->device) != hipSuccess) return hip_failed(hipErrorInvalidDevice);
  const size_t per = (size_t)(pv->in / 16) * (pv->out / 16) * pv->f.n;
  hipError_t e = exl3::launch_decode_matrix((const uint16_t *)w->w.data + per * expert, pv->f,
                                            (int)pv->in, (int)pv->out, (uint16_t *)out.data,
                                            (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_failed(e);
}

exl3_verdict exl3_prepare(const exl3_weight *w, exl3_array x, exl3_array xp, exl3_stream stream) {
  const WeightPriv *pv = priv_of(w);
  if (!pv) return refuse(EXL3_FAILED, "turboexl3_mi355x: null argument");
  if (pv->experts != 0) return kShape;
  const int xdt = act_of(x.dtype);
  if (xdt < 0 || xp.dtype != EXL3_DT_F16) return kDtype;
  if (!x.data || !xp.data || x.ndim < 1 || x.shape[x.ndim - 1] != pv->in || numel(xp) != numel(x))
    return kShape;
  const int64_t rows = numel(x) / pv->in;
  if (hipSetDevice(pv->device) != hipSuccess) return hip_failed(hipErrorInvalidDevice);
  hipError_t e = hipSuccess;
  for (int64_t r0 = 0; r0 < rows && e == hipSuccess; r0 += 65535) {
    const int r = (int)std::min<int64_t>(65535, rows - r0);
    e = exl3::launch_prepare((const char *)x.data + (size_t)r0 * pv->in * dt_size(x.dtype), xdt,
                             (const uint16_t *)w->scales.data,
                             (uint16_t *)xp.data + (size_t)r0 * pv->in, r, (int)pv->in,
                             (hipStream_t)stream);
  }
  return e == hipSuccess ? ok() : hip_failed(e);
}

exl3_verdict exl3_finish(const exl3_weight *w, exl3_array z, exl3_array y, exl3_stream stream) {
  const WeightPriv *pv = priv_of(w);
  if (!pv) return refuse(EXL3_FAILED, "turboexl3_mi355x: null argument");
  if (pv->experts != 0) return kShape;
  const int ydt = act_of(y.dtype);
  if (ydt < 0 || z.dtype != EXL3_DT_F16) return kDtype;
  if (!z.data || !y.data || z.ndim < 1 || z.shape[z.ndim - 1] != pv->out || numel(y) != numel(z))
    return kShape;
  const int64_t rows = numel(z) / pv->out;
  if (hipSetDevice(pv->device) != hipSuccess) return hip_failed(hipErrorInvalidDevice);
  const size_t ysz = dt_size(y.dtype);
  hipError_t e = hipSuccess;
  for (int64_t r0 = 0; r0 < rows && e == hipSuccess; r0 += 65535) {
    const int r = (int)std::min<int64_t>(65535, rows - r0);
    e = exl3::launch_finish((const uint16_t *)z.data + (size_t)r0 * pv->out,
                            (const uint16_t *)w->biases.data,
                            (char *)y.data + (size_t)r0 * pv->out * ysz, ydt, r, (int)pv->out,
                            (hipStream_t)stream);
  }
  return e == hipSuccess ? ok() : hip_failed(e);
}

exl3_verdict exl3_inner(const exl3_weight *w, exl3_array xp, exl3_array z, exl3_stream stream) {
  const WeightPriv *pv = priv_of(w);
  if (!pv) return refuse(EXL3_FAILED, "turboexl3_mi355x: null argument");
  if (pv->experts != 0) return kShape;
  if (xp.dtype != EXL3_DT_F16 || z.dtype != EXL3_DT_F16) return kDtype;
  if (!xp.data || !z.data || xp.ndim < 1 || xp.shape[xp.ndim - 1] != pv->in) return kShape;
  const int64_t rows = numel(xp) / pv->in;
  if (numel(z) != rows * pv->out) return kShape;
  hipStream_t s = (hipStream_t)stream;
  if (hipSetDevice(pv->device) != hipSuccess) return hip_failed(hipErrorInvalidDevice);
  StreamScratch *ss = scratch_for(pv->device, s);
  std::lock_guard<std::mutex> g(ss->mu);
  hipError_t e = run_linear(w, pv, xp.data, exl3::ACT_F16, true, nullptr, 0, (uint16_t *)z.data,
                            rows, ss, s);
  return e == hipSuccess ? ok() : hip_failed(e);
}

// ------------------------------------------------ split entries (LinearParts)

// A new device array of `dt` with x's leading dims and last dimension `last`
// (2-D [rows, last] when lead is null), `extra` bytes beyond the data.
static exl3_verdict new_array(exl3_array *out, const exl3_array *lead, int64_t rows, int64_t last,
                              int dt, size_t extra, int device, hipStream_t s) {
  const size_t bytes = ((size_t)(rows * last) * dt_size(dt) + 255) & ~(size_t)255;
  void *p = out_alloc(device, s, bytes + extra);
  if (p == nullptr) return refuse(EXL3_TOO_LARGE, "turboexl3_mi355x: out of device memory");
  exl3_array a{};
  if (lead) {
    a = *lead;
    a.shape[a.ndim - 1] = last;
  } else {
    a.ndim = 2;
    a.shape[0] = rows;
    a.shape[1] = last;
  }
  a.data = p;
  a.dtype = dt;
  a.owned = 1;
  a._pad = 0;
  *out = a;
  return ok();
}

static bool parts_ok(const exl3_linear_parts *o) {
  return o && o->size >= (uint32_t)sizeof(exl3_linear_parts);
}

const exl3_verdict kParts = {EXL3_FAILED,
                             "turboexl3_mi355x: LinearParts missing or older than this library's"};

exl3_verdict exl3_linear_split(const exl3_weight *w, exl3_array x, const exl3_linear_parts *opts,
                               exl3_stream stream, exl3_array *out) {
  const WeightPriv *pv = single_linear(w);
  if (!pv || !out) return refuse(EXL3_FAILED, "turboexl3_mi355x: null argument or not one linear");
  if (!parts_ok(opts)) return kParts;
  const int xdt = act_of(x.dtype);
  if (xdt < 0) return kDtype;
  if (x.ndim < 1 || !x.data || x.shape[x.ndim - 1] != pv->in) return kShape;
  const int64_t rows = numel(x) / pv->in;
  if (rows <= 0 || rows > (int64_t)1 << 24) return kShape;
  hipStream_t s = (hipStream_t)stream;
  hipStream_t side = opts->side ? (hipStream_t)opts->side : s;
  if (hipSetDevice(pv->device) != hipSuccess) return hip_failed(hipErrorInvalidDevice);
  const int odt = opts->inner ? (int)EXL3_DT_F16 : (int)x.dtype;
  // with a side stream the prepared rows ride behind the result in its allocation
  const size_t xp_bytes = side != s ? (size_t)rows * pv->in * 2 : 0;
  exl3_verdict v = new_array(out, &x, rows, pv->out, odt, xp_bytes, pv->device, s);
  if (v.code != EXL3_OK) return v;
  void *y = opts->inner ? nullptr : out->data;
  uint16_t *z = opts->inner ? (uint16_t *)out->data : nullptr;
  hipError_t e = hipSuccess;
  if (side == s) {
    StreamScratch *ss = scratch_for(pv->device, s);
    std::lock_guard<std::mutex> g(ss->mu);
    e = run_linear(w, pv, x.data, xdt, false, y, xdt, z, rows, ss, s);
  } else {
    const size_t ybytes = ((size_t)(rows * pv->out) * dt_size(odt) + 255) & ~(size_t)255;
    uint16_t *xp = (uint16_t *)((char *)out->data + ybytes);
    for (int64_t r0 = 0; r0 < rows && e == hipSuccess; r0 += 65535) {
      const int r = (int)std::min<int64_t>(65535, rows - r0);
      e = exl3::launch_prepare((const char *)x.data + (size_t)r0 * pv->in * dt_size(x.dtype), xdt,
                               (const uint16_t *)w->scales.data, xp + (size_t)r0 * pv->in, r,
                               (int)pv->in, s);
    }
    hipEvent_t ev = nullptr;
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(ev, s);
    if (e == hipSuccess) e = hipStreamWaitEvent(side, ev, 0);
    if (ev) (void)hipEventDestroy(ev);
    if (e == hipSuccess) {
      StreamScratch *ss = scratch_for(pv->device, side);
      std::lock_guard<std::mutex> g(ss->mu);
      e = run_linear(w, pv, xp, exl3::ACT_F16, true, y, xdt, z, rows, ss, side);
    }
  }
  if (e != hipSuccess) {
    exl3_array_free(out);
    return hip_failed(e);
  }
  return ok();
}

exl3_verdict exl3_linear_finish(const exl3_weight *w, const exl3_linear_parts *opts,
                                exl3_stream stream, exl3_array *out) {
  const WeightPriv *pv = single_linear(w);
  if (!pv || !out) return refuse(EXL3_FAILED, "turboexl3_mi355x: null argument or not one linear");
  if (!parts_ok(opts)) return kParts;
  const int ydt = act_of(opts->dtype);
  if (ydt < 0) return kDtype;
  if (opts->parts.len == 0 || !opts->parts.ptr) return kShape;
  int64_t rows = 0;
  for (size_t i = 0; i < opts->parts.len; ++i) {
    const exl3_array &z = opts->parts.ptr[i];
    if (z.dtype != EXL3_DT_F16) return kDtype;
    if (!z.data || z.ndim < 1 || z.shape[z.ndim - 1] != pv->out) return kShape;
    rows += numel(z) / pv->out;
  }
  if (rows <= 0 || rows > (int64_t)1 << 24) return kShape;
  hipStream_t s = (hipStream_t)stream;
  if (hipSetDevice(pv->device) != hipSuccess) return hip_failed(hipErrorInvalidDevice);
  exl3_verdict v = new_array(out, nullptr, rows, pv->out, opts->dtype, 0, pv->device, s);
  if (v.code != EXL3_OK) return v;
  const size_t ysz = dt_size(opts->dtype);
  hipError_t e = hipSuccess;
  int64_t at = 0;
  for (size_t i = 0; i < opts->parts.len && e == hipSuccess; ++i) {
    const exl3_array &z = opts->parts.ptr[i];
    const int64_t n = numel(z) / pv->out;
    for (int64_t r0 = 0; r0 < n && e == hipSuccess; r0 += 65535) {
      const int r = (int)std::min<int64_t>(65535, n - r0);
      e = exl3::launch_finish((const uint16_t *)z.data + (size_t)r0 * pv->out,
                              (const uint16_t *)w->biases.data,
                              (char *)out->data + (size_t)(at + r0) * pv->out * ysz, ydt, r,
                              (int)pv->out, s);
    }
    at += n;
  }
  if (e != hipSuccess) {
    exl3_array_free(out);
    return hip_failed(e);
  }
  return ok();
}

exl3_verdict exl3_linear_prepared(const exl3_weight *w, exl3_array xp,
                                  const exl3_linear_parts *opts, exl3_stream stream,
                                  exl3_array *out) {
  const WeightPriv *pv = single_linear(w);
  if (!pv || !out) return refuse(EXL3_FAILED, "turboexl3_mi355x: null argument or not one linear");
  if (!parts_ok(opts)) return kParts;
  const int ydt = act_of(opts->dtype);
  if (ydt < 0 || xp.dtype != EXL3_DT_F16) return kDtype;
  if (xp.ndim < 1 || !xp.data || xp.shape[xp.ndim - 1] != pv->in) return kShape;
  const int64_t rows = numel(xp) / pv->in;
  if (rows <= 0 || rows > (int64_t)1 << 24) return kShape;
  hipStream_t s = (hipStream_t)stream;
  if (hipSetDevice(pv->device) != hipSuccess) return hip_failed(hipErrorInvalidDevice);
  exl3_verdict v = new_array(out, &xp, rows, pv->out, opts->dtype, 0, pv->device, s);
  if (v.code != EXL3_OK) return v;
  StreamScratch *ss = scratch_for(pv->device, s);
  std::lock_guard<std::mutex> g(ss->mu);
  hipError_t e = run_linear(w, pv, xp.data, exl3::ACT_F16, true, out->data, ydt, nullptr, rows, ss, s);
  if (e != hipSuccess) {
    exl3_array_free(out);
    return hip_failed(e);
  }
  return ok();
}

// The kernel path of a call of `rows` rows (run_linears' choice).
static bool gemm_path(const WeightPriv *pv, int64_t rows) {
  return rows > exl3::GEMV_ROWS_MAX && pv->f.gemm_rate();
}

exl3_verdict exl3_linear_pieces(const exl3_weight *w, const exl3_linear_parts *opts,
                                exl3_stream stream, exl3_array *out) {
  (void)stream;
  const WeightPriv *pv = single_linear(w);
  if (!pv || !out) return refuse(EXL3_FAILED, "turboexl3_mi355x: null argument or not one linear");
  if (!parts_ok(opts)) return kParts;
  if (act_of(opts->dtype) < 0) return kDtype;
  if (opts->rows.len == 0 || !opts->rows.ptr) return kShape;
  int64_t total = 0;
  for (size_t i = 0; i < opts->rows.len; ++i) {
    if (opts->rows.ptr[i] == 0) return kShape;
    total += opts->rows.ptr[i];
  }
  const bool whole = gemm_path(pv, total);
  for (size_t i = 0; i < opts->rows.len; ++i)
    if (gemm_path(pv, opts->rows.ptr[i]) != whole)
      return refuse(EXL3_UNSUPPORTED,
                    "turboexl3_mi355x: a piece takes another kernel path (GEMV / GEMM) than the "
                    "whole call");
  *out = w->w;  // the packed trellis, borrowed: the pieces' kernels decode it
  out->owned = 0;
  return ok();
}

exl3_verdict exl3_linear_piece(const exl3_weight *w, exl3_array x, const exl3_linear_parts *opts,
                               exl3_stream stream, exl3_array *out) {
  const WeightPriv *pv = single_linear(w);
  if (!pv || !out) return refuse(EXL3_FAILED, "turboexl3_mi355x: null argument or not one linear");
  if (!parts_ok(opts)) return kParts;
  if (opts->held.data != w->w.data)
    return refuse(EXL3_FAILED, "turboexl3_mi355x: held is not what linear_pieces made for this weight");
  const int xdt = opts->prepared ? (int)exl3::ACT_F16 : act_of(x.dtype);
  if (xdt < 0 || (opts->prepared && x.dtype != EXL3_DT_F16)) return kDtype;
  if (x.ndim < 1 || !x.data || x.shape[x.ndim - 1] != pv->in) return kShape;
  const int64_t rows = numel(x) / pv->in;
  if (rows <= 0 || rows > (int64_t)1 << 24) return kShape;
  hipStream_t s = (hipStream_t)stream;
  if (hipSetDevice(pv->device) != hipSuccess) return hip_failed(hipErrorInvalidDevice);
  exl3_verdict v = new_array(out, &x, rows, pv->out, EXL3_DT_F16, 0, pv->device, s);
  if (v.code != EXL3_OK) return v;
  StreamScratch *ss = scratch_for(pv->device, s);
  std::lock_guard<std::mutex> g(ss->mu);
  hipError_t e = run_linear(w, pv, x.data, xdt, opts->prepared, nullptr, 0, (uint16_t *)out->data,
                            rows, ss, s);
  if (e != hipSuccess) {
    exl3_array_free(out);
    return hip_failed(e);
  }
  return ok();
}

exl3_verdict exl3_scratch_release(int32_t device, exl3_stream stream) {
  hipStream_t s = (hipStream_t)stream;
  StreamScratch *ss = nullptr;
  {
    std::lock_guard<std::mutex> g(g_scratch_mu);
    auto it = g_scratch.find({device, s});
    if (it != g_scratch.end()) ss = &it->second;
  }
  if (hipSetDevice(device) != hipSuccess) return hip_failed(hipErrorInvalidDevice);
  if (capturing(s))
    return refuse(EXL3_FAILED, "turboexl3_mi355x: scratch released while its stream is being captured");
  std::unique_lock<std::mutex> g;
  if (ss) g = std::unique_lock<std::mutex>(ss->mu);
  hipError_t e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_failed(e);
  out_pool_drop(device, s);  // the freed output arrays the stream's calls kept
  if (!ss) return ok();
  for (void **p : {&ss->xp, &ss->kpart, &ss->slots, &ss->moe, &ss->aux}) {
    if (*p) (void)hipFree(*p);
    *p = nullptr;
  }
  ss->xp_bytes = ss->kpart_bytes = ss->slot_bytes = ss->moe_bytes = ss->aux_bytes = 0;
  for (void *p : ss->retired) (void)hipFree(p);
  ss->retired.clear();
  for (auto &b : ss->retired_slots) (void)hipFree(b.first);
  ss->retired_slots.clear();
  return ok();
}

void exl3_set_splitk_poll_bound(int32_t polls) { exl3::set_splitk_poll_max(polls); }

void exl3_set_splitk_test_drop(int32_t on) { exl3::set_splitk_drop(on); }

exl3_verdict exl3_stream_status(int32_t device, exl3_stream stream) {
  hipStream_t s = (hipStream_t)stream;
  StreamScratch *ss = nullptr;
  {
    std::lock_guard<std::mutex> g(g_scratch_mu);
    auto it = g_scratch.find({device, s});
    if (it != g_scratch.end()) ss = &it->second;
  }
  if (hipSetDevice(device) != hipSuccess) return hip_failed(hipErrorInvalidDevice);
  if (capturing(s))
    return refuse(EXL3_FAILED, "turboexl3_mi355x: status read while its stream is being captured");
  std::unique_lock<std::mutex> g;
  if (ss) g = std::unique_lock<std::mutex>(ss->mu);
  hipError_t e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_failed(e);
  // the device's no-alloc array (exl3_matmul_noalloc) has a status word too
  bool failed = false;
  e = exl3::noalloc_status(device, &failed);
  if (e != hipSuccess) return hip_failed(e);
  std::vector<std::pair<void *, size_t>> bufs;
  if (ss) {
    bufs = ss->retired_slots;
    if (ss->slots) bufs.push_back({ss->slots, ss->slot_bytes});
  }
  for (auto &b : bufs) {
    uint32_t st = 0;
    e = hipMemcpy(&st, b.first, 4, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_failed(e);
    if (st == 0) continue;
    failed = true;
    // the stream is idle, so every late store has landed: empty the slots
    e = hipMemset((char *)b.first + exl3::SLOT_HEADER_BYTES, 0xFF,
                  b.second - exl3::SLOT_HEADER_BYTES);
    if (e == hipSuccess) e = hipMemset(b.first, 0, 4);
    if (e != hipSuccess) return hip_failed(e);
  }
  if (failed)
    return refuse(EXL3_FAILED,
                  "turboexl3_mi355x: a split-K partial sum did not arrive within the wait's bound; "
                  "outputs of this stream's calls since the last check may hold NaN (the slots "
                  "are reset)");
  return ok();
}

const char *exl3_version(void) { return "exl3_mi355x 0.2.0 (gfx950)"; }

const char *exl3_matmul_path(const exl3_weight *w, int64_t rows) {
  const WeightPriv *pv = priv_of(w);
  if (!pv) return "none";
  if (pv->groups != 0)  // rows: rows of each group
    return rows > exl3::GEMV_ROWS_MAX && pv->f.integer_rate() ? "gemm-groups" : "per-group";
  if (rows <= exl3::GEMV_ROWS_MAX) return "gemv";
  return pv->f.gemm_rate() ? "gemm" : "gemv";
}

const char *exl3_swiglu_path(const exl3_weight *gate, const exl3_weight *up,
                             const exl3_weight *down, int64_t rows, int32_t topk,
                             bool verify_rows) {
  const WeightPriv *pg = priv_of(gate), *pu = priv_of(up), *pd = priv_of(down);
  if (!pg || !pu || !pd || rows <= 0) return "none";
  if (topk <= 0) {
    if (rows <= exl3::GEMV_ROWS_MAX && pg->f.same_decode(pu->f)) return "dense-gemv";
    if (pg->f.gemm_rate() && pu->f.gemm_rate() && pd->f.gemm_rate()) return "dense-gemm";
    return "dense-items";
  }
  exl3::MoeArgs a{};
  a.rows = (int)rows;
  a.topk = (int)topk;
  a.experts = (int)std::max<int64_t>(pg->experts, 1);
  a.inds = reinterpret_cast<const uint32_t *>(&a);  // routed: any non-null
  a.verify_rows = verify_rows;
  return exl3::moe_uses_gemm(a, !pg->f.integer_rate(), !pd->f.integer_rate()) ? "routed-gemm"
                                                                              : "routed-gemv";
}

// QuantTable.resident (quant.zig:98-99): admits ws' single linears, whose
// decoded matrices (W_inner f16, in * out * 2 bytes each) are then held from
// each one's first prefill-width matmul on; *bytes = what ws' matrices take.
// Refused too_large past room (0: no bound), admitting none of them; an
// empty ws drops every kept matrix.
exl3_verdict exl3_resident(exl3_weight_span ws, uint64_t room, exl3_stream stream,
                           uint64_t *bytes) {
  (void)stream;
  if (!bytes || (ws.len && !ws.ptr)) return refuse(EXL3_FAILED, "turboexl3_mi355x: null argument");
  std::lock_guard<std::mutex> g(g_res_mu);
  if (ws.len == 0) {
    for (WeightPriv *pv : g_resident) resident_drop(pv);
    g_resident.clear();
    *bytes = 0;
    return ok();
  }
  uint64_t total = 0;
  for (size_t i = 0; i < ws.len; ++i) {
    const WeightPriv *pv = single_linear(&ws.ptr[i]);
    if (!pv)
      return refuse(EXL3_UNSUPPORTED,
                    "turboexl3_mi355x: resident matrices are kept for single linears (banks run "
                    "through swiglu)");
    total += resident_bytes(pv);
  }
  if (room != 0 && total > room)
    return refuse(EXL3_TOO_LARGE, "turboexl3_mi355x: the decoded matrices exceed room");
  for (size_t i = 0; i < ws.len; ++i) {
    WeightPriv *pv = priv_of(&ws.ptr[i]);
    pv->res.admitted = true;
    g_resident.insert(pv);
  }
  *bytes = total;
  return ok();
}

// QuantTable.resident_pending (quant.zig:100-101): the bytes admitted and
// not held yet.
uint64_t exl3_resident_pending(void) {
  std::lock_guard<std::mutex> g(g_res_mu);
  uint64_t n = 0;
  for (const WeightPriv *pv : g_resident)
    if (pv->res.admitted && !pv->res.inner && !pv->res.joined) n += resident_bytes(pv);
  return n;
}

// QuantTable.unrotate (quant.zig:102-104): ws in groups of sizes[g] weights
// that read one input; each group's resident matrices become one public
// matrix [in, sum of outs] in `act`, members side by side in their order
// (W_public = diag(suh) H W_inner H diag(svh) / 128, the reference's
// reconstructPublic order), and each member's W_inner is freed.  took[g]:
// whether group g took -- its members admitted single linears of one input
// width and device, not yet in another group (a group already joined as
// asked takes again).  Members not yet held are decoded first.
exl3_verdict exl3_unrotate(exl3_weight_span ws, exl3_u8_span sizes, int32_t act,
                           exl3_stream stream, bool *took) {
  if ((ws.len && !ws.ptr) || (sizes.len && (!sizes.ptr || !took)))
    return refuse(EXL3_FAILED, "turboexl3_mi355x: null argument");
  const int kact = act_of(act);
  if (kact < 0) return kDtype;
  size_t n = 0;
  for (size_t g = 0; g < sizes.len; ++g) n += sizes.ptr[g];
  if (n != ws.len) return kShape;
  hipStream_t s = (hipStream_t)stream;
  std::lock_guard<std::mutex> lk(g_res_mu);
  size_t off = 0;
  for (size_t g = 0; g < sizes.len; off += sizes.ptr[g], ++g) {
    took[g] = false;
    const size_t m = sizes.ptr[g];
    if (m == 0) continue;
    std::vector<WeightPriv *> mem;
    bool fit = true;
    int64_t cols = 0;
    for (size_t i = 0; i < m && fit; ++i) {
      WeightPriv *pv = priv_of(&ws.ptr[off + i]);
      fit = single_linear(&ws.ptr[off + i]) && pv->res.admitted && pv->in == priv_of(&ws.ptr[off])->in &&
            pv->device == priv_of(&ws.ptr[off])->device;
      if (fit) {
        mem.push_back(pv);
        cols += pv->out;
      }
    }
    if (!fit) continue;
    // already this group, in this dtype: it takes again
    const std::shared_ptr<Joined> j0 = mem[0]->res.joined;
    if (j0 && j0->act == act && j0->members == mem) {
      took[g] = true;
      continue;
    }
    bool free_members = true;
    for (WeightPriv *pv : mem) free_members = free_members && !pv->res.joined;
    if (!free_members) continue;
    if (hipSetDevice(mem[0]->device) != hipSuccess) return hip_failed(hipErrorInvalidDevice);
    hipError_t e = hipSuccess;
    for (size_t i = 0; i < m && e == hipSuccess; ++i) e = resident_hold(&ws.ptr[off + i], mem[i], s);
    if (e != hipSuccess) return hip_failed(e);
    auto j = std::make_shared<Joined>();
    j->act = act;
    j->in = mem[0]->in;
    j->cols = cols;
    j->device = mem[0]->device;
    e = hipMalloc(&j->data, (size_t)j->in * cols * dt_size(act));
    if (e != hipSuccess) return hip_failed(e);
    int64_t col = 0;
    for (size_t i = 0; i < m && e == hipSuccess; ++i) {
      const exl3_weight &w = ws.ptr[off + i];
      e = exl3::launch_unrotate(mem[i]->res.inner, (const uint16_t *)w.scales.data,
                                (const uint16_t *)w.biases.data, (int)j->in, (int)mem[i]->out,
                                (char *)j->data + (size_t)col * dt_size(act), cols, kact, s);
      col += mem[i]->out;
    }
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
      (void)hipFree(j->data);
      return hip_failed(e);
    }
    col = 0;
    for (WeightPriv *pv : mem) {
      (void)hipFree(pv->res.inner);
      pv->res.inner = nullptr;
      pv->res.joined = j;
      pv->res.col = col;
      col += pv->out;
    }
    j->members = mem;
    took[g] = true;
  }
  return ok();
}

// QuantTable.linear_joined (quant.zig:105-107): x [..., in] times the joined
// public matrix of the un-rotated group whose members are ws, in order:
// [..., sum of outs] in x's dtype (the group's `act`).  Refused where the
// members are not such a group (not un-rotated, another order, a part of
// one) and at decode widths (up to 16 rows: the EXL3 GEMV serves them).
exl3_verdict exl3_linear_joined(exl3_weight_span ws, exl3_array x, exl3_stream stream,
                                exl3_array *out) {
  if (!out || ws.len == 0 || !ws.ptr) return refuse(EXL3_FAILED, "turboexl3_mi355x: null argument");
  std::shared_ptr<Joined> j;
  {
    std::lock_guard<std::mutex> lk(g_res_mu);
    j = priv_of(&ws.ptr[0]) ? priv_of(&ws.ptr[0])->res.joined : nullptr;
    bool same = j && j->members.size() == ws.len;
    for (size_t i = 0; same && i < ws.len; ++i) same = priv_of(&ws.ptr[i]) == j->members[i];
    if (!same)
      return refuse(EXL3_UNSUPPORTED,
                    "turboexl3_mi355x: linear_joined takes an un-rotated group's members in order");
  }
  const int xdt = act_of(x.dtype);
  if (xdt < 0 || x.dtype != j->act) return kDtype;
  if (x.ndim < 1 || !x.data || x.shape[x.ndim - 1] != j->in) return kShape;
  const int64_t rows = numel(x) / j->in;
  if (rows <= 0 || rows > (int64_t)1 << 24) return kShape;
  if (rows <= exl3::GEMV_ROWS_MAX)
    return refuse(EXL3_UNSUPPORTED,
                  "turboexl3_mi355x: linear_joined at decode widths (the EXL3 GEMV serves them)");
  if (hipSetDevice(j->device) != hipSuccess) return hip_failed(hipErrorInvalidDevice);
  exl3_verdict v = output_for(out, x, j->cols, rows, j->device, (hipStream_t)stream);
  if (v.code != EXL3_OK) return v;
  const hipError_t e = exl3::dense_gemm(x.data, xdt, j->data, j->cols, out->data, xdt, rows, j->in,
                                        j->cols, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_failed(e);
}

static exl3_verdict register_kernels(const void *host) {
  (void)host;
  return ok();
}

#define EXL3_TABLE_ENTRIES                                                       \
  &exl3_validate, &exl3_bill, &exl3_open, &exl3_close, &exl3_load_tensor, &exl3_load_bank, \
      &exl3_release, &exl3_matmul, &exl3_moe, &register_kernels, &exl3_swiglu,           \
      &exl3_linear_split, &exl3_linear_finish, &exl3_linear_prepared, &exl3_linear_pieces, \
      &exl3_linear_piece, nullptr /* attn_in: the host's chain */, nullptr /* attn_prep */, \
      nullptr /* linear_prepared_idx */, nullptr /* gated_out */,                        \
      nullptr /* merged_gated_out */, nullptr /* q_planes */, nullptr /* indexer */,       \
      &exl3_swiglu_shared, &exl3_resident, &exl3_resident_pending, &exl3_unrotate,        \
      &exl3_linear_joined

// The two tables differ only in their claim: ds41's rule (kTable) and
// qwen38's (kTableQwen38, under its own name).
static const exl3_quant_table kTable = {
    (uint32_t)sizeof(exl3_quant_table), EXL3_ABI_VERSION, {kName, 16}, &exl3_claims,
    EXL3_TABLE_ENTRIES};
static const exl3_quant_table kTableQwen38 = {
    (uint32_t)sizeof(exl3_quant_table), EXL3_ABI_VERSION, {kNameQwen38, 23}, &exl3_claims_qwen38,
    EXL3_TABLE_ENTRIES};
#undef EXL3_TABLE_ENTRIES

const exl3_quant_table *exl3_quant_table_get(void) { return &kTable; }
const exl3_quant_table *exl3_quant_table_qwen38_get(void) { return &kTableQwen38; }

}  // extern "C"

// ------------------------------------------------ decode-step fused linears

int exl3d_linears(const exl3_weight *const *ws, int count, const void *x, int B,
                  const uint16_t *norm_w, const float *nssq, float eps, const uint16_t *up,
                  float *res, float *res_ssq, uint16_t *const *outs, hipStream_t s) {
  if (!ws || !x || count < 1 || count > 4 || B < 1 || B > exl3::GEMV_ROWS_MAX) return -1;
  if ((norm_w != nullptr) != (nssq != nullptr) || (norm_w && up)) return -1;
  if (res && (count != 1 || !res_ssq)) return -1;
  const WeightPriv *pvs[4];
  for (int i = 0; i < count; ++i) {
    pvs[i] = priv_of(ws[i]);
    if (!pvs[i] || pvs[i]->experts != 0) return -1;
    if (pvs[i]->in != pvs[0]->in || pvs[i]->f.n != pvs[0]->f.n ||
        !pvs[i]->f.same_decode(pvs[0]->f) || pvs[i]->device != pvs[0]->device)
      return -1;
    if (!res && (!outs || !outs[i])) return -1;
  }
  if (hipSetDevice(pvs[0]->device) != hipSuccess) return hipErrorInvalidDevice;
  const int in = (int)pvs[0]->in;
  StreamScratch *ss = scratch_for(pvs[0]->device, s);
  std::lock_guard<std::mutex> g(ss->mu);
  int wouts[4];
  exl3::GemvLinear ls[4];
  for (int i = 0; i < count; ++i) {
    wouts[i] = (int)pvs[i]->out;
    ls[i].trellis = (const uint16_t *)ws[i]->w.data;
    ls[i].suh = (const uint16_t *)ws[i]->scales.data;
    ls[i].svh = (const uint16_t *)ws[i]->biases.data;
    ls[i].y = outs ? outs[i] : nullptr;
    ls[i].zout = nullptr;
    ls[i].out = wouts[i];
  }
  exl3::Scratch sc[4];
  hipError_t e = gemv_scratch(ss, wouts, count, in, B, !pvs[0]->f.integer_rate(), sc, s);
  if (e != hipSuccess) return e;
  exl3::GemvFuse fz;
  fz.up = up;
  fz.nssq = nssq;
  fz.norm_w = norm_w;
  fz.eps = eps;
  fz.res = res;
  fz.res_ssq = res_ssq;
  int xdt = norm_w ? exl3::ACT_F32 : exl3::ACT_F16;
  int total = 0;
  for (int i = 0; i < count; ++i) total += wouts[i];
  const bool pre_norm = norm_w && (!exl3::gemv_one_batch(in, total, !pvs[0]->f.integer_rate(), B) ||
                                   in / 128 > exl3::NORM_MAXBLK);
  const bool pre_swiglu = up && B > exl3::SWIGLU_PROLOGUE_ROWS;
  // rows the prologue does not take: the RMSNorm (of h as it stands) or the
  // SwiGLU first, with each weight's prepare in the same pass where the
  // shapes allow (every column group of the GEMV would otherwise redo the
  // prepare of its k-slice for all rows), into scratch as stacked prepared
  // rows; else the plain rows, then a GEMV that prepares them
  const bool prep_norm = pre_norm && in % 512 == 0 && in <= 8192;
  const bool prep_swiglu = pre_swiglu && count == 1 && in % 128 == 0;
  if (prep_norm || prep_swiglu) {
    const int sets = prep_norm ? count : 1;
    e = grow(ss, &ss->xp, &ss->xp_bytes, (size_t)sets * B * in * sizeof(uint16_t), s);
    if (e != hipSuccess) return e;
    uint16_t *xs = (uint16_t *)ss->xp;
    if (prep_norm) {
      const uint16_t *suhs[4];
      for (int i = 0; i < count; ++i) suhs[i] = ls[i].suh;
      e = exl3::launch_rmsnorm_prepare((const float *)x, norm_w, B, in, eps, suhs, count, xs, s);
      fz.nssq = nullptr;
      fz.norm_w = nullptr;
    } else {
      e = exl3::launch_swiglu_prepare((const uint16_t *)x, up, ls[0].suh, xs, B, in, 0.0f, s);
      fz.up = nullptr;
    }
    if (e != hipSuccess) return e;
    fz.stacked = true;
    x = xs;
    xdt = exl3::ACT_F16;
  } else if (pre_norm || pre_swiglu) {
    e = grow(ss, &ss->xp, &ss->xp_bytes, (size_t)B * in * sizeof(uint16_t), s);
    if (e != hipSuccess) return e;
    uint16_t *xs = (uint16_t *)ss->xp;
    if (pre_norm) {
      const int r = exl3d_add_rmsnorm((float *)x, nullptr, norm_w, xs, B, in, eps, s);
      if (r != 0) return r;
      fz.nssq = nullptr;
      fz.norm_w = nullptr;
    } else {
      e = exl3::launch_swiglu((const uint16_t *)x, up, xs, (size_t)B * in, 0.0f, s);
      if (e != hipSuccess) return e;
      fz.up = nullptr;
    }
    x = xs;
    xdt = exl3::ACT_F16;
  }
  e = exl3::launch_gemv_fused(ls, count, pvs[0]->f, x, xdt, exl3::ACT_F16, B, in, sc, fz, s);
  if (e == hipErrorInvalidValue) return -1;
  return e;
}

int exl3d_attn_o(const uint16_t *q, const uint16_t *k, const uint16_t *v, const uint16_t *qn,
                 const uint16_t *kn, const int32_t *pos, int B, int nq, int nkv, float eps,
                 float theta, uint16_t *kcache, uint16_t *vcache, int Tmax, float scale,
                 const exl3_weight *o, float *res, float *res_ssq, uint16_t *att, float *scratch,
                 size_t scratch_bytes, hipStream_t s) {
  const WeightPriv *pv = priv_of(o);
  if (!pv || pv->experts != 0 || !res || !res_ssq || B < 1 || B > exl3::GEMV_ROWS_MAX) return -1;
  const int G = exl3d_attn_heads_per_kv();
  const int ns = exl3d_attn_splits(B, nkv, Tmax);
  if (ns < 1 || nq != G * nkv || pv->in != (int64_t)nq * EXL3D_HEAD_DIM) return -1;
  const bool fused = exl3::gemv_one_batch((int)pv->in, (int)pv->out, !pv->f.integer_rate(), B);
  if (!fused && !att) return -1;
  if (hipSetDevice(pv->device) != hipSuccess) return hipErrorInvalidDevice;
  int r = exl3d_attn_decode_rope(q, k, v, qn, kn, pos, B, nq, nkv, eps, theta, kcache, vcache,
                                 Tmax, scale, nullptr, scratch, scratch_bytes, s);
  if (r != 0) return r;
  const int in = (int)pv->in;
  if (!fused) {
    // the combine writes att as o's prepared rows, so o's column groups do
    // not each redo the prepare of their k-slice for all rows
    hipError_t e = exl3::launch_attn_combine_prepare(scratch, B, nq, nkv, Tmax,
                                                     (const uint16_t *)o->scales.data, att, s);
    if (e != hipSuccess) return e;
    StreamScratch *ss = scratch_for(pv->device, s);
    std::lock_guard<std::mutex> g(ss->mu);
    int wout = (int)pv->out;
    exl3::GemvLinear l;
    l.trellis = (const uint16_t *)o->w.data;
    l.suh = (const uint16_t *)o->scales.data;
    l.svh = (const uint16_t *)o->biases.data;
    l.y = nullptr;
    l.zout = nullptr;
    l.out = wout;
    exl3::Scratch sc;
    e = gemv_scratch(ss, &wout, 1, in, B, !pv->f.integer_rate(), &sc, s);
    if (e != hipSuccess) return e;
    exl3::GemvFuse fz;
    fz.res = res;
    fz.res_ssq = res_ssq;
    fz.stacked = true;
    e = exl3::launch_gemv_fused(&l, 1, pv->f, att, exl3::ACT_F16, exl3::ACT_F16, B, in, &sc, fz,
                                s);
    if (e == hipErrorInvalidValue) return -1;
    return e;
  }
  StreamScratch *ss = scratch_for(pv->device, s);
  std::lock_guard<std::mutex> g(ss->mu);
  int wout = (int)pv->out;
  exl3::GemvLinear l;
  l.trellis = (const uint16_t *)o->w.data;
  l.suh = (const uint16_t *)o->scales.data;
  l.svh = (const uint16_t *)o->biases.data;
  l.y = nullptr;
  l.zout = nullptr;
  l.out = wout;
  exl3::Scratch sc;
  hipError_t e = gemv_scratch(ss, &wout, 1, in, B, !pv->f.integer_rate(), &sc, s);
  if (e != hipSuccess) return e;
  exl3::GemvFuse fz;
  fz.res = res;
  fz.res_ssq = res_ssq;
  fz.attn_part = scratch;
  fz.attn_nkv = nkv;
  fz.attn_g = G;
  fz.attn_nsplit = ns;
  e = exl3::launch_gemv_fused(&l, 1, pv->f, scratch, exl3::ACT_F16, exl3::ACT_F16, B, in, &sc, fz,
                              s);
  if (e == hipErrorInvalidValue) return -1;
  return e;
}
