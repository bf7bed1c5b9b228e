// capi.cpp -- the C ABI of the gfx950 executor: the context (device, stream,
// device arena / rodata / source images, scratch, refusal word) and the
// instruction dispatcher.
//
// seeai_execute decodes each 64-byte UpdateInstruction exactly as the
// reference CPU backend decodes it (runtime/executor/cpu_backend.cc:260-646:
// operand slots, packed dim words, flag bits, the imm word) and enqueues the
// matching HIP kernels; nothing here computes on the host except the
// per-step scalars the reference also hoists (AdamW's bias corrections,
// RoPE's frequency step), evaluated with the reference's expressions.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "../../include/seeai_hip.h"
#include "common.h"
#include "operands.h"

using namespace seeai;

namespace {

// runtime/executor/backend.h:65-80 -- the reference's shared verdicts.
const char* const kNonFiniteNormRefusal =
    "gradient norm is not finite \xe2\x80\x94 the step was refused with the parameters "
    "and optimizer state untouched";
const char* const kClipThresholdRefusal =
    "clip threshold is not a finite positive float \xe2\x80\x94 the instruction was "
    "refused with the gradient untouched";

// source/plan/instruction.h:25-42 -- reference encoding.
constexpr uint64_t kRodataBit = 1ULL << 63;
constexpr uint64_t kSourceBit = 1ULL << 62;
constexpr uint64_t kNullRef = ~0ULL;
constexpr uint64_t kArenaAlignment = 16384;  // backend.h:51

// instruction.h:311-382 -- flag bits.
constexpr uint16_t kFlagEpilogueBias = 1u << 0;
constexpr uint16_t kFlagGemmAddend = 1u << 3;
constexpr uint16_t kFlagQ8ColScale = 1u << 4;
constexpr uint16_t kFlagRelaxed = 1u << 5;

#pragma pack(push, 1)
struct Instruction {  // instruction.h:438-447
  uint16_t opcode;
  uint16_t flags;
  uint32_t imm;
  uint64_t in[4];
  uint64_t out[3];
};
#pragma pack(pop)
static_assert(sizeof(Instruction) == 64, "UpdateInstruction is one 64-byte word");

float BitsToF32(uint64_t w) {
  const uint32_t u = static_cast<uint32_t>(w);
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

constexpr size_t kSmallBytes = 4096;  // refusal word, scale slot, accuracy counts
constexpr size_t kInitialScratch = 1u << 20;      // grown on demand

// The no-allocation entry points' workspace (seeai_xent_fwd_noalloc): a
// file-scope device array each GPU holds from the library's load to the
// process's end.  Host code never uses its name as an address: the device
// address of each GPU's copy comes from hipGetSymbolAddress, taken once per
// device at seeai_create with that device current, and kept below.
constexpr size_t kNoAllocScratchBytes = size_t{2} << 20;  // 2 MiB
__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
struct NoAllocSlot {
  std::once_flag once;
  void* ptr = nullptr;       // this device's copy of `scratch`
  hipError_t status = hipSuccess;
};
NoAllocSlot g_noalloc[kMaxDevices];

// Looks the array's address up on `device` (which must be current), once.
hipError_t NoAllocScratchInit(int device) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  NoAllocSlot& slot = g_noalloc[device];
  std::call_once(slot.once, [&slot] {
    void* p = nullptr;
    slot.status = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (slot.status == hipSuccess) slot.ptr = p;
  });
  return slot.status;
}

}  // namespace

struct seeai_ctx {
  int device = 0;
  hipStream_t own_stream = nullptr;
  hipStream_t stream = nullptr;
  uint8_t* arena = nullptr;
  uint64_t arena_bytes = 0;
  uint8_t* rodata = nullptr;
  uint64_t rodata_bytes = 0;
  uint8_t* source = nullptr;
  uint64_t source_bytes = 0;
  uint8_t* small = nullptr;  // [0] refusal word, [64] scale slot, [128] two u64 counts,
                             // [256] the optimizer's step values for replayed graphs
  int* host_flag = nullptr;  // pinned
  void* scratch = nullptr;
  size_t scratch_bytes = 0;
  int allow_relaxed = 1;
  // Relaxed tiled attention on bf16 operands (the flash kernels) instead of
  // f32 products; off by default (seeai_set_attention_bf16).
  int attn_bf16 = 0;
  uint64_t relaxed = 0;
  // The program of the range being executed (seeai_begin_range, the seam's
  // BeginRange): lets two adjacent instructions run as one dispatch.
  const uint8_t* prog = nullptr;
  uint64_t prog_count = 0, range_end = 0;
  // Instructions of the range already run by a fused dispatch, in the order
  // the engine will present them (a LoRA site's t product and rank-r
  // product; the rest of a run of AdamW steps).
  const uint8_t* done[kAdamWMulti] = {};
  int ndone = 0;
  int allow_fusion = 1;
  int allow_dma = 1;  // relaxed frozen-weight GEMMs on the bf16 shadow path
  int allow_lowrank = 1;  // LoRA sites folded into the frozen product's epilogue
  int allow_dead_store_drop = 1;  // fused passes skip stores the range overwrites unread
  int allow_sinks = 1;  // producers write the next relaxed product's bf16 activation
  uint64_t dropped_stores = 0;
  uint64_t sinks = 0;  // conversions fused into their producers
  // The program `dead` was decided for: its address, length and a hash of
  // its words (a caller may present another program of the same length at
  // the same address, e.g. a temporary buffer freed and reallocated).
  const uint8_t* dead_prog = nullptr;
  uint64_t dead_hash = 0;
  uint64_t prog_hash = 0;  // of the range's program, taken at begin_range
  std::vector<int8_t> dead;  // per instruction and asking site: -1 undecided, 0 kept, 1 dropped
  TilePolicy policy;  // kernel geometry (seeai_configure)
  // The relaxed GEMMs' bf16 copy of their activations, and what it holds:
  // a later relaxed GEMM of the same range that rounds the same bytes the
  // same way reuses it when every instruction between wrote elsewhere.
  void* cvt = nullptr;
  size_t cvt_bytes = 0;
  // More copy slots, the size of the first, filled only by conversion sinks:
  // slot 0 by a producer's second sink (two outputs of one pass, each the
  // activation of one of the two relaxed products after it), slots 1 .. 3 in
  // turn by sinks whose product comes later in the range (FarSink).
  static constexpr int kXSlots = 4;
  void* xcvt[kXSlots] = {};
  size_t xcvt_bytes = 0;
  int far_next = 0;
  // Partial row maxima a GEMM epilogue left for the loss turn at `at`
  // (instruction index, this epoch): of logits C [M, N].
  float* pmax = nullptr;
  size_t pmax_bytes = 0;
  struct {
    const float* C = nullptr;
    uint64_t M = 0, N = 0, at = 0, epoch = 0;
  } pmax_key;
  // bf16 copies of relaxed attention's operands (q, k, v, dO: four slots of
  // B·S·H·64) for the bf16-operand kernels, and what they hold: the sources
  // and the instruction that converted them.
  void* a16 = nullptr;
  size_t a16_bytes = 0;
  struct A16Key {
    const float* src[4];
    uint64_t n;
    const uint8_t* at;
  } a16_key{};
  int attn16_plans = 1;  // SEEAI_ATTN16_PLANS=0: the f32-operand kernels
  // The forward's bf16 copies of q, k, v, one buffer per source triple, kept
  // for the backward of the same range run: `idx` is the converting
  // instruction, `epoch` the range run it belongs to, `clean_to` how far the
  // scan for writes into the sources has reached.
  struct A16Saved {
    const float* src[3];
    uint64_t n;
    uint64_t idx, clean_to, epoch;
    void* buf;
  };
  std::vector<A16Saved> a16_saved;
  uint64_t a16_saved_cap = uint64_t{4} << 30;  // bytes over every saved triple
  uint64_t a16_epoch = 1;
  // Operand copies a producer wrote for the attention at instruction `at`,
  // in this epoch: a RoPE forward's q or k (slots 0, 1) and a LoRA site's v
  // (slot 2) into the forward's saved copies, a LoRA site's dO (slot 3) into
  // the operand buffer's dO slot.
  struct {
    const float* src = nullptr;
    uint64_t at = 0, epoch = 0;
  } a16_pre[4];
  struct CvtKey {
    const float* A = nullptr;
    uint64_t M = 0, K = 0;
    float alpha = 0.0f;
    const float* ks = nullptr;
    const uint8_t* at = nullptr;  // the converting instruction in the range; null: none
  } cvt_key, xcvt_key[kXSlots];
  const uint8_t* cur_at = nullptr;  // the instruction being executed, when in the range
  uint64_t fused = 0;
  // bf16 copies [N, Kp] of frozen weights for the relaxed GEMMs, keyed by
  // (weight, layout, kind, N, K); valid until the next bind.
  std::map<std::tuple<const void*, int, int, uint64_t, uint64_t>, void*> shadows;
  // Whole ranges captured as HIP graphs (seeai_run_range) and replayed when
  // the same range of the same program runs again with nothing it depends
  // on changed since the capture: every binding, setting or workspace change
  // drops them (DropGraphs, which also advances graph_gen).
  struct RangeGraph {
    const uint8_t* prog = nullptr;
    uint64_t count = 0, begin = 0, end = 0, hash = 0, gen = 0;
    int runs = 0;             // eager runs so far (the first sizes the workspaces)
    bool ungraphable = false;  // its capture failed: always eager
    hipGraphExec_t exec = nullptr;
    uint64_t relaxed = 0, fused = 0, dropped = 0, sinks = 0;  // counter increments per run
  };
  std::vector<RangeGraph> graphs;
  // Off by default: on MI355X the replay measured no faster than the
  // launches it replaces (the GPU's own per-dispatch cost sets the pace of
  // these ranges, not the host's launches).
  int graph_replay = 0;
  uint64_t graph_gen = 0;
  uint64_t graph_launches = 0;
  bool capturing = false;           // the optimizer reads hyper() instead of arguments
  float* host_hyper = nullptr;      // pinned: the step's {lr, inv_bc1, inv_bc2}
  hipEvent_t hyper_copied = nullptr;
  // Captures record on a stream of their own: the context's stream keeps
  // serving other threads' event waits (the feeder's) while one is recorded.
  hipStream_t capture_stream = nullptr;
  std::string err;

  int* flag() { return reinterpret_cast<int*>(small); }
  float* scale_slot() { return reinterpret_cast<float*>(small + 64); }
  uint64_t* counts() { return reinterpret_cast<uint64_t*>(small + 128); }
  float* hyper() { return reinterpret_cast<float*>(small + 256); }
};

namespace {

int Fail(seeai_ctx* c, int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (c) c->err = buf;
  return code;
}

int Hip(seeai_ctx* c, hipError_t e, const char* what) {
  if (e == hipSuccess) return SEEAI_OK;
  return Fail(c, SEEAI_HIP_ERROR, "hip: %s: %s", what, hipGetErrorString(e));
}

#define SEEAI_TRY(ctx, expr, what)                         \
  do {                                                     \
    const int seeai_rc_ = Hip((ctx), (expr), (what));      \
    if (seeai_rc_ != SEEAI_OK) return seeai_rc_;           \
  } while (0)

// Destroys the captured range graphs (after the stream drains: one may be
// running) and advances the generation every capture is checked against.
// The arena may have changed outside the program (or the program itself):
// no bf16 copy made earlier may be taken for current.
void ForgetCopies(seeai_ctx* c) {
  c->cvt_key.at = nullptr;
  for (auto& k : c->xcvt_key) k.at = nullptr;
  c->a16_key.at = nullptr;
  ++c->a16_epoch;
}

// The forward's saved attention copies (they name the binding's pointers).
void DropSavedCopies(seeai_ctx* c) {
  for (auto& sv : c->a16_saved)
    if (sv.buf) (void)hipFree(sv.buf);
  c->a16_saved.clear();
}

void DropGraphs(seeai_ctx* c) {
  ++c->graph_gen;
  if (c->graphs.empty()) return;
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  for (auto& g : c->graphs)
    if (g.exec) (void)hipGraphExecDestroy(g.exec);
  c->graphs.clear();
}

// Scratch for reductions; grown (after draining the stream) when an op
// needs more than it holds.
int Scratch(seeai_ctx* c, size_t bytes, void** out) {
  if (bytes > c->scratch_bytes) {
    DropGraphs(c);
    SEEAI_TRY(c, hipStreamSynchronize(c->stream), "scratch drain");
    if (c->scratch) SEEAI_TRY(c, hipFree(c->scratch), "scratch free");
    c->scratch = nullptr;
    c->scratch_bytes = 0;
    size_t want = kInitialScratch;
    while (want < bytes) want *= 2;
    SEEAI_TRY(c, hipMalloc(&c->scratch, want), "scratch alloc");
    c->scratch_bytes = want;
  }
  *out = c->scratch;
  return SEEAI_OK;
}

struct Ptrs {
  seeai_ctx* c;
  uint8_t* at(uint64_t ref) const {
    const uint64_t off = ref & ~(kRodataBit | kSourceBit);
    if (ref & kRodataBit) return c->rodata + off;
    if ((ref & (kRodataBit | kSourceBit)) == kSourceBit) return c->source + off;
    return c->arena + off;
  }
  float* f(uint64_t ref) const { return reinterpret_cast<float*>(at(ref)); }
  const float* fo(uint64_t ref) const { return ref == kNullRef ? nullptr : f(ref); }
  int32_t* i32(uint64_t ref) const { return reinterpret_cast<int32_t*>(at(ref)); }
};

// The step's optimizer values {lr, 1 / (1 - beta1^t), 1 / (1 - beta2^t)}
// (optimizer.cc:115-118, evaluated on the host with the reference's powf).
void StepHyper(const seeai_step_params& P, float out[3]) {
  out[0] = P.lr;
  out[1] = 1.0f / (1.0f - std::pow(P.beta1, static_cast<float>(P.step)));
  out[2] = 1.0f / (1.0f - std::pow(P.beta2, static_cast<float>(P.step)));
}

int AdamWLaunch(seeai_ctx* c, float* p, const float* g, float* m, float* v, uint64_t n,
                const seeai_step_params& P, float clip) {
  float hy[3];
  StepHyper(P, hy);
  const float inv_bc1 = hy[1], inv_bc2 = hy[2];
  const float* scale = nullptr;
  if (clip > 0.0f) {
    void* ws;
    if (int rc = Scratch(c, 8 * 1024, &ws)) return rc;
    SEEAI_TRY(c, LaunchClipFactor(g, n, clip, c->scale_slot(), c->flag(), ws, c->stream),
              "adamw clip");
    scale = c->scale_slot();
  }
  SEEAI_TRY(c,
            LaunchAdamW(p, g, m, v, n, P.lr, P.beta1, P.beta2, P.eps, P.weight_decay, inv_bc1,
                        inv_bc2, scale, c->flag(), c->stream, c->capturing ? c->hyper() : nullptr),
            "adamw");
  return SEEAI_OK;
}

void DropShadows(seeai_ctx* c) {
  DropGraphs(c);
  for (auto& kv : c->shadows) (void)hipFree(kv.second);
  c->shadows.clear();
}

// Memory no instruction writes between binds: the rodata and source images.
bool Immutable(const seeai_ctx* c, const void* p) {
  const auto* q = static_cast<const uint8_t*>(p);
  return (c->rodata && q >= c->rodata && q < c->rodata + c->rodata_bytes) ||
         (c->source && q >= c->source && q < c->source + c->source_bytes);
}

const char* DecodeGemm(seeai_ctx* c, const Instruction& ins, GemmArgs* out);
bool Overlap(const uint8_t* a, uint64_t na, const uint8_t* b, uint64_t nb);
uint64_t CurIndex(const seeai_ctx* c);

// Whether the conversion buffer already holds this GEMM's A' (range
// fusion): the same A, shape, alpha and k-scale converted by an earlier
// instruction of this range, and every instruction between them a GEMM
// whose output misses A.  Anything else -- another opcode between, a write
// into A, a copy of the instruction word run outside the range -- converts
// again.
bool ConvertedAlready(seeai_ctx* c, const GemmArgs& a, const seeai_ctx::CvtKey& k) {
  if (!c->allow_fusion || !c->cur_at || !k.at || k.at >= c->cur_at || k.A != a.A || k.M != a.M ||
      k.K != a.K || k.alpha != a.alpha_a || k.ks != a.a_k_scale)
    return false;
  const auto* A = reinterpret_cast<const uint8_t*>(a.A);
  const uint64_t bytes = a.M * a.K * 4;
  for (const uint8_t* p = k.at + 64; p < c->cur_at; p += 64) {
    Instruction ins;
    std::memcpy(&ins, p, sizeof ins);
    GemmArgs g{};
    if (!DecodeGemm(c, ins, &g)) return false;
    if (Overlap(reinterpret_cast<const uint8_t*>(g.C), g.M * g.N * 4, A, bytes)) return false;
  }
  return true;
}

// The relaxed frozen-weight product on the bf16 direct-to-LDS kernel: the
// weight's bf16 shadow (made once), A rounded into the workspace with its
// scales, then the GEMM and its epilogue.
int GemmBf16Dma(seeai_ctx* c, GemmArgs& a, const char* what) {
  const auto key = std::make_tuple(a.B, a.layout, a.b_kind, static_cast<uint64_t>(a.N),
                                   static_cast<uint64_t>(a.K));
  void* shadow = nullptr;
  if (auto it = c->shadows.find(key); it != c->shadows.end()) {
    shadow = it->second;
  } else {
    SEEAI_TRY(c, hipMalloc(&shadow, a.N * Bf16DmaKp(a.K) * 2), "weight shadow alloc");
    c->shadows[key] = shadow;
    SEEAI_TRY(c, LaunchWeightShadow(a, shadow, c->stream), "weight shadow");
  }
  const size_t need = a.M * Bf16DmaKp(a.K) * 2;
  // A copy a conversion sink left in one of the other slots.
  for (int s = 0; s < seeai_ctx::kXSlots; ++s)
    if (c->xcvt[s] && ConvertedAlready(c, a, c->xcvt_key[s])) {
      SEEAI_TRY(c, LaunchGemmBf16Dma(c->xcvt[s], shadow, a, c->stream), what);
      return SEEAI_OK;
    }
  if (!ConvertedAlready(c, a, c->cvt_key)) {
    if (need > c->cvt_bytes) {  // grow after draining the stream
      c->cvt_key.at = nullptr;
      DropGraphs(c);
      SEEAI_TRY(c, hipStreamSynchronize(c->stream), "conversion buffer drain");
      if (c->cvt) SEEAI_TRY(c, hipFree(c->cvt), "conversion buffer free");
      c->cvt = nullptr;
      c->cvt_bytes = 0;
      SEEAI_TRY(c, hipMalloc(&c->cvt, need), "conversion buffer alloc");
      c->cvt_bytes = need;
    }
    c->cvt_key = {a.A, a.M, a.K, a.alpha_a, a.a_k_scale, c->cur_at};
    SEEAI_TRY(c,
              LaunchConvertRowsBf16(a.A, a.M, a.K, a.alpha_a, a.a_k_scale, c->cvt,
                                    c->policy.convert_wgs_per_cu, c->stream),
              what);
  }
  SEEAI_TRY(c, LaunchGemmBf16Dma(c->cvt, shadow, a, c->stream), what);
  return SEEAI_OK;
}

// A GEMM launch with the workspace its kernel may use.
int Gemm(seeai_ctx* c, GemmArgs& a, const char* what) {
  a.policy = &c->policy;
  if (a.relaxed && c->allow_dma && Bf16DmaFits(a) && Immutable(c, a.B)) return GemmBf16Dma(c, a, what);
  if (const size_t bytes = a.relaxed ? 0 : GemmExactScratchBytes(a)) {
    void* ws;
    if (int rc = Scratch(c, bytes, &ws)) return rc;
    a.scratch = static_cast<float*>(ws);
  }
  SEEAI_TRY(c, LaunchGemm(a, c->stream), what);
  return SEEAI_OK;
}

// kFlagRelaxed (instruction.h:356-384) taken as a permission when the
// context allows it; each relaxed execution is counted (backend.h:149-162).
int Relaxed(seeai_ctx* c, const Instruction& ins) {
  const int r = (ins.flags & kFlagRelaxed) && c->allow_relaxed ? 1 : 0;
  c->relaxed += r;
  return r;
}

// A relaxed tiled-attention instruction (instruction.h:384-390: f32 products
// with the sums reordered, at head widths up to 64) runs the f32 MFMA
// family unless the backend is switched to bf16 attention; only the bf16
// kernels are a relaxed execution.
bool IsRelaxedAttention(const seeai_ctx* c, const Instruction& ins) {
  return (ins.flags & kFlagRelaxed) && c->allow_relaxed && c->attn_bf16;
}
int RelaxedAttention(seeai_ctx* c, const Instruction& ins) {
  const int r = IsRelaxedAttention(c, ins) ? 1 : 0;
  c->relaxed += r;
  return r;
}

bool Overlap(const uint8_t* a, uint64_t na, const uint8_t* b, uint64_t nb) {
  return a < b + nb && b < a + na;
}

// One operand's byte extent and whether the instruction writes it (a
// read-modify-write operand is one write extent, as the reference's
// validator describes it, plan_validator.cc:365-745): what the dead-store
// scan and the attention copies below ask of an instruction.
struct Touch {
  const uint8_t* p;
  uint64_t n;
  bool write;
};
bool TouchExtents(seeai_ctx* c, const Instruction& ins, Touch* out, int* n);

// Relaxed bf16 attention with head width 64 runs the bf16-operand kernels
// (k_attn16.hip) on bf16 copies of its f32 operands: rounding them once per
// instruction (or once for a dQ and the dK / dV right after it) costs less
// than the f32-operand kernels' rounding as they stage.  The kernels round
// the same values to bf16 (RNE), so the relaxed grant is unchanged.
bool Attn16Plan(const seeai_ctx* c, uint64_t B, uint64_t S, uint64_t H, uint64_t d) {
  return c->attn16_plans && c->attn_bf16 && c->allow_relaxed && Attn16Fits(B, S, H, d) &&
         (H * d) % 32 == 0;
}

// The bf16 copies of the operands `need` marks (bit i: slot i = q, k, v,
// dO), each [B·S, H·64]: converted here, or kept from the instruction just
// before when it converted the same sources and wrote none of them.
int Attn16Operands(seeai_ctx* c, const float* const src[4], unsigned need, uint64_t rows,
                   uint64_t cols, uint16_t* out[4]) {
  const uint64_t n = rows * cols;
  const size_t bytes = 4 * n * 2;
  if (bytes > c->a16_bytes) {
    c->a16_key.at = nullptr;
    DropGraphs(c);
    SEEAI_TRY(c, hipStreamSynchronize(c->stream), "attention copies drain");
    if (c->a16) SEEAI_TRY(c, hipFree(c->a16), "attention copies free");
    c->a16 = nullptr;
    c->a16_bytes = 0;
    SEEAI_TRY(c, hipMalloc(&c->a16, bytes), "attention copies alloc");
    c->a16_bytes = bytes;
  }
  bool keep = c->cur_at && c->a16_key.at && c->a16_key.at + 64 == c->cur_at && c->a16_key.n == n;
  if (keep) {  // the previous instruction must not have written a kept source
    Instruction prev;
    std::memcpy(&prev, c->a16_key.at, sizeof prev);
    Touch t[16];
    int nt = 0;
    keep = TouchExtents(c, prev, t, &nt);
    for (int i = 0; keep && i < nt; ++i)
      for (int j = 0; j < 4; ++j)
        if (t[i].write && src[j] &&
            Overlap(t[i].p, t[i].n, reinterpret_cast<const uint8_t*>(src[j]), n * 4))
          keep = false;
  }
  for (int i = 0; i < 4; ++i) {
    out[i] = static_cast<uint16_t*>(c->a16) + static_cast<size_t>(i) * n;
    if (!(need & (1u << i))) continue;
    if (keep && c->a16_key.src[i] == src[i]) continue;
    if (i == 3 && c->cur_at && c->a16_pre[3].src == src[3] && c->a16_pre[3].at == CurIndex(c) &&
        c->a16_pre[3].epoch == c->a16_epoch) {
      c->a16_pre[3].src = nullptr;  // written by the LoRA site just before
      ++c->sinks;
      continue;
    }
    SEEAI_TRY(c,
              LaunchConvertRowsBf16(src[i], rows, cols, 1.0f, nullptr, out[i],
                                    c->policy.convert_wgs_per_cu, c->stream),
              "attention operand to bf16");
  }
  for (int i = 0; i < 4; ++i)
    if (need & (1u << i)) c->a16_key.src[i] = src[i];
    else if (!keep) c->a16_key.src[i] = nullptr;
  c->a16_key.n = n;
  c->a16_key.at = c->cur_at;
  return SEEAI_OK;
}

// Range-level fusion of the attention backward (the seam's whole-program
// visibility, backend.h:139-142; the reference's Metal backend fuses the
// low-rank pair the same way, metal_backend.mm:1155-1340).  kAttnDKTiled and
// kAttnDVTiled of one attention -- adjacent in the range, same q, k, dO,
// stats and geometry, both relaxed -- run as one pass that forms S, P and dP
// once for both accumulations; the second instruction is then skipped at its
// own place.  Each output keeps its one writer and the products and their
// order of the separate kernels, so the arena holds the same bytes.  Refused
// (the two run apart) when either output overlaps the other or anything the
// pass reads: the separate order may legally reuse a buffer the first
// instruction alone still reads.  Returns -1 when the pair does not fuse.
// The saved forward copies of (q, k, v) over n floats each, or null.
seeai_ctx::A16Saved* SavedCopies(seeai_ctx* c, const float* q, const float* k, const float* v,
                                 uint64_t n) {
  for (auto& sv : c->a16_saved)
    if (sv.src[0] == q && sv.src[1] == k && sv.src[2] == v && sv.n == n) return &sv;
  return nullptr;
}

// A buffer for the forward's copies of (q, k, v) (made ahead of a range by
// PresizeWorkspaces, so none is allocated inside one): 6 bytes per element
// of q, one buffer per distinct source triple (a decoder keeps one per
// layer, every forward-to-backward interval of a step overlapping the
// others), kept until the next bind.  The buffers together stay within
// c->a16_saved_cap bytes; a triple past the cap keeps no copies and its
// backward converts q, k and v again, as a separate range would.
int MakeSavedCopies(seeai_ctx* c, const float* q, const float* k, const float* v, uint64_t n) {
  if (SavedCopies(c, q, k, v, n)) return SEEAI_OK;
  uint64_t held = 0;
  for (const auto& sv : c->a16_saved) held += 3 * sv.n * 2;
  if (held + 3 * n * 2 > c->a16_saved_cap) return SEEAI_OK;
  void* buf = nullptr;
  SEEAI_TRY(c, hipMalloc(&buf, 3 * n * 2), "attention forward copies alloc");
  c->a16_saved.push_back({{q, k, v}, n, 0, 0, 0, buf});
  return SEEAI_OK;
}

// Whether the saved copies still match their sources at the current
// instruction: made in this range run, and no instruction since has written
// into a source (each instruction between scanned once).
bool SavedCurrent(seeai_ctx* c, seeai_ctx::A16Saved* sv) {
  if (!sv || sv->epoch != c->a16_epoch || !c->cur_at || !c->prog) return false;
  const uint64_t cur = static_cast<uint64_t>(c->cur_at - c->prog) / 64;
  if (cur <= sv->idx) return false;
  for (uint64_t i = std::max(sv->clean_to, sv->idx + 1); i < cur; ++i) {
    Instruction ins;
    std::memcpy(&ins, c->prog + i * 64, sizeof ins);
    Touch t[16];
    int nt = 0;
    bool ok = TouchExtents(c, ins, t, &nt);
    for (int j = 0; ok && j < nt; ++j)
      for (int s = 0; s < 3; ++s)
        if (t[j].write &&
            Overlap(t[j].p, t[j].n, reinterpret_cast<const uint8_t*>(sv->src[s]), sv->n * 4))
          ok = false;
    if (!ok) {
      sv->epoch = 0;
      return false;
    }
    sv->clean_to = i + 1;
  }
  return true;
}

// A RoPE forward whose output y is the q or k operand of a bf16-copy
// attention forward at most two instructions on (the instruction between,
// the other RoPE, writes neither y nor the copies) writes y's bf16 copy into
// that attention's saved copies as it stores y; the attention then skips
// that operand's conversion.  Returns the copy's slot, or null.
uint16_t* RopeAttnCopy(seeai_ctx* c, const float* x, const float* y, uint64_t B, uint64_t S,
                       uint64_t H, uint64_t d, const float* table) {
  if (!c->allow_fusion || !c->allow_sinks || !c->cur_at || !c->prog ||
      !RopeRowsFits(x, y, B, S, H, d, table))
    return nullptr;
  const uint64_t at = CurIndex(c), n = B * S * H * d;
  for (uint64_t a = at + 1; a <= at + 2 && a < c->range_end; ++a) {
    Instruction ins;
    std::memcpy(&ins, c->prog + a * 64, sizeof ins);
    if (ins.opcode != 47 && ins.opcode != 57) {
      Touch t[16];
      int nt = 0;
      if (!TouchExtents(c, ins, t, &nt)) return nullptr;
      for (int j = 0; j < nt; ++j)
        if (t[j].write && Overlap(t[j].p, t[j].n, reinterpret_cast<const uint8_t*>(y), n * 4))
          return nullptr;
      continue;
    }
    uint64_t aB, aS, aH, ad;
    if (ins.opcode == 47) {
      aB = ins.out[1] >> 32, aS = ins.out[1] & 0xFFFFFFFFu, aH = ins.out[2] >> 32,
      ad = ins.out[2] & 0xFFFFFFFFu;
    } else {
      const uint64_t g = ins.out[1];
      aB = g >> 48, aS = (g >> 32) & 0xFFFF, aH = (g >> 16) & 0xFFFF, ad = g & 0xFFFF;
    }
    if (aB * aS * aH * ad != n || !IsRelaxedAttention(c, ins) || !Attn16Plan(c, aB, aS, aH, ad))
      return nullptr;
    Ptrs R{c};
    const float* src[3] = {R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2])};
    seeai_ctx::A16Saved* sv = SavedCopies(c, src[0], src[1], src[2], n);
    if (!sv) return nullptr;
    const int slot = src[0] == y ? 0 : src[1] == y ? 1 : -1;
    if (slot < 0) return nullptr;
    c->a16_pre[slot].src = y;
    c->a16_pre[slot].at = a;
    c->a16_pre[slot].epoch = c->a16_epoch;
    return static_cast<uint16_t*>(sv->buf) + static_cast<size_t>(slot) * n;
  }
  return nullptr;
}

// A LoRA site's output y (n floats, the fused pass's last instruction at
// `last`) read by a bf16-copy attention: as v by a forward within three
// instructions (those between write neither y nor the copies -- the RoPE
// forwards, which write the q and k slots), or as dO by a backward right
// after.  The site's epilogue then writes y's bf16 copy where that attention
// takes it: the forward's saved copies (slot 2), the operand buffer's dO
// slot (slot 3).  Returns the copy's address with *slot and the attention's
// index *at, or null.
uint16_t* PlanAttnCopy(seeai_ctx* c, uint64_t last, const float* y, uint64_t n, int* slot,
                       uint64_t* at) {
  if (!c->allow_fusion || !c->allow_sinks || !c->prog) return nullptr;
  const Ptrs R{c};
  for (uint64_t f = last + 1; f <= last + 3 && f < c->range_end; ++f) {
    Instruction ins;
    std::memcpy(&ins, c->prog + f * 64, sizeof ins);
    if (ins.opcode == 47 || ins.opcode == 57) {
      uint64_t aB, aS, aH, ad;
      if (ins.opcode == 47) {
        aB = ins.out[1] >> 32, aS = ins.out[1] & 0xFFFFFFFFu, aH = ins.out[2] >> 32,
        ad = ins.out[2] & 0xFFFFFFFFu;
      } else {
        const uint64_t g = ins.out[1];
        aB = g >> 48, aS = (g >> 32) & 0xFFFF, aH = (g >> 16) & 0xFFFF, ad = g & 0xFFFF;
      }
      if (aB * aS * aH * ad != n || !IsRelaxedAttention(c, ins) || !Attn16Plan(c, aB, aS, aH, ad))
        return nullptr;
      const float* src[3] = {R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2])};
      if (src[2] != y || src[0] == y || src[1] == y) return nullptr;
      seeai_ctx::A16Saved* sv = SavedCopies(c, src[0], src[1], src[2], n);
      if (!sv) return nullptr;
      *slot = 2;
      *at = f;
      return static_cast<uint16_t*>(sv->buf) + 2 * static_cast<size_t>(n);
    }
    if (f == last + 1 && (ins.opcode == 48 || ins.opcode == 49 || ins.opcode == 50)) {
      const uint64_t g = ins.out[2];
      const uint64_t B = g >> 48, S = (g >> 32) & 0xFFFF, H = (g >> 16) & 0xFFFF, d = g & 0xFFFF;
      if (B * S * H * d != n || !IsRelaxedAttention(c, ins) || !Attn16Plan(c, B, S, H, d) ||
          (ins.opcode == 50 && ins.in[2] == kNullRef))
        return nullptr;
      if (R.f(ins.in[3]) != y || R.f(ins.in[0]) == y || R.f(ins.in[1]) == y ||
          R.f(ins.in[2]) == y)
        return nullptr;
      if (!c->a16 || c->a16_bytes < 4 * n * 2) return nullptr;  // sized by an earlier run
      *slot = 3;
      *at = f;
      return static_cast<uint16_t*>(c->a16) + 3 * static_cast<size_t>(n);
    }
    Touch t[16];
    int nt = 0;
    if (!TouchExtents(c, ins, t, &nt)) return nullptr;
    for (int j = 0; j < nt; ++j)
      if (t[j].write && Overlap(t[j].p, t[j].n, reinterpret_cast<const uint8_t*>(y), n * 4))
        return nullptr;
  }
  return nullptr;
}

// The operands of a backward instruction: q, k, v from the forward's saved
// copies where they are current, else converted with dO.
int Attn16BwdOperands(seeai_ctx* c, const float* const src[4], uint64_t rows, uint64_t cols,
                      uint16_t* out[4]) {
  seeai_ctx::A16Saved* sv = SavedCopies(c, src[0], src[1], src[2], rows * cols);
  if (SavedCurrent(c, sv)) {
    if (int rc = Attn16Operands(c, src, 8u, rows, cols, out)) return rc;
    for (int i = 0; i < 3; ++i)
      out[i] = static_cast<uint16_t*>(sv->buf) + static_cast<size_t>(i) * rows * cols;
    return SEEAI_OK;
  }
  return Attn16Operands(c, src, 15u, rows, cols, out);
}

bool PlanFarSink(seeai_ctx* c, uint64_t last, const float* out, uint64_t n, Bf16Sink* sink,
                 GemmArgs* ga, int* xslot, uint64_t* key_at);
void FarSinkDone(seeai_ctx* c, uint64_t key_at, const GemmArgs& a, int xslot);

int TryFuseAttnBwd(seeai_ctx* c, const Instruction& ins, const uint8_t* at) {
  if (!c->allow_fusion || !c->prog || at < c->prog || at >= c->prog + c->prog_count * 64 ||
      (at - c->prog) % 64 != 0)
    return -1;
  const uint64_t idx = static_cast<uint64_t>(at - c->prog) / 64;
  if (idx + 1 >= c->range_end) return -1;
  Instruction nx;
  std::memcpy(&nx, at + 64, sizeof nx);
  if (ins.opcode + nx.opcode != 49 + 50 || (ins.opcode != 49 && ins.opcode != 50)) return -1;
  // Both on the relaxed bf16 kernels, or both in the exact family (which
  // relaxed instructions run when attention is not on bf16).
  const bool relaxed = IsRelaxedAttention(c, ins);
  if (relaxed != IsRelaxedAttention(c, nx)) return -1;
  if (ins.in[0] != nx.in[0] || ins.in[1] != nx.in[1] || ins.in[3] != nx.in[3] ||
      ins.out[0] != nx.out[0] || ins.out[2] != nx.out[2])
    return -1;
  const Instruction& dki = ins.opcode == 49 ? ins : nx;
  const Instruction& dvi = ins.opcode == 49 ? nx : ins;
  const uint64_t g = ins.out[2];
  const uint64_t B = g >> 48, S = (g >> 32) & 0xFFFF, H = (g >> 16) & 0xFFFF, d = g & 0xFFFF;
  const Ptrs R{c};
  const float *q = R.f(dki.in[0]), *k = R.f(dki.in[1]), *v = R.f(dki.in[2]), *dout = R.f(dki.in[3]);
  const float* stats = R.f(dki.out[0]);
  float *dk = R.f(dki.out[1]), *dv = R.f(dvi.out[1]);
  if (relaxed ? !AttnDKDVFusable(q, k, v, dout, dk, dv, B, S, H, d)
              : !AttnDKDVExactFusable(q, k, v, dout, stats, dk, dv, B, S, H, d))
    return -1;
  const uint64_t act = B * S * H * d * 4, st = B * H * S * 16;
  const auto* o1 = reinterpret_cast<const uint8_t*>(dk);
  const auto* o2 = reinterpret_cast<const uint8_t*>(dv);
  if (Overlap(o1, act, o2, act)) return -1;
  for (const float* in : {q, k, v, dout})
    for (const uint8_t* o : {o1, o2})
      if (Overlap(o, act, reinterpret_cast<const uint8_t*>(in), act)) return -1;
  for (const uint8_t* o : {o1, o2})
    if (Overlap(o, act, reinterpret_cast<const uint8_t*>(stats), st)) return -1;
  RelaxedAttention(c, ins);
  RelaxedAttention(c, nx);
  if (!relaxed) {
    SEEAI_TRY(c, LaunchAttnDKDVExact(q, k, v, dout, stats, dk, dv, B, S, H, d, c->stream),
              "attn.dkdv_exact");
  } else if (Attn16Plan(c, B, S, H, d)) {
    const float* src[4] = {q, k, v, dout};
    uint16_t* b16[4];
    if (int rc = Attn16BwdOperands(c, src, B * S, H * d, b16)) return rc;
    // dV's copy for the relaxed product that takes it past the adapter GEMMs.
    Bf16Sink sink;
    GemmArgs ga{};
    int xslot = -1;
    uint64_t key_at = 0;
    if (c->cur_at) PlanFarSink(c, idx + 1, dv, B * S * H * d, &sink, &ga, &xslot, &key_at);
    SEEAI_TRY(c,
              LaunchAttn16DKDV(b16[0], b16[1], b16[2], b16[3], stats, dk, dv, B, S, H, c->stream,
                               sink),
              "attn.dkdv_bf16");
    if (xslot >= 0) FarSinkDone(c, key_at, ga, xslot);
  } else {
    SEEAI_TRY(c, LaunchAttnDKDVFused(q, k, v, dout, stats, dk, dv, B, S, H, d, c->stream),
              "attn.dkdv_fused");
  }
  c->done[0] = at + 64;
  c->ndone = 1;
  ++c->fused;
  return SEEAI_OK;
}

// A GEMM instruction's operands (every GEMM opcode; the caller sets
// `relaxed`).  Returns the op's name for messages, or null for another opcode.
const char* DecodeGemm(seeai_ctx* c, const Instruction& ins, GemmArgs* out) {
  const Ptrs R{c};
  const int act = (ins.flags >> 1) & 3;
  const float alpha = ins.imm == 0 ? 1.0f : BitsToF32(ins.imm);
  GemmArgs a{};
  a.A = R.f(ins.in[0]);
  a.C = R.f(ins.in[2]);
  a.M = ins.out[0];
  a.N = ins.out[1];
  a.K = ins.out[2];
  const char* what = nullptr;
  switch (ins.opcode) {
    case 1:    // kGemmNN
    case 2:    // kGemmNT
    case 3:    // kGemmTN
      a.layout = ins.opcode - 1;
      a.b_kind = 0;
      a.B = R.f(ins.in[1]);
      // instruction.h:384-404: NN / TN fold alpha into A, NT onto the dot.
      a.alpha_a = ins.opcode == 2 ? 1.0f : alpha;
      a.alpha_dot = ins.opcode == 2 ? alpha : 1.0f;
      a.addend = (ins.flags & kFlagGemmAddend) ? R.f(ins.in[3]) : nullptr;
      a.bias = (ins.opcode == 1 && (ins.flags & kFlagEpilogueBias)) ? R.f(ins.in[3]) : nullptr;
      a.act = ins.opcode == 1 ? act : 0;
      what = "gemm";
      break;
    case 4:  // kGemmAccNN: C += alpha A@B, alpha bits in in[3]
      a.layout = 0;
      a.B = R.f(ins.in[1]);
      a.alpha_a = BitsToF32(ins.in[3]);
      a.alpha_dot = 1.0f;
      a.accumulate = 1;
      what = "gemm.acc_nn";
      break;
    case 29:    // kGemmNNQ8
    case 30: {  // kGemmNTQ8
      const bool nt = ins.opcode == 30;
      const bool cs = (ins.flags & kFlagQ8ColScale) != 0;
      a.layout = nt ? 1 : 0;
      a.b_kind = 1;
      a.B = R.at(ins.in[1]);
      const float scale = cs ? 1.0f : BitsToF32(ins.in[3]);
      // gemm.cc:626-674: NN per-tensor scale folds into A, a column scale
      // joins the widening; NT per-tensor scale multiplies the dot, a
      // k-scale multiplies A's elements.
      a.alpha_a = nt ? 1.0f : scale;
      a.alpha_dot = nt ? scale : 1.0f;
      if (cs) {
        if (nt)
          a.a_k_scale = R.f(ins.in[3]);
        else
          a.b_col_scale = R.f(ins.in[3]);
      }
      a.act = nt ? 0 : act;
      what = "gemm.q8";
      break;
    }
    case 43:    // kGemmNNBF16
    case 44: {  // kGemmNTBF16
      const bool nt = ins.opcode == 44;
      a.layout = nt ? 1 : 0;
      a.b_kind = 2;
      a.B = R.at(ins.in[1]);
      a.alpha_a = 1.0f;
      a.alpha_dot = 1.0f;
      a.bias = (!nt && (ins.flags & kFlagEpilogueBias)) ? R.f(ins.in[3]) : nullptr;
      a.act = nt ? 0 : act;
      what = "gemm.bf16";
      break;
    }
    default:
      return nullptr;
  }
  *out = a;
  return what;
}

bool PlanSink(seeai_ctx* c, uint64_t last, uint64_t writer, const float* out, uint64_t n,
              Bf16Sink* sink, GemmArgs* ga, int slot = 1, int site = 0);
void SinkDone(seeai_ctx* c, uint64_t last, const GemmArgs& a, int slot = 1);
// The index of the instruction being executed within its range's program
// (c->cur_at set).
uint64_t CurIndex(const seeai_ctx* c) { return static_cast<uint64_t>(c->cur_at - c->prog) / 64; }

// A relaxed product on the direct-to-LDS kernel whose C the softmax-xent
// forward right after takes as its logits: its epilogue also leaves C's
// partial row maxima (a->row_max_part), from which the loss turn forms the
// row max without its own pass over the logits.
int PlanRowMaxParts(seeai_ctx* c, GemmArgs* a) {
  if (!c->allow_fusion || !c->cur_at || !c->prog || !a->relaxed || !c->allow_dma) return SEEAI_OK;
  const uint64_t idx = CurIndex(c);
  if (idx + 1 >= c->range_end) return SEEAI_OK;
  Instruction nx;
  std::memcpy(&nx, c->prog + (idx + 1) * 64, sizeof nx);
  const Ptrs R{c};
  if ((nx.opcode != 11 && nx.opcode != 51) || R.f(nx.in[0]) != a->C || nx.out[0] != a->M ||
      nx.out[1] != a->N || XEntOneWorkgroup(a->M, a->N))
    return SEEAI_OK;
  a->policy = &c->policy;
  if (!Bf16DmaRowMaxFits(*a) || !Immutable(c, a->B)) return SEEAI_OK;
  const size_t bytes = a->M * ((a->N + 63) / 64) * 4;
  if (bytes > c->pmax_bytes) {  // grow after draining the stream
    DropGraphs(c);
    SEEAI_TRY(c, hipStreamSynchronize(c->stream), "row maxima drain");
    if (c->pmax) SEEAI_TRY(c, hipFree(c->pmax), "row maxima free");
    c->pmax = nullptr;
    c->pmax_bytes = 0;
    SEEAI_TRY(c, hipMalloc(&c->pmax, bytes), "row maxima alloc");
    c->pmax_bytes = bytes;
  }
  a->row_max_part = c->pmax;
  return SEEAI_OK;
}

int ExecuteOne(seeai_ctx* c, const Instruction& ins, const seeai_step_params& P) {
  if (!c->arena) return Fail(c, SEEAI_INVALID, "execute: no arena is bound");
  const Ptrs R{c};
  hipStream_t s = c->stream;
  const int act = (ins.flags >> 1) & 3;
  const float alpha = ins.imm == 0 ? 1.0f : BitsToF32(ins.imm);
  const float norm_eps = ins.imm == 0 ? 1e-5f : BitsToF32(ins.imm);
  const uint64_t hi0 = ins.out[0] >> 32, lo0 = ins.out[0] & 0xFFFFFFFFu;
  switch (ins.opcode) {
    case 0:  // kNop
      return SEEAI_OK;
    case 1:     // kGemmNN
    case 2:     // kGemmNT
    case 3:     // kGemmTN
    case 4:     // kGemmAccNN
    case 29:    // kGemmNNQ8
    case 30:    // kGemmNTQ8
    case 43:    // kGemmNNBF16
    case 44: {  // kGemmNTBF16
      GemmArgs a{};
      const char* what = DecodeGemm(c, ins, &a);
      a.relaxed = Relaxed(c, ins);
      if (int rc = PlanRowMaxParts(c, &a)) return rc;
      // C read next by a bf16-copy attention (a backward's dO): its copy
      // written in the epilogue.
      int pre_slot = -1;
      uint64_t pre_at = 0;
      if (c->cur_at && a.relaxed && c->allow_dma && !a.row_max_part) {
        a.policy = &c->policy;
        GemmArgs t = a;
        t.lr_sink = PlanAttnCopy(c, CurIndex(c), a.C, a.M * a.N, &pre_slot, &pre_at);
        if (t.lr_sink && Bf16DmaRowMaxFits(t) && Immutable(c, t.B)) a = t;
        else pre_slot = -1;
      }
      if (int rc = Gemm(c, a, what)) return rc;
      if (a.row_max_part)
        c->pmax_key = {a.C, a.M, a.N, CurIndex(c) + 1, c->a16_epoch};
      if (pre_slot >= 0) {
        c->a16_pre[pre_slot].src = a.C;
        c->a16_pre[pre_slot].at = pre_at;
        c->a16_pre[pre_slot].epoch = c->a16_epoch;
      }
      return SEEAI_OK;
    }
    case 5: {
      Bf16Sink sink;
      GemmArgs ga{};
      const bool sunk = c->cur_at &&
                        NormSinkFits(ins.out[0], {R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2])}) &&
                        PlanSink(c, CurIndex(c), CurIndex(c), R.f(ins.in[2]), ins.out[0], &sink, &ga);
      SEEAI_TRY(c, LaunchAddEW(R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]), ins.out[0], s, sink),
                "add");
      if (sunk) SinkDone(c, CurIndex(c), ga);
      return SEEAI_OK;
    }
    case 21:
      SEEAI_TRY(c, LaunchMulEW(R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]), ins.out[0], s), "mul");
      return SEEAI_OK;
    case 6:
      SEEAI_TRY(c,
                LaunchAddBias(R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]), ins.out[0],
                              ins.out[1], s),
                "add.bias");
      return SEEAI_OK;
    case 7:   // ReluFwd
    case 22:  // GeluFwd
    case 24:  // SiluFwd
    {
      const int kind = ins.opcode == 7 ? 1 : ins.opcode == 22 ? 2 : 3;
      Bf16Sink sink;
      GemmArgs ga{};
      const bool sunk = c->cur_at && ElementwiseSinkFits(kind, ins.out[0], R.f(ins.in[0]), nullptr,
                                                         R.f(ins.in[1])) &&
                        PlanSink(c, CurIndex(c), CurIndex(c), R.f(ins.in[1]), ins.out[0], &sink, &ga);
      SEEAI_TRY(c, LaunchUnary(kind, R.f(ins.in[0]), R.f(ins.in[1]), ins.out[0], 1.0f, s, sink),
                "act.fwd");
      if (sunk) SinkDone(c, CurIndex(c), ga);
      return SEEAI_OK;
    }
    case 8:   // ReluBwd
    case 23:  // GeluBwd
    case 25:  // SiluBwd
    {
      const int kind = ins.opcode == 8 ? 1 : ins.opcode == 23 ? 2 : 3;
      Bf16Sink sink;
      GemmArgs ga{};
      const bool sunk = c->cur_at && ElementwiseSinkFits(kind, ins.out[0], R.f(ins.in[0]),
                                                         R.f(ins.in[1]), R.f(ins.in[2])) &&
                        PlanSink(c, CurIndex(c), CurIndex(c), R.f(ins.in[2]), ins.out[0], &sink, &ga);
      SEEAI_TRY(c,
                LaunchBinaryBwd(kind, R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]), ins.out[0], s,
                                sink),
                "act.bwd");
      if (sunk) SinkDone(c, CurIndex(c), ga);
      return SEEAI_OK;
    }
    case 9:  // kScale
      SEEAI_TRY(c,
                LaunchUnary(4, R.f(ins.in[0]), R.f(ins.in[1]), ins.out[0], BitsToF32(ins.in[2]), s),
                "scale");
      return SEEAI_OK;
    case 10:
      SEEAI_TRY(c, LaunchReduceRows(R.f(ins.in[0]), R.f(ins.in[1]), ins.out[0], ins.out[1], s),
                "reduce_rows");
      return SEEAI_OK;
    case 11:
    case 51: {  // SoftmaxXEntFwd (+masked)
      void* ws;
      if (int rc = Scratch(c, XEntFwdScratchBytes(ins.out[0]), &ws)) return rc;
      SEEAI_TRY(c,
                LaunchXEntFwd(R.f(ins.in[0]), R.i32(ins.in[1]), R.f(ins.in[2]), R.f(ins.in[3]),
                              ins.out[0], ins.out[1], ins.opcode == 51, ws, s),
                "softmax_xent.fwd");
      return SEEAI_OK;
    }
    case 12:
    case 52: {  // SoftmaxXEntBwd (+masked)
      void* ws;
      if (int rc = Scratch(c, 64, &ws)) return rc;
      Bf16Sink sink;
      GemmArgs ga{};
      const bool sunk = c->cur_at && XEntBwdSinkFits(R.f(ins.in[0]), R.f(ins.in[3]), ins.out[1]) &&
                        PlanSink(c, CurIndex(c), CurIndex(c), R.f(ins.in[3]),
                                 ins.out[0] * ins.out[1], &sink, &ga);
      SEEAI_TRY(c,
                LaunchXEntBwd(R.f(ins.in[0]), R.i32(ins.in[1]), R.f(ins.in[2]), R.f(ins.in[3]),
                              ins.out[0], ins.out[1], ins.opcode == 52, ws, s, sink),
                "softmax_xent.bwd");
      if (sunk) SinkDone(c, CurIndex(c), ga);
      return SEEAI_OK;
    }
    case 17: {  // kSgdStep
      const float clip = BitsToF32(ins.out[1]);
      const float* scale = nullptr;
      if (clip > 0.0f) {
        void* ws;
        if (int rc = Scratch(c, 8 * 1024, &ws)) return rc;
        SEEAI_TRY(c,
                  LaunchClipFactor(R.f(ins.in[1]), ins.out[0], clip, c->scale_slot(), c->flag(),
                                   ws, s),
                  "sgd clip");
        scale = c->scale_slot();
      }
      SEEAI_TRY(c,
                LaunchSgd(R.f(ins.in[0]), R.f(ins.in[1]), ins.out[0], P.lr, P.weight_decay, scale,
                          c->flag(), s, c->capturing ? c->hyper() : nullptr),
                "sgd");
      return SEEAI_OK;
    }
    case 18:  // kAdamWStep (+ fused clip in out[1])
      return AdamWLaunch(c, R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]), R.f(ins.in[3]),
                         ins.out[0], P, BitsToF32(ins.out[1]));
    case 28: {  // kClipNorm
      const float cap = BitsToF32(ins.in[1]);
      if (!std::isfinite(cap) || !(cap > 0.0f)) return Fail(c, SEEAI_REFUSED, "%s", kClipThresholdRefusal);
      void* ws;
      if (int rc = Scratch(c, 8 * 1024, &ws)) return rc;
      SEEAI_TRY(c, LaunchClipFactor(R.f(ins.in[0]), ins.out[0], cap, c->scale_slot(), c->flag(), ws, s),
                "clip");
      SEEAI_TRY(c, LaunchScaleByFactor(R.f(ins.in[0]), ins.out[0], c->scale_slot(), c->flag(), s),
                "clip scale");
      return SEEAI_OK;
    }
    case 53: {  // kSqNormAccum
      void* ws;
      if (int rc = Scratch(c, 8 * 1024, &ws)) return rc;
      SEEAI_TRY(c, LaunchSqNormAccum(R.f(ins.in[0]), ins.out[0], R.f(ins.in[1]), ws, s), "sqnorm");
      return SEEAI_OK;
    }
    case 54: {  // kClipGlobal
      const float cap = BitsToF32(ins.in[2]);
      if (!std::isfinite(cap) || !(cap > 0.0f)) return Fail(c, SEEAI_REFUSED, "%s", kClipThresholdRefusal);
      SEEAI_TRY(c, LaunchGlobalClipFactor(R.f(ins.in[1]), cap, c->scale_slot(), c->flag(), s),
                "clip.global");
      SEEAI_TRY(c, LaunchScaleByFactor(R.f(ins.in[0]), ins.out[0], c->scale_slot(), c->flag(), s),
                "clip.global scale");
      return SEEAI_OK;
    }
    case 19:
      SEEAI_TRY(c, LaunchFill(R.f(ins.in[0]), BitsToF32(ins.in[1]), ins.out[0], s), "fill");
      return SEEAI_OK;
    case 20:
      SEEAI_TRY(c, LaunchCopy(R.f(ins.in[0]), R.f(ins.in[1]), ins.out[0], s), "copy");
      return SEEAI_OK;
    case 42:
      SEEAI_TRY(c, LaunchAccumulate(R.f(ins.in[0]), R.f(ins.in[1]), ins.out[0], s), "accumulate");
      return SEEAI_OK;
    case 26:
    case 27:
    case 31:
    case 32: {  // LayerNorm / RMSNorm forward and backward
      const uint64_t shape = ins.opcode == 27 ? ins.out[2] : ins.opcode == 32 ? ins.out[1] : ins.out[0];
      const uint64_t rows = shape >> 32, cols = shape & 0xFFFFFFFFu;
      // The row-shaped output: y (forward) or dx (backward).
      const float* out = R.f(ins.opcode == 31 ? ins.in[2] : ins.in[3]);
      Bf16Sink sink;
      GemmArgs ga{};
      const bool sunk =
          c->cur_at &&
          NormSinkFits(cols, {R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]), R.f(ins.in[3])}) &&
          PlanSink(c, CurIndex(c), CurIndex(c), out, rows * cols, &sink, &ga);
      if (ins.opcode == 26)
        SEEAI_TRY(c,
                  LaunchLayerNormFwd(R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]), R.f(ins.in[3]),
                                     R.f(ins.out[1]), R.f(ins.out[2]), rows, cols, norm_eps, s, sink),
                  "layernorm.fwd");
      else if (ins.opcode == 27)
        SEEAI_TRY(c,
                  LaunchLayerNormBwd(R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]), R.f(ins.out[0]),
                                     R.f(ins.out[1]), R.f(ins.in[3]), rows, cols, s, sink),
                  "layernorm.bwd");
      else if (ins.opcode == 31)
        SEEAI_TRY(c,
                  LaunchRmsNormFwd(R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]), R.f(ins.in[3]),
                                   rows, cols, norm_eps, s, sink),
                  "rmsnorm.fwd");
      else
        SEEAI_TRY(c,
                  LaunchRmsNormBwd(R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]), R.f(ins.out[0]),
                                   R.f(ins.in[3]), rows, cols, s, sink),
                  "rmsnorm.bwd");
      if (sunk) SinkDone(c, CurIndex(c), ga);
      return SEEAI_OK;
    }
    case 33:
    case 34: {  // RopeFwd / RopeBwd (v12 table in in[2])
      const uint64_t d = ins.out[1] & 0xFFFFFFFFu;
      const float base = BitsToF32(ins.out[2]);
      const float step = std::pow(base, -2.0f / static_cast<float>(d));  // attention.cc:123
      // The forward writes the bf16-copy attention's copy of its output; the
      // backward the bf16 copy of the relaxed product that takes its output
      // later (the input-gradient product of a q / k site, past the
      // adapter GEMMs).
      Bf16Sink sink;
      GemmArgs ga{};
      int xslot = -1;
      uint64_t key_at = 0;
      const uint64_t rows = hi0 * lo0, width = (ins.out[1] >> 32) * d;
      if (ins.opcode == 33) {
        sink.out = RopeAttnCopy(c, R.f(ins.in[0]), R.f(ins.in[1]), hi0, lo0, ins.out[1] >> 32, d,
                                R.fo(ins.in[2]));
        sink.K = static_cast<uint32_t>(width);
      } else if (c->cur_at && RopeRowsFits(R.f(ins.in[0]), R.f(ins.in[1]), hi0, lo0,
                                            ins.out[1] >> 32, d, R.fo(ins.in[2]))) {
        PlanFarSink(c, CurIndex(c), R.f(ins.in[1]), rows * width, &sink, &ga, &xslot, &key_at);
      }
      SEEAI_TRY(c,
                LaunchRope(R.f(ins.in[0]), R.f(ins.in[1]), hi0, lo0, ins.out[1] >> 32, d, step,
                           R.fo(ins.in[2]), ins.opcode == 34, s, sink),
                "rope");
      if (xslot >= 0) FarSinkDone(c, key_at, ga, xslot);
      return SEEAI_OK;
    }
    case 45: {  // RopeTable
      const float step = std::pow(BitsToF32(ins.out[1]), -2.0f / static_cast<float>(lo0));
      SEEAI_TRY(c, LaunchRopeTable(R.f(ins.in[0]), hi0, lo0, step, s), "rope.table");
      return SEEAI_OK;
    }
    case 46: {  // FusedMap
      SEEAI_TRY(c,
                LaunchFusedMap(R.f(ins.in[0]), R.fo(ins.in[1]), R.fo(ins.in[2]), R.f(ins.in[3]),
                               ins.out[0], ins.out[1], BitsToF32(ins.out[2]),
                               BitsToF32(ins.out[2] >> 32), s),
                "fused_map");
      return SEEAI_OK;
    }
    case 41:
      SEEAI_TRY(c,
                LaunchEmbed(R.i32(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]), ins.out[0],
                            ins.out[1] & 0xFFFFFFFFu, s),
                "embed");
      return SEEAI_OK;
    case 55:
      SEEAI_TRY(c,
                LaunchSegmentStarts(R.i32(ins.in[0]), R.i32(ins.in[1]), hi0, lo0,
                                    static_cast<int32_t>(ins.out[1]), s),
                "segment_starts");
      return SEEAI_OK;
    case 35:
    case 56: {  // AttnFwd (+Seg): cached family
      uint64_t B, S, H, d;
      const int32_t* starts = nullptr;
      if (ins.opcode == 35) {
        B = ins.out[1] >> 32, S = ins.out[1] & 0xFFFFFFFFu, H = ins.out[2] >> 32,
        d = ins.out[2] & 0xFFFFFFFFu;
      } else {
        const uint64_t g = ins.out[1];
        B = g >> 48, S = (g >> 32) & 0xFFFF, H = (g >> 16) & 0xFFFF, d = g & 0xFFFF;
        starts = R.i32(ins.out[2]);
      }
      SEEAI_TRY(c,
                LaunchAttnFwdCached(R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]), R.f(ins.in[3]),
                                    R.f(ins.out[0]), B, S, H, d, starts, s),
                "attn.fwd");
      return SEEAI_OK;
    }
    case 36:
      SEEAI_TRY(c,
                LaunchAttnDP(R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]), hi0, lo0,
                             ins.out[1] >> 32, ins.out[1] & 0xFFFFFFFFu, s),
                "attn.dp");
      return SEEAI_OK;
    case 37:
      SEEAI_TRY(c,
                LaunchAttnDV(R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]), hi0, lo0,
                             ins.out[1] >> 32, ins.out[1] & 0xFFFFFFFFu, s),
                "attn.dv");
      return SEEAI_OK;
    case 38:
      SEEAI_TRY(c,
                LaunchSoftmaxRowsBwd(R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]), hi0, lo0, s),
                "softmax_rows.bwd");
      return SEEAI_OK;
    case 39:
      SEEAI_TRY(c,
                LaunchAttnDQ(R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]), hi0, lo0,
                             ins.out[1] >> 32, ins.out[1] & 0xFFFFFFFFu, s),
                "attn.dq");
      return SEEAI_OK;
    case 40:
      SEEAI_TRY(c,
                LaunchAttnDK(R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]), hi0, lo0,
                             ins.out[1] >> 32, ins.out[1] & 0xFFFFFFFFu, s),
                "attn.dk");
      return SEEAI_OK;
    case 47:
    case 57: {  // AttnFwdTiled (+Seg)
      uint64_t B, S, H, d;
      const int32_t* starts = nullptr;
      if (ins.opcode == 47) {
        B = ins.out[1] >> 32, S = ins.out[1] & 0xFFFFFFFFu, H = ins.out[2] >> 32,
        d = ins.out[2] & 0xFFFFFFFFu;
      } else {
        const uint64_t g = ins.out[1];
        B = g >> 48, S = (g >> 32) & 0xFFFF, H = (g >> 16) & 0xFFFF, d = g & 0xFFFF;
        starts = R.i32(ins.out[2]);
      }
      const int dt = RelaxedAttention(c, ins);
      if (dt == 1 && Attn16Plan(c, B, S, H, d)) {
        const float* src[4] = {R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]), nullptr};
        uint16_t* b16[4];
        const uint64_t n = B * S * H * d;
        seeai_ctx::A16Saved* sv = c->cur_at ? SavedCopies(c, src[0], src[1], src[2], n) : nullptr;
        if (sv) {  // into the copies the backward of this range run may take
          for (int i = 0; i < 3; ++i) {
            b16[i] = static_cast<uint16_t*>(sv->buf) + static_cast<size_t>(i) * n;
            if (c->a16_pre[i].src == src[i] && c->a16_pre[i].at == CurIndex(c) &&
                c->a16_pre[i].epoch == c->a16_epoch) {
              c->a16_pre[i].src = nullptr;  // written by a RoPE forward or a LoRA site before
              ++c->sinks;
              continue;
            }
            SEEAI_TRY(c,
                      LaunchConvertRowsBf16(src[i], B * S, H * d, 1.0f, nullptr, b16[i],
                                            c->policy.convert_wgs_per_cu, s),
                      "attention operand to bf16");
          }
          sv->idx = static_cast<uint64_t>(c->cur_at - c->prog) / 64;
          sv->clean_to = sv->idx + 1;
          sv->epoch = c->a16_epoch;
        } else if (int rc = Attn16Operands(c, src, 7u, B * S, H * d, b16)) {
          return rc;
        }
        // The output's bf16 copy for the relaxed product reading it next.
        Bf16Sink sink;
        GemmArgs ga{};
        const bool sunk = c->cur_at && NormSinkFits(H * d, {R.f(ins.in[3])}) &&
                          PlanSink(c, CurIndex(c), CurIndex(c), R.f(ins.in[3]), B * S * H * d,
                                   &sink, &ga);
        SEEAI_TRY(c,
                  LaunchAttn16Fwd(b16[0], b16[1], b16[2], R.f(ins.in[3]), R.f(ins.out[0]), B, S,
                                  H, starts, s, sink),
                  "attn.fwd_bf16");
        if (sunk) SinkDone(c, CurIndex(c), ga);
        return SEEAI_OK;
      }
      SEEAI_TRY(c,
                LaunchAttnFwdTiled(dt, R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]),
                                   R.f(ins.in[3]), R.f(ins.out[0]), B, S, H, d, starts, s),
                "attn.fwd_tiled");
      return SEEAI_OK;
    }
    case 48:
    case 49:
    case 50: {  // AttnDQTiled / DKTiled / DVTiled
      const uint64_t g = ins.out[2];
      const uint64_t B = g >> 48, S = (g >> 32) & 0xFFFF, H = (g >> 16) & 0xFFFF, d = g & 0xFFFF;
      const int dt = RelaxedAttention(c, ins);
      // The bf16-operand kernels read v for dV too (it forms dP): a dV
      // instruction without a v operand keeps the f32-operand kernel.
      if (dt == 1 && Attn16Plan(c, B, S, H, d) && (ins.opcode != 50 || ins.in[2] != kNullRef)) {
        const float* src[4] = {R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]), R.f(ins.in[3])};
        uint16_t* b16[4];
        if (int rc = Attn16BwdOperands(c, src, B * S, H * d, b16)) return rc;
        hipError_t e;
        if (ins.opcode == 48)
          e = LaunchAttn16DQ(b16[0], b16[1], b16[2], b16[3], R.f(ins.out[0]), R.f(ins.out[1]), B,
                             S, H, s);
        else
          e = LaunchAttn16DKDV(b16[0], b16[1], b16[2], b16[3], R.f(ins.out[0]),
                               ins.opcode == 49 ? R.f(ins.out[1]) : nullptr,
                               ins.opcode == 50 ? R.f(ins.out[1]) : nullptr, B, S, H, s);
        SEEAI_TRY(c, e, "attn.bwd_bf16");
        return SEEAI_OK;
      }
      hipError_t e;
      if (ins.opcode == 48)
        e = LaunchAttnDQTiled(dt, R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]), R.f(ins.in[3]),
                              R.f(ins.out[0]), R.f(ins.out[1]), B, S, H, d, s);
      else if (ins.opcode == 49)
        e = LaunchAttnDKTiled(dt, R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]), R.f(ins.in[3]),
                              R.f(ins.out[0]), R.f(ins.out[1]), B, S, H, d, s);
      else
        e = LaunchAttnDVTiled(dt, R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[3]), R.f(ins.out[0]),
                              R.f(ins.out[1]), B, S, H, d, s);
      SEEAI_TRY(c, e, "attn.bwd_tiled");
      return SEEAI_OK;
    }
    default:
      // kMseFwd/Bwd (13/14) and kKLDistillFwd/Bwd (15/16) are outside this
      // executor's hot path.
      return Fail(c, SEEAI_INVALID, "execute: opcode %u is not supported by the gfx950 executor",
                  static_cast<unsigned>(ins.opcode));
  }
}

}  // namespace

extern "C" {

int seeai_create(int device, seeai_ctx** out) {
  if (!out) return SEEAI_INVALID;
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= device || device < 0) return SEEAI_HIP_ERROR;
  auto* c = new seeai_ctx();
  c->device = device;
  // SEEAI_RELAXED_DMA=0 keeps the relaxed frozen-weight GEMMs on the
  // register-staged kernel (a same-session comparison switch).
  if (const char* e = std::getenv("SEEAI_RELAXED_DMA"); e && e[0] == '0') c->allow_dma = 0;
  // SEEAI_UNFUSED_LOWRANK=1 keeps each LoRA site's products apart: the
  // same-session control of the low-rank fold (the reference's Metal backend
  // keeps SEEML_METAL_UNFUSED_LOWRANK for the same purpose).
  if (const char* e = std::getenv("SEEAI_UNFUSED_LOWRANK"); e && e[0] == '1') c->allow_lowrank = 0;
  // SEEAI_KEEP_DEAD_STORES=1 keeps every store of a fused pass (the
  // same-session control of the dead-store scan).
  if (const char* e = std::getenv("SEEAI_KEEP_DEAD_STORES"); e && e[0] == '1')
    c->allow_dead_store_drop = 0;
  // SEEAI_UNFUSED_CONVERSIONS=1: every relaxed product converts its own
  // activation (the same-session control of the producers' bf16 copies).
  if (const char* e = std::getenv("SEEAI_UNFUSED_CONVERSIONS"); e && e[0] == '1') c->allow_sinks = 0;
  // SEEAI_ATTENTION_BF16=1: relaxed attention on bf16 operands from the
  // start (seeai_set_attention_bf16 for a caller that sets it itself).
  if (const char* e = std::getenv("SEEAI_ATTENTION_BF16"); e && e[0] == '1') c->attn_bf16 = 1;
  // SEEAI_ATTN16_PLANS=0: relaxed bf16 attention on the f32-operand kernels
  // (the same-session control of the bf16 copies).
  if (const char* e = std::getenv("SEEAI_ATTN16_PLANS"); e && e[0] == '0') c->attn16_plans = 0;
  // SEEAI_ATTN_SAVED_MB: the cap on the forward's saved bf16 copies of q,
  // k and v (4096 MiB by default: C5's 16 layers take 1.6 GB).
  if (const char* e = std::getenv("SEEAI_ATTN_SAVED_MB"))
    c->a16_saved_cap = std::strtoull(e, nullptr, 10) << 20;
  int rc = Hip(c, hipSetDevice(device), "set device");
  if (rc == SEEAI_OK) rc = Hip(c, NoAllocScratchInit(device), "no-allocation workspace address");
  if (rc == SEEAI_OK) rc = Hip(c, hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking), "stream");
  if (rc == SEEAI_OK) rc = Hip(c, hipMalloc(&c->small, kSmallBytes), "small alloc");
  if (rc == SEEAI_OK) rc = Hip(c, hipMemset(c->small, 0, kSmallBytes), "small clear");
  if (rc == SEEAI_OK) rc = Hip(c, hipHostMalloc(reinterpret_cast<void**>(&c->host_flag), 64), "pinned");
  if (rc == SEEAI_OK)
    rc = Hip(c, hipHostMalloc(reinterpret_cast<void**>(&c->host_hyper), 64), "pinned step values");
  if (rc == SEEAI_OK)
    rc = Hip(c, hipEventCreateWithFlags(&c->hyper_copied, hipEventDisableTiming), "event");
  // SEEAI_GRAPHS=1: ranges replayed from captured graphs from the start
  // (seeai_set_graph_replay for a caller that sets it itself).
  if (const char* e = std::getenv("SEEAI_GRAPHS"); e && e[0] == '1') c->graph_replay = 1;
  if (rc != SEEAI_OK) {
    seeai_destroy(c);
    return rc;
  }
  c->stream = c->own_stream;
  *out = c;
  return SEEAI_OK;
}

void seeai_destroy(seeai_ctx* c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  DropGraphs(c);
  if (c->arena) (void)hipFree(c->arena);
  if (c->rodata) (void)hipFree(c->rodata);
  if (c->source) (void)hipFree(c->source);
  if (c->scratch) (void)hipFree(c->scratch);
  if (c->cvt) (void)hipFree(c->cvt);
  for (void* p : c->xcvt)
    if (p) (void)hipFree(p);
  if (c->pmax) (void)hipFree(c->pmax);
  if (c->a16) (void)hipFree(c->a16);
  DropSavedCopies(c);
  DropShadows(c);
  if (c->small) (void)hipFree(c->small);
  if (c->host_flag) (void)hipHostFree(c->host_flag);
  if (c->hyper_copied) (void)hipEventDestroy(c->hyper_copied);
  if (c->capture_stream) (void)hipStreamDestroy(c->capture_stream);
  if (c->host_hyper) (void)hipHostFree(c->host_hyper);
  if (c->own_stream) (void)hipStreamDestroy(c->own_stream);
  delete c;
}

const char* seeai_last_error(const seeai_ctx* c) { return c ? c->err.c_str() : "no context"; }

int seeai_set_stream(seeai_ctx* c, void* stream) {
  if (!c) return SEEAI_INVALID;
  c->stream = static_cast<hipStream_t>(stream);
  return SEEAI_OK;
}
void* seeai_get_stream(seeai_ctx* c) { return c ? static_cast<void*>(c->stream) : nullptr; }
int seeai_set_relaxed(seeai_ctx* c, int allow) {
  if (!c) return SEEAI_INVALID;
  DropGraphs(c);
  c->allow_relaxed = allow ? 1 : 0;
  return SEEAI_OK;
}
uint64_t seeai_relaxed_executions(const seeai_ctx* c) { return c ? c->relaxed : 0; }
int seeai_set_attention_bf16(seeai_ctx* c, int on) {
  if (!c) return SEEAI_INVALID;
  DropGraphs(c);
  c->attn_bf16 = on ? 1 : 0;
  return SEEAI_OK;
}

int seeai_bind(seeai_ctx* c, uint64_t arena_bytes, const void* rodata, uint64_t rodata_bytes) {
  if (!c) return SEEAI_INVALID;
  DropGraphs(c);
  ForgetCopies(c);
  c->dead_prog = nullptr;  // dead-store decisions name the old binding's pointers
  const uint64_t bytes = (arena_bytes + kArenaAlignment - 1) / kArenaAlignment * kArenaAlignment;
  uint8_t* arena = nullptr;
  uint8_t* ro = nullptr;
  // Build the new binding completely before replacing the old one, so a
  // refused bind leaves the previous binding executable (backend.h:89-98).
  hipError_t e = hipMalloc(&arena, bytes ? bytes : kArenaAlignment);
  if (e == hipSuccess) e = hipMemsetAsync(arena, 0, bytes ? bytes : kArenaAlignment, c->stream);
  if (e == hipSuccess && rodata_bytes) e = hipMalloc(&ro, rodata_bytes);
  if (e == hipSuccess && rodata_bytes)
    e = hipMemcpyAsync(ro, rodata, rodata_bytes, hipMemcpyHostToDevice, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) {
    if (arena) (void)hipFree(arena);
    if (ro) (void)hipFree(ro);
    return Hip(c, e, "bind");
  }
  DropShadows(c);  // made from the old rodata
  DropSavedCopies(c);  // of the old arena's activations
  if (c->arena) (void)hipFree(c->arena);
  if (c->rodata) (void)hipFree(c->rodata);
  c->arena = arena;
  c->arena_bytes = bytes;
  c->rodata = ro;
  c->rodata_bytes = rodata_bytes;
  return SEEAI_OK;
}

int seeai_bind_source(seeai_ctx* c, const void* data, uint64_t bytes) {
  if (!c) return SEEAI_INVALID;
  DropGraphs(c);
  ForgetCopies(c);
  c->dead_prog = nullptr;
  SEEAI_TRY(c, hipStreamSynchronize(c->stream), "bind_source drain");
  DropShadows(c);  // some may be of the old source image
  if (c->source) (void)hipFree(c->source);
  c->source = nullptr;
  c->source_bytes = 0;
  if (!data || !bytes) return SEEAI_OK;
  SEEAI_TRY(c, hipMalloc(&c->source, bytes), "bind_source alloc");
  SEEAI_TRY(c, hipMemcpy(c->source, data, bytes, hipMemcpyHostToDevice), "bind_source copy");
  c->source_bytes = bytes;
  return SEEAI_OK;
}

int seeai_upload(seeai_ctx* c, uint64_t off, const void* src, uint64_t bytes) {
  if (!c || !c->arena || off + bytes > c->arena_bytes) return Fail(c, SEEAI_INVALID, "upload: extent outside the arena");
  if (!bytes) return SEEAI_OK;
  ForgetCopies(c);  // the arena changed outside the program
  SEEAI_TRY(c, hipMemcpyAsync(c->arena + off, src, bytes, hipMemcpyHostToDevice, c->stream), "upload");
  // The source buffer is the caller's pageable memory: complete the copy
  // before returning so the caller may reuse it at once.
  SEEAI_TRY(c, hipStreamSynchronize(c->stream), "upload sync");
  return SEEAI_OK;
}

int seeai_download(seeai_ctx* c, uint64_t off, void* dst, uint64_t bytes) {
  if (!c || !c->arena || off + bytes > c->arena_bytes) return Fail(c, SEEAI_INVALID, "download: extent outside the arena");
  if (!bytes) return SEEAI_OK;
  SEEAI_TRY(c, hipMemcpyAsync(dst, c->arena + off, bytes, hipMemcpyDeviceToHost, c->stream), "download");
  SEEAI_TRY(c, hipStreamSynchronize(c->stream), "download sync");
  return SEEAI_OK;
}

struct seeai_feeder {
  seeai_ctx* ctx = nullptr;
  int device = 0;
  hipStream_t stream = nullptr;  // the uploads, at the default priority
  uint64_t input_bytes = 0, label_bytes = 0;
  uint8_t* pinned[2] = {nullptr, nullptr};  // hipHostMalloc
  uint8_t* staged[2] = {nullptr, nullptr};  // device
  hipEvent_t uploaded[2] = {nullptr, nullptr};
  hipEvent_t consumed[2] = {nullptr, nullptr};  // the arena copy that read the slot
  bool upload_recorded[2] = {false, false};
  bool consume_recorded[2] = {false, false};
  int head = 0, tail = 0, count = 0;  // next slot to stage, next to hand over, staged
  std::mutex mu;
  std::string error;
};

namespace {
int FeederFail(seeai_feeder* f, int status, const char* what, hipError_t e) {
  f->error = std::string("feeder: ") + what + ": " + hipGetErrorString(e);
  return status;
}
}  // namespace

int seeai_feeder_create(seeai_ctx* c, uint64_t input_bytes, uint64_t label_bytes,
                        seeai_feeder** out) {
  if (!c || !out || input_bytes == 0) return Fail(c, SEEAI_INVALID, "feeder_create: no input slot");
  *out = nullptr;
  auto* f = new seeai_feeder;
  f->ctx = c;
  f->device = c->device;
  f->input_bytes = input_bytes;
  f->label_bytes = label_bytes;
  const uint64_t bytes = input_bytes + label_bytes;
  hipError_t e = hipSetDevice(c->device);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&f->stream, hipStreamNonBlocking);
  for (int s = 0; s < 2 && e == hipSuccess; ++s) {
    e = hipHostMalloc(reinterpret_cast<void**>(&f->pinned[s]), bytes, hipHostMallocDefault);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&f->staged[s]), bytes);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&f->uploaded[s], hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&f->consumed[s], hipEventDisableTiming);
  }
  if (e != hipSuccess) {
    seeai_feeder_destroy(f);
    return Fail(c, SEEAI_HIP_ERROR, "feeder_create: %s", hipGetErrorString(e));
  }
  *out = f;
  return SEEAI_OK;
}

void seeai_feeder_destroy(seeai_feeder* f) {
  if (!f) return;
  (void)hipSetDevice(f->device);
  if (f->stream) (void)hipStreamSynchronize(f->stream);
  if (f->ctx && f->ctx->stream) (void)hipStreamSynchronize(f->ctx->stream);
  for (int s = 0; s < 2; ++s) {
    if (f->uploaded[s]) (void)hipEventDestroy(f->uploaded[s]);
    if (f->consumed[s]) (void)hipEventDestroy(f->consumed[s]);
    if (f->staged[s]) (void)hipFree(f->staged[s]);
    if (f->pinned[s]) (void)hipHostFree(f->pinned[s]);
  }
  if (f->stream) (void)hipStreamDestroy(f->stream);
  delete f;
}

const char* seeai_feeder_last_error(const seeai_feeder* f) {
  return f ? f->error.c_str() : "no feeder";
}

int seeai_feeder_stage(seeai_feeder* f, const void* input, const void* labels) {
  if (!f || !input || (f->label_bytes && !labels)) return SEEAI_INVALID;
  int slot;
  bool consumed;
  {
    std::lock_guard<std::mutex> lock(f->mu);
    if (f->count == 2) {
      f->error = "feeder: two batches are already staged";
      return SEEAI_INVALID;
    }
    slot = f->head;
    consumed = f->consume_recorded[slot];
  }
  hipError_t e = hipSetDevice(f->device);
  if (e != hipSuccess) return FeederFail(f, SEEAI_HIP_ERROR, "set device", e);
  // The pinned slot's previous upload has left it before it is refilled.
  if (f->upload_recorded[slot] && (e = hipEventSynchronize(f->uploaded[slot])) != hipSuccess)
    return FeederFail(f, SEEAI_HIP_ERROR, "upload wait", e);
  std::memcpy(f->pinned[slot], input, f->input_bytes);
  if (f->label_bytes) std::memcpy(f->pinned[slot] + f->input_bytes, labels, f->label_bytes);
  // The device slot is refilled after the arena copy that read it.
  if (consumed && (e = hipStreamWaitEvent(f->stream, f->consumed[slot], 0)) != hipSuccess)
    return FeederFail(f, SEEAI_HIP_ERROR, "consume wait", e);
  if ((e = hipMemcpyAsync(f->staged[slot], f->pinned[slot], f->input_bytes + f->label_bytes,
                          hipMemcpyHostToDevice, f->stream)) != hipSuccess)
    return FeederFail(f, SEEAI_HIP_ERROR, "upload", e);
  if ((e = hipEventRecord(f->uploaded[slot], f->stream)) != hipSuccess)
    return FeederFail(f, SEEAI_HIP_ERROR, "upload event", e);
  f->upload_recorded[slot] = true;
  std::lock_guard<std::mutex> lock(f->mu);
  f->head ^= 1;
  ++f->count;
  return SEEAI_OK;
}

int seeai_feeder_next(seeai_feeder* f, uint64_t input_off, uint64_t label_off) {
  if (!f) return SEEAI_INVALID;
  seeai_ctx* c = f->ctx;
  if (!c->arena || input_off + f->input_bytes > c->arena_bytes ||
      (f->label_bytes && label_off + f->label_bytes > c->arena_bytes))
    return Fail(c, SEEAI_INVALID, "feeder_next: I/O slot outside the arena");
  int slot;
  {
    std::lock_guard<std::mutex> lock(f->mu);
    if (f->count == 0) return Fail(c, SEEAI_INVALID, "feeder_next: no batch staged");
    slot = f->tail;
  }
  SEEAI_TRY(c, hipStreamWaitEvent(c->stream, f->uploaded[slot], 0), "feeder_next wait");
  SEEAI_TRY(c, hipMemcpyAsync(c->arena + input_off, f->staged[slot], f->input_bytes,
                              hipMemcpyDeviceToDevice, c->stream), "feeder_next input");
  if (f->label_bytes)
    SEEAI_TRY(c, hipMemcpyAsync(c->arena + label_off, f->staged[slot] + f->input_bytes,
                                f->label_bytes, hipMemcpyDeviceToDevice, c->stream),
              "feeder_next labels");
  SEEAI_TRY(c, hipEventRecord(f->consumed[slot], c->stream), "feeder_next event");
  ForgetCopies(c);  // the arena changed outside the program
  std::lock_guard<std::mutex> lock(f->mu);
  f->consume_recorded[slot] = true;
  f->tail ^= 1;
  --f->count;
  return SEEAI_OK;
}

void* seeai_arena(seeai_ctx* c) { return c ? c->arena : nullptr; }
uint64_t seeai_arena_bytes(const seeai_ctx* c) { return c ? c->arena_bytes : 0; }

namespace {

// Byte extents a GEMM reads and writes.
struct Extent {
  const uint8_t* p;
  uint64_t n;
};
uint64_t BElem(const GemmArgs& a) { return a.b_kind == 1 ? 1 : a.b_kind == 2 ? 2 : 4; }
int GemmReads(const GemmArgs& a, Extent* out) {
  int k = 0;
  const auto add = [&](const void* p, uint64_t n) {
    if (p && n) out[k++] = {static_cast<const uint8_t*>(p), n};
  };
  add(a.A, a.M * a.K * 4);
  add(a.B, a.N * a.K * BElem(a));
  add(a.addend, a.M * a.N * 4);
  add(a.bias, a.N * 4);
  add(a.b_col_scale, a.N * 4);
  add(a.a_k_scale, a.K * 4);
  if (a.accumulate) add(a.C, a.M * a.N * 4);
  return k;
}
Extent GemmWrites(const GemmArgs& a) { return {reinterpret_cast<const uint8_t*>(a.C), a.M * a.N * 4}; }
bool Hits(const Extent& x, const Extent* set, int n) {
  for (int i = 0; i < n; ++i)
    if (Overlap(x.p, x.n, set[i].p, set[i].n)) return true;
  return false;
}


// --- Dead-store scan ----------------------------------------------------------
// Every operand extent of an instruction (the validator's roles and sizes,
// plan_validator.cc:368-745, as operands.h states them), resolved to device
// addresses.  False for opcodes not modelled there.
bool TouchExtents(seeai_ctx* c, const Instruction& ins, Touch* out, int* n) {
  const Ptrs R{c};
  OperandRef ops[kMaxOperands];
  const int count = DescribeOperands(ins, ops);
  if (count < 0) return false;
  int k = 0;
  for (int i = 0; i < count; ++i)
    if (ops[i].ref != kNullRef && ops[i].elems)
      out[k++] = {R.at(ops[i].ref), ops[i].elems * ops[i].elem_bytes, ops[i].write};
  *n = k;
  return true;
}

// Whether an opcode's write extents are stores alone; the others read what
// they write (metal_backend.mm:1139-1152).
bool OverwritesWhatItWrites(uint16_t op) {
  switch (op) {
    case 4: case 42: case 28: case 53: case 54: case 17: case 18: case 48:
      return false;
    default:
      return true;
  }
}

// Whether the store of E made by instruction `writer` (before `from`) is
// dead, under the reference's rule for a LoRA site's base value
// (metal_backend.mm:1281-1313): over the whole program, not the range, the
// first instruction at or after `from` to touch E writes all of it, reads
// none of it and overwrites what it writes, or no instruction touches it.
// The program runs again at the next step, so the scan wraps round to the
// start and ends at the writer: a value that only the next step's earlier
// instructions read keeps its store.  An instruction whose extents are not
// modelled keeps the store.
int SiluOperand(seeai_ctx* c, uint64_t at_idx, const float* p0, const float* p1, const float* x,
                uint64_t n);

// Whether the SwiGLU backward triple at index t (kMulEW, kMulEW, kSiluBwd)
// runs as the fused pass that forms its y = SiLU(x) rather than reading it,
// and E is exactly that y, read by nothing else of the triple: the same
// checks the pass makes (TryFuseElementwise), on the same program words.
bool SwigluBwdRecomputes(seeai_ctx* c, uint64_t t, const Extent& E) {
  if (!c->allow_fusion || !c->prog || !c->cur_at || t + 2 >= c->range_end) return false;
  Instruction i0, i1, i2;
  std::memcpy(&i0, c->prog + t * 64, sizeof i0);
  std::memcpy(&i1, c->prog + (t + 1) * 64, sizeof i1);
  std::memcpy(&i2, c->prog + (t + 2) * 64, sizeof i2);
  const uint64_t n = i0.out[0];
  if (i0.opcode != 21 || i1.opcode != 21 || i2.opcode != 25 || i1.out[0] != n ||
      i2.out[0] != n || E.n != n * 4)
    return false;
  const bool first = i2.in[0] == i0.in[2];
  if (!first && i2.in[0] != i1.in[2]) return false;
  const Instruction& m1 = first ? i0 : i1;
  const Instruction& m2 = first ? i1 : i0;
  const Ptrs R{c};
  const float *a1 = R.f(m1.in[0]), *b1 = R.f(m1.in[1]), *a2 = R.f(m2.in[0]), *b2 = R.f(m2.in[1]),
              *x = R.f(i2.in[1]);
  float *o1 = R.f(m1.in[2]), *o2 = R.f(m2.in[2]), *dx = R.f(i2.in[2]);
  const uint64_t nb = n * 4;
  for (const float* o : {o1, o2, dx}) {
    const auto* op = reinterpret_cast<const uint8_t*>(o);
    for (const float* q : {o1, o2, dx})
      if (q != o && Overlap(op, nb, reinterpret_cast<const uint8_t*>(q), nb)) return false;
    for (const float* q : {a1, b1, a2, b2, x})
      if (Overlap(op, nb, reinterpret_cast<const uint8_t*>(q), nb)) return false;
  }
  if (!SwigluFits(n, {a1, b1, o1, a2, b2, o2, x, dx})) return false;
  const int silu = SiluOperand(c, t, a2, b2, x, n);
  const float* y = silu == 1 ? a2 : silu == 2 ? b2 : nullptr;
  if (!y || reinterpret_cast<const uint8_t*>(y) != E.p) return false;
  const float* other = silu == 1 ? b2 : a2;
  for (const float* q : {a1, b1, other, x})
    if (Overlap(reinterpret_cast<const uint8_t*>(q), nb, E.p, E.n)) return false;
  return true;
}

bool DeadFrom(seeai_ctx* c, uint64_t writer, uint64_t from, const Extent& E) {
  for (uint64_t i = from; i < c->prog_count + writer + 1; ++i) {
    const uint64_t k = i < c->prog_count ? i : i - c->prog_count;
    Instruction ins;
    std::memcpy(&ins, c->prog + k * 64, sizeof ins);
    Touch t[16];
    int n = 0;
    if (!TouchExtents(c, ins, t, &n)) return false;
    bool touched = false, read = false, covered = false;
    for (int i = 0; i < n; ++i) {
      if (!Overlap(t[i].p, t[i].n, E.p, E.n)) continue;
      touched = true;
      if (!t[i].write) read = true;
      else if (t[i].p <= E.p && E.p + E.n <= t[i].p + t[i].n) covered = true;
    }
    // A read that the fused SwiGLU backward replaces by forming y itself is
    // none (the triple reads E nowhere else; scanning goes on past it).
    if (touched && read && !covered && i < c->prog_count &&
        (SwigluBwdRecomputes(c, k, E) || (k > 0 && SwigluBwdRecomputes(c, k - 1, E))))
      continue;
    if (touched) return covered && !read && OverwritesWhatItWrites(ins.opcode);
  }
  return true;
}

// Range-analysis answers, decided once per program, instruction and asking
// site (each site asks one question of an instruction: 0 the producers'
// sinks and the elementwise chains, 1 the low-rank fold, 2 the residual add
// behind a GEMM, 3 the residual add behind a normalisation's gradient -- all
// DeadFrom -- and 4 the SwiGLU backward's SiLU recompute): an answer depends
// on the program's words and the binding alone (dropped at bind).  -1:
// undecided.
constexpr int kDeadSites = 5;
int8_t& RangeMemo(seeai_ctx* c, uint64_t at_idx, int site) {
  if (c->dead_prog != c->prog || c->dead.size() != c->prog_count * kDeadSites ||
      c->dead_hash != c->prog_hash) {
    c->dead_prog = c->prog;
    c->dead_hash = c->prog_hash;
    c->dead.assign(c->prog_count * kDeadSites, -1);
  }
  return c->dead[at_idx * kDeadSites + site];
}
bool DeadStore(seeai_ctx* c, uint64_t at_idx, uint64_t from, const Extent& E, int site = 0) {
  if (!c->allow_dead_store_drop) return false;
  int8_t& v = RangeMemo(c, at_idx, site);
  if (v < 0) v = DeadFrom(c, at_idx, from, E) ? 1 : 0;
  if (v) ++c->dropped_stores;
  return v != 0;
}

// Which operand of the SwiGLU backward's second product (instruction
// `at_idx`, n floats each) is y = SiLU(x) for this pass's x, by the range:
// y's last writer before the pass is a SiLU forward (opcode 24) of exactly x
// into exactly y, and no instruction since writes into x or y.  The pass
// then forms y from x as that forward did (the same expression, so the same
// bits) instead of reading it.  0: neither (y is read); 1: p0; 2: p1.
int SiluOperand(seeai_ctx* c, uint64_t at_idx, const float* p0, const float* p1, const float* x,
                uint64_t n) {
  if (!c->allow_fusion || !c->prog || !c->cur_at) return 0;
  int8_t& v = RangeMemo(c, at_idx, 4);
  if (v >= 0) return v;
  v = 0;
  const auto* xb = reinterpret_cast<const uint8_t*>(x);
  const float* cand[2] = {p0, p1};
  bool alive[2] = {p0 != x, p1 != x};
  for (uint64_t i = at_idx; i-- > 0;) {
    Instruction ins;
    std::memcpy(&ins, c->prog + i * 64, sizeof ins);
    Touch t[16];
    int nt = 0;
    if (!TouchExtents(c, ins, t, &nt)) return v;
    const Ptrs R{c};
    for (int k = 0; k < 2; ++k) {
      if (!alive[k]) continue;
      const auto* yb = reinterpret_cast<const uint8_t*>(cand[k]);
      bool hit = false;
      for (int j = 0; j < nt; ++j)
        if (t[j].write && Overlap(t[j].p, t[j].n, yb, n * 4)) hit = true;
      if (!hit) continue;
      if (ins.opcode == 24 && ins.out[0] == n && R.f(ins.in[0]) == x && R.f(ins.in[1]) == cand[k])
        return v = static_cast<int8_t>(k + 1);
      alive[k] = false;  // written by something else
    }
    for (int j = 0; j < nt; ++j)
      if (t[j].write && Overlap(t[j].p, t[j].n, xb, n * 4)) return v;  // x changed since
    if (!alive[0] && !alive[1]) return v;
  }
  return v;
}

// Conversion fused into a producer: when the instruction after index `last`
// is a relaxed frozen-weight product on the direct-to-LDS path whose
// activation is the producer's output `out` (n floats, K a multiple of 32),
// `sink` writes that product's bf16 copy into the conversion workspace as
// the producer stores, and the f32 store is dropped where nothing after the
// product reads `out` (the dead-store rule, decided for instruction
// `writer`, memoised under `site`).  Slot 2 (a producer's second sink): the
// product is the one after the next, into the second workspace, and the
// instruction between is a GEMM that neither reads nor writes `out` (so the
// dead-store question starts after the product, and ConvertedAlready finds
// the copy when the product runs).  *ga: the product's arguments,
// for SinkDone.
bool PlanSink(seeai_ctx* c, uint64_t last, uint64_t writer, const float* out, uint64_t n,
              Bf16Sink* sink, GemmArgs* ga, int slot, int site) {
  const uint64_t at = last + static_cast<uint64_t>(slot);
  if (!c->allow_fusion || !c->allow_sinks || !c->prog || at >= c->range_end) return false;
  if (slot == 2) {  // the product between: a GEMM clear of `out` (no read, no write)
    Instruction mid;
    std::memcpy(&mid, c->prog + (last + 1) * 64, sizeof mid);
    GemmArgs m{};
    Touch t[16];
    int nt = 0;
    if (!DecodeGemm(c, mid, &m) || !TouchExtents(c, mid, t, &nt)) return false;
    for (int i = 0; i < nt; ++i)
      if (Overlap(t[i].p, t[i].n, reinterpret_cast<const uint8_t*>(out), n * 4)) return false;
  }
  Instruction nx;
  std::memcpy(&nx, c->prog + at * 64, sizeof nx);
  GemmArgs a{};
  if (!DecodeGemm(c, nx, &a)) return false;
  a.relaxed = (nx.flags & kFlagRelaxed) && c->allow_relaxed ? 1 : 0;
  a.policy = &c->policy;
  if (!a.relaxed || !c->allow_dma || !Bf16DmaFits(a) || !Immutable(c, a.B)) return false;
  const size_t cap = slot == 2 ? c->xcvt_bytes : c->cvt_bytes;
  if (a.A != out || a.M * a.K != n || a.K % 32 != 0 || a.M * a.K * 2 > cap) return false;
  if (reinterpret_cast<uintptr_t>(a.a_k_scale) & 15) return false;
  sink->out = static_cast<uint16_t*>(slot == 2 ? c->xcvt[0] : c->cvt);
  sink->ks = a.a_k_scale;
  sink->alpha = a.alpha_a;
  sink->K = static_cast<uint32_t>(a.K);
  sink->store_f32 = DeadStore(c, writer, at + 1,
                              Extent{reinterpret_cast<const uint8_t*>(out), n * 4}, site)
                        ? 0
                        : 1;
  *ga = a;
  return true;
}

// After a producer ran with its sink: the workspace holds the product's A'
// (its ConvertedAlready finds it; slot 2's product has the GEMM PlanSink
// checked between them).
void SinkDone(seeai_ctx* c, uint64_t last, const GemmArgs& a, int slot) {
  (slot == 2 ? c->xcvt_key[0] : c->cvt_key) =
      seeai_ctx::CvtKey{a.A, a.M, a.K, a.alpha_a, a.a_k_scale, c->prog + last * 64};
  ++c->sinks;
}

// A sink whose product comes later in the range: the first relaxed
// frozen-weight product on the direct-to-LDS path that takes the producer's
// output `out` (producer at index `last`) as its activation, within
// kFarWindow instructions, no instruction before it writing into `out`
// (those that read `out` -- exact GEMMs taking it as an operand -- read the
// f32 store, which is always kept).  The copy goes to extra slots 1 .. 3 in
// turn (a slot taken again before its product runs only costs that product
// its own conversion: its key no longer matches).  *key_at: the last
// instruction before the product that is not a GEMM, from where
// ConvertedAlready walks the GEMMs to the product; *ga: the product's
// arguments.
bool PlanFarSink(seeai_ctx* c, uint64_t last, const float* out, uint64_t n, Bf16Sink* sink,
                 GemmArgs* ga, int* xslot, uint64_t* key_at) {
  constexpr uint64_t kFarWindow = 24;
  if (!c->allow_fusion || !c->allow_sinks || !c->prog || !c->xcvt[1]) return false;
  const auto* o = reinterpret_cast<const uint8_t*>(out);
  uint64_t free_at = last;
  for (uint64_t f = last + 1; f < c->range_end && f <= last + kFarWindow; ++f) {
    Instruction ins;
    std::memcpy(&ins, c->prog + f * 64, sizeof ins);
    GemmArgs a{};
    const bool gemm = DecodeGemm(c, ins, &a) != nullptr;
    if (gemm && a.A == out && (ins.flags & kFlagRelaxed)) {
      a.relaxed = c->allow_relaxed ? 1 : 0;
      a.policy = &c->policy;
      if (!a.relaxed || !c->allow_dma || !Bf16DmaFits(a) || !Immutable(c, a.B)) return false;
      if (a.M * a.K != n || a.K % 32 != 0 || a.M * a.K * 2 > c->xcvt_bytes) return false;
      if (reinterpret_cast<uintptr_t>(a.a_k_scale) & 15) return false;
      const int s = 1 + c->far_next;
      c->far_next = (c->far_next + 1) % (seeai_ctx::kXSlots - 1);
      sink->out = static_cast<uint16_t*>(c->xcvt[s]);
      sink->ks = a.a_k_scale;
      sink->alpha = a.alpha_a;
      sink->K = static_cast<uint32_t>(a.K);
      sink->store_f32 = 1;
      *ga = a;
      *xslot = s;
      *key_at = free_at;
      return true;
    }
    Touch t[16];
    int nt = 0;
    if (!TouchExtents(c, ins, t, &nt)) return false;
    for (int i = 0; i < nt; ++i)
      if (t[i].write && Overlap(t[i].p, t[i].n, o, n * 4)) return false;
    if (!gemm) free_at = f;
  }
  return false;
}

void FarSinkDone(seeai_ctx* c, uint64_t key_at, const GemmArgs& a, int xslot) {
  c->xcvt_key[xslot] =
      seeai_ctx::CvtKey{a.A, a.M, a.K, a.alpha_a, a.a_k_scale, c->prog + key_at * 64};
  ++c->sinks;
}

// Range-level fusion of a LoRA site (the seam's whole-program visibility,
// backend.h:139-142; the reference's Metal backend folds the same pair,
// metal_kernels.h:290-358, docs/runtime.md:119).  A relaxed frozen-weight
// product writing C on the direct-to-LDS kernel, followed -- next, or after
// up to three exact GEMMs (the site's t = x A; on a backward site its dt, dB
// and dA) that neither touch C nor write what the product reads -- by an
// exact rank-r GEMM (NN or NT, r <= 16, no bias or activation) whose addend
// is C, runs as one dispatch: the in-between GEMMs first, in their order,
// then the frozen product with the rank-r term in its epilogue, which
// forms C as before, stores it, and writes C' = C + the rank-r product in the
// rank-r instruction's own chain.  The arena holds the bytes of the separate
// dispatches.  Refused (each runs at its place) when an output overlaps
// anything the fused pass reads or the other output.  Returns -1 when the
// instructions do not fuse.
int TryFuseLowRank(seeai_ctx* c, const Instruction& ins, const uint8_t* at,
                   const seeai_step_params& P) {
  if (!c->allow_fusion || !c->allow_lowrank || !c->allow_relaxed || !c->allow_dma || !c->prog ||
      at < c->prog ||
      at >= c->prog + c->prog_count * 64 || (at - c->prog) % 64 != 0)
    return -1;
  if (!(ins.flags & kFlagRelaxed)) return -1;
  GemmArgs a{};
  if (!DecodeGemm(c, ins, &a)) return -1;
  a.relaxed = 1;
  a.policy = &c->policy;  // the same kernel choice the product makes alone
  if (a.accumulate || !Bf16DmaFits(a) || !Immutable(c, a.B)) return -1;
  const uint64_t idx = static_cast<uint64_t>(at - c->prog) / 64;
  Extent reads_a[8];
  const int na = GemmReads(a, reads_a);
  const Extent out_a = GemmWrites(a);
  constexpr uint64_t kMaxGap = 3;
  Instruction mids[kMaxGap];
  for (uint64_t gap = 0; gap <= kMaxGap; ++gap) {
    const uint64_t j = idx + 1 + gap;
    if (j >= c->range_end) return -1;
    Instruction nj;
    std::memcpy(&nj, c->prog + j * 64, sizeof nj);
    const bool exact_j = !(nj.flags & kFlagRelaxed);
    if ((nj.opcode == 1 || nj.opcode == 2) && exact_j && (nj.flags & kFlagGemmAddend) &&
        ((nj.flags >> 1) & 3) == 0 && nj.in[3] == ins.in[2]) {
      GemmArgs b{};
      DecodeGemm(c, nj, &b);
      if (b.M != a.M || b.N != a.N || b.bias) return -1;
      a.lr_t = b.A;
      a.lr_b = static_cast<const float*>(b.B);
      a.lr_out = b.C;
      a.lr_layout = b.layout;
      a.lr_k = static_cast<int>(b.K);
      a.lr_alpha = b.layout == 0 ? b.alpha_a : b.alpha_dot;
      a.lr_store_c = 1;
      if (!Bf16DmaLowRankFits(a)) return -1;
      // The fused pass reads A, the scales, t and the rank operand, writes C
      // and C'.
      const Extent out_b = GemmWrites(b);
      const Extent t_b{reinterpret_cast<const uint8_t*>(b.A), b.M * b.K * 4};
      const Extent r_b{static_cast<const uint8_t*>(b.B), b.N * b.K * 4};
      // C' may be written over the product's own addend, exactly (the dX
      // chains' ping-pong buffers): each element's addend is read by the
      // lane that then writes its C', before it does.
      const bool over_addend = a.addend &&
                               reinterpret_cast<const uint8_t*>(a.addend) == out_b.p &&
                               out_b.n == a.M * a.N * 4;
      bool b_hits_reads = false;
      for (int i = 0; i < na; ++i)
        if (!(over_addend && reads_a[i].p == out_b.p && reads_a[i].n == out_b.n) &&
            Overlap(out_b.p, out_b.n, reads_a[i].p, reads_a[i].n))
          b_hits_reads = true;
      if (Overlap(out_a.p, out_a.n, out_b.p, out_b.n) || Hits(out_a, &t_b, 1) ||
          Hits(out_a, &r_b, 1) || b_hits_reads || Hits(out_b, &t_b, 1) || Hits(out_b, &r_b, 1))
        return -1;
      // C's store is dropped where the rest of the range overwrites C
      // before anything reads it.
      if (DeadStore(c, idx, j + 1, out_a, 1)) a.lr_store_c = 0;
      // A residual add of C' next (kAddEW, C' on one side, C' read by
      // nothing after it: the dX chains on NT sites, the forward's residual
      // behind an NN site of rank 8 or 16 with a plain epilogue) joins the
      // epilogue: the add's output takes R + C' in C''s place.  Its output may be R
      // itself, or C when C's store is dropped; it misses everything else
      // the pass reads.
      bool res_add = false;
      if (j + 1 < c->range_end && !over_addend) {
        Instruction ad;
        std::memcpy(&ad, c->prog + (j + 1) * 64, sizeof ad);
        const Ptrs R{c};
        if (ad.opcode == 5 && ad.out[0] == a.M * a.N &&
            (R.f(ad.in[0]) == b.C) != (R.f(ad.in[1]) == b.C)) {
          const float* res = R.f(ad.in[0]) == b.C ? R.f(ad.in[1]) : R.f(ad.in[0]);
          float* aout = R.f(ad.in[2]);
          const uint64_t nb = a.M * a.N * 4;
          const Extent e_res{reinterpret_cast<const uint8_t*>(res), nb};
          const Extent e_out{reinterpret_cast<const uint8_t*>(aout), nb};
          const bool clear =
              !Hits(e_out, reads_a, na) && !Hits(e_out, &t_b, 1) && !Hits(e_out, &r_b, 1) &&
              !Hits(e_res, &out_b, 1) && (aout == res || !Hits(e_out, &e_res, 1)) &&
              (!a.lr_store_c || (!Hits(e_out, &out_a, 1) && !Hits(e_res, &out_a, 1)));
          GemmArgs t = a;
          t.lr_res = res;
          t.lr_out = aout;
          if (clear && Bf16DmaLowRankFits(t) && DeadStore(c, j, j + 2, out_b, 2)) {
            a = t;
            res_add = true;
          }
        }
      }
      // The site's output read next by a bf16-copy attention: its copy is
      // written in the epilogue (the constant-rank pass only).
      int pre_slot = -1;
      uint64_t pre_at = 0;
      {
        GemmArgs t = a;
        t.lr_sink = PlanAttnCopy(c, res_add ? j + 1 : j, a.lr_out, a.M * a.N, &pre_slot, &pre_at);
        if (t.lr_sink && Bf16DmaLowRankFits(t)) a = t;
        else pre_slot = -1;
      }
      for (uint64_t g = 0; g < gap; ++g)
        if (int rc = ExecuteOne(c, mids[g], P)) return rc;
      Relaxed(c, ins);
      if (int rc = GemmBf16Dma(c, a, "gemm.low_rank")) return rc;
      if (pre_slot >= 0) {
        c->a16_pre[pre_slot].src = a.lr_out;
        c->a16_pre[pre_slot].at = pre_at;
        c->a16_pre[pre_slot].epoch = c->a16_epoch;
      }
      c->ndone = 0;
      for (uint64_t g = 0; g < gap; ++g) c->done[c->ndone++] = c->prog + (idx + 1 + g) * 64;
      c->done[c->ndone++] = c->prog + j * 64;
      if (res_add) c->done[c->ndone++] = c->prog + (j + 1) * 64;
      ++c->fused;
      return SEEAI_OK;
    }
    // Not the rank-r GEMM: it may sit between the two as an exact GEMM that
    // writes nothing the product reads or writes and reads nothing the
    // product writes (it then runs first).
    if (gap == kMaxGap) return -1;
    GemmArgs m{};
    if (!DecodeGemm(c, nj, &m) || ((nj.flags & kFlagRelaxed) && c->allow_relaxed)) return -1;
    Extent reads_m[8];
    const int nm = GemmReads(m, reads_m);
    const Extent out_m = GemmWrites(m);
    if (Hits(out_m, reads_a, na) || Overlap(out_m.p, out_m.n, out_a.p, out_a.n) ||
        Hits(out_a, reads_m, nm))
      return -1;
    mids[gap] = nj;
  }
  return -1;
}

// Range-level fusion of SwiGLU's elementwise chains (the seam's
// whole-program visibility, backend.h:139-142): kSiluFwd followed by a
// kMulEW of its output (y = SiLU(x), h = y * u), and two kMulEW followed by
// the kSiluBwd of one of their outputs (dsg = dh * up, dup = dh * sg,
// dgt = SiluBwd(dsg, gt)) run as one pass each over the same n, with the
// standalone kernels' expressions; every output is still written.  Refused
// when the element counts differ or any output overlaps another operand.
// Returns -1 when the instructions do not fuse.
int TryFuseElementwise(seeai_ctx* c, const Instruction& ins, const uint8_t* at);

// A run of adjacent kAdamWStep instructions without a fused clip (the end of
// every train program: one per adapter tensor) as one launch: each
// element's update is AdamWKernel's, so the bits are the separate launches'.
// Refused when any tensor's p, m or v overlaps another operand of the run.
int TryFuseAdamW(seeai_ctx* c, const Instruction& ins, const uint8_t* at,
                 const seeai_step_params& P) {
  if (!c->allow_fusion || ins.opcode != 18 || !c->prog || at < c->prog ||
      at >= c->prog + c->prog_count * 64 || (at - c->prog) % 64 != 0)
    return -1;
  const uint64_t idx = static_cast<uint64_t>(at - c->prog) / 64;
  const Ptrs R{c};
  AdamWTable tab{};
  std::vector<std::pair<const uint8_t*, uint64_t>> writes, reads;
  for (uint64_t j = idx; j < c->range_end && tab.count < kAdamWMulti; ++j) {
    Instruction x;
    std::memcpy(&x, c->prog + j * 64, sizeof x);
    if (x.opcode != 18 || BitsToF32(x.out[1]) > 0.0f || x.out[0] == 0) break;
    const uint64_t nb = x.out[0] * 4;
    const uint8_t* ops[4] = {R.at(x.in[0]), R.at(x.in[1]), R.at(x.in[2]), R.at(x.in[3])};
    bool clash = false;
    for (int w : {0, 2, 3}) {
      for (const auto& o : writes) clash |= Overlap(ops[w], nb, o.first, o.second);
      for (const auto& o : reads) clash |= Overlap(ops[w], nb, o.first, o.second);
    }
    for (const auto& o : writes) clash |= Overlap(ops[1], nb, o.first, o.second);
    for (int a = 0; a < 4; ++a)
      for (int b = a + 1; b < 4; ++b) clash |= Overlap(ops[a], nb, ops[b], nb);
    if (clash) break;
    for (int w : {0, 2, 3}) writes.push_back({ops[w], nb});
    reads.push_back({ops[1], nb});
    tab.t[tab.count++] = {R.f(x.in[0]), R.f(x.in[1]), R.f(x.in[2]), R.f(x.in[3]), x.out[0]};
  }
  if (tab.count < 2) return -1;
  float hy[3];
  StepHyper(P, hy);
  SEEAI_TRY(c,
            LaunchAdamWMulti(tab, hy[0], P.beta1, P.beta2, P.eps, P.weight_decay, hy[1], hy[2],
                             c->flag(), c->stream, c->capturing ? c->hyper() : nullptr),
            "adamw");
  for (int i = 1; i < tab.count; ++i) c->done[i - 1] = at + 64 * i;
  c->ndone = tab.count - 1;
  c->fused += tab.count - 1;
  return SEEAI_OK;
}

int TryFuseElementwise(seeai_ctx* c, const Instruction& ins, const uint8_t* at) {
  if (!c->allow_fusion || !c->prog || at < c->prog || at >= c->prog + c->prog_count * 64 ||
      (at - c->prog) % 64 != 0)
    return -1;
  const uint64_t idx = static_cast<uint64_t>(at - c->prog) / 64;
  const auto next = [&](uint64_t k, Instruction* out) {
    if (idx + k >= c->range_end) return false;
    std::memcpy(out, c->prog + (idx + k) * 64, sizeof *out);
    return true;
  };
  const Ptrs R{c};
  const uint64_t n = ins.out[0];
  const uint64_t nb = n * 4;
  // Outputs must miss every other operand (inputs may repeat).
  const auto clear = [&](std::initializer_list<const float*> outs,
                         std::initializer_list<const float*> ins_) {
    for (const float* o : outs) {
      const auto* op = reinterpret_cast<const uint8_t*>(o);
      for (const float* q : outs)
        if (q != o && Overlap(op, nb, reinterpret_cast<const uint8_t*>(q), nb)) return false;
      for (const float* q : ins_)
        if (Overlap(op, nb, reinterpret_cast<const uint8_t*>(q), nb)) return false;
    }
    return true;
  };
  Instruction n1, n2;
  if (ins.opcode == 24 && next(1, &n1) && n1.opcode == 21 && n1.out[0] == n &&
      (n1.in[0] == ins.in[1]) != (n1.in[1] == ins.in[1])) {  // SiluFwd, MulEW(y, u)
    const float *x = R.f(ins.in[0]), *u = R.f(n1.in[0] == ins.in[1] ? n1.in[1] : n1.in[0]);
    float *y = R.f(ins.in[1]), *h = R.f(n1.in[2]);
    if (!clear({y, h}, {x, u})) return -1;
    Bf16Sink sink;
    GemmArgs ga{};
    const bool fits = SwigluFits(n, {x, u, y, h});
    const bool sunk = fits && PlanSink(c, idx + 1, idx + 1, h, n, &sink, &ga);
    // y's store is dropped where nothing reads it before it is written again
    // -- the backward pass that forms y from x does not read it.
    float* y_store =
        fits && DeadStore(c, idx, idx + 2, Extent{reinterpret_cast<const uint8_t*>(y), nb}) ? nullptr
                                                                                           : y;
    SEEAI_TRY(c, LaunchSiluMul(x, u, y_store, h, n, c->stream, sink), "silu_mul");
    if (sunk) SinkDone(c, idx + 1, ga);
    c->done[0] = at + 64;
    c->ndone = 1;
    ++c->fused;
    return SEEAI_OK;
  }
  if (ins.opcode == 21 && next(1, &n1) && n1.opcode == 21 && next(2, &n2) && n2.opcode == 25 &&
      n1.out[0] == n && n2.out[0] == n) {  // MulEW, MulEW, SiluBwd(one product, x)
    const bool first = n2.in[0] == ins.in[2];
    if (!first && n2.in[0] != n1.in[2]) return -1;
    const Instruction& m1 = first ? ins : n1;  // the product SiluBwd reads
    const Instruction& m2 = first ? n1 : ins;
    const float *a1 = R.f(m1.in[0]), *b1 = R.f(m1.in[1]), *a2 = R.f(m2.in[0]),
                *b2 = R.f(m2.in[1]), *x = R.f(n2.in[1]);
    float *o1 = R.f(m1.in[2]), *o2 = R.f(m2.in[2]), *dx = R.f(n2.in[2]);
    if (!clear({o1, o2, dx}, {a1, b1, a2, b2, x})) return -1;
    // The second product's y = SiLU(x) formed from x where the range shows
    // it is (x is read anyway; y then is not).
    const int silu = SiluOperand(c, idx, a2, b2, x, n);
    if (silu == 1) std::swap(a2, b2);  // IEEE multiplication commutes: b2 is y
    // The product SiluBwd reads is stored only where the range reads it again.
    float* o1_store = o1;
    if (DeadStore(c, idx, idx + 3, Extent{reinterpret_cast<const uint8_t*>(o1), nb}))
      o1_store = nullptr;
    // dx feeds the product right after the pass; the other product (o2)
    // commonly feeds the one after that: each takes a sink of its own.
    Bf16Sink sink, sink2;
    GemmArgs ga{}, ga2{};
    const bool fits = SwigluFits(n, {a1, b1, o1, a2, b2, o2, x, dx});
    const bool sunk = fits && PlanSink(c, idx + 2, idx + 2, dx, n, &sink, &ga);
    const bool sunk2 = sunk && PlanSink(c, idx + 2, idx + (first ? 1 : 0), o2, n, &sink2, &ga2, 2, 1);
    SEEAI_TRY(c,
              LaunchSwigluBwd(a1, b1, o1_store, a2, b2, o2, x, dx, n, c->stream, sink,
                              sunk2 ? sink2 : Bf16Sink{}, silu != 0),
              "swiglu_bwd");
    if (sunk) SinkDone(c, idx + 2, ga);
    if (sunk2) SinkDone(c, idx + 2, ga2, 2);
    c->done[0] = at + 64;
    c->done[1] = at + 128;
    c->ndone = 2;
    ++c->fused;
    return SEEAI_OK;
  }
  return -1;
}

// The add behind a product: a GEMM with no addend, accumulate, bias or
// activation whose C the next instruction, kAddEW, adds to another operand
// X (either side; IEEE addition commutes) runs with X as its addend and the
// add's output as C -- the epilogue's X + dot is the add's X + C, the same
// rounding; and a GEMM with no bias, accumulate or activation (an addend
// allowed) whose C the next instruction, kAddBias, offsets by a bias row
// runs with that bias -- the epilogue adds it after the addend, as the
// instruction would.  Either when C is read by nothing after the add (the
// dead-store rule) and the add's output misses everything the product
// reads (it may be X, or C, itself).  One pass instead of two over M x N.
int TryFuseAddend(seeai_ctx* c, const Instruction& ins, const uint8_t* at) {
  if (!c->allow_fusion || !c->prog || at < c->prog || at >= c->prog + c->prog_count * 64 ||
      (at - c->prog) % 64 != 0)
    return -1;
  const uint64_t idx = static_cast<uint64_t>(at - c->prog) / 64;
  if (idx + 1 >= c->range_end) return -1;
  Instruction nx;
  std::memcpy(&nx, c->prog + (idx + 1) * 64, sizeof nx);
  if (nx.opcode != 5 && nx.opcode != 6) return -1;
  GemmArgs a{};
  const char* what = DecodeGemm(c, ins, &a);
  if (!what || a.accumulate || a.bias || a.act) return -1;
  const Ptrs R{c};
  if (nx.opcode == 6) {  // kAddBias [x, b, out], [rows, cols]
    float* out = R.f(nx.in[2]);
    const float* bias = R.f(nx.in[1]);
    if (R.f(nx.in[0]) != a.C || nx.out[0] != a.M || nx.out[1] != a.N) return -1;
    const Extent e_out{reinterpret_cast<const uint8_t*>(out), a.M * a.N * 4};
    const Extent e_b{reinterpret_cast<const uint8_t*>(bias), a.N * 4};
    const Extent e_c = GemmWrites(a);
    Extent reads[8];
    const int nr = GemmReads(a, reads);
    if (Hits(e_out, reads, nr) || Hits(e_out, &e_b, 1) || Hits(e_c, &e_b, 1) ||
        (out != a.C && Hits(e_out, &e_c, 1)))
      return -1;
    if (!DeadStore(c, idx, idx + 2, e_c, 2)) return -1;
    a.relaxed = Relaxed(c, ins);
    a.bias = bias;
    a.C = out;
    if (int rc = Gemm(c, a, what)) return rc;
    c->done[0] = at + 64;
    c->ndone = 1;
    ++c->fused;
    return SEEAI_OK;
  }
  if (a.addend || a.M * a.N != nx.out[0]) return -1;
  const float *x0 = R.f(nx.in[0]), *x1 = R.f(nx.in[1]);
  float* out = R.f(nx.in[2]);
  if ((x0 == a.C) == (x1 == a.C)) return -1;  // C on exactly one side
  const float* X = x0 == a.C ? x1 : x0;
  const uint64_t nb = a.M * a.N * 4;
  const Extent e_out{reinterpret_cast<const uint8_t*>(out), nb};
  const Extent e_x{reinterpret_cast<const uint8_t*>(X), nb};
  const Extent e_c = GemmWrites(a);
  Extent reads[8];
  const int nr = GemmReads(a, reads);
  if (Hits(e_out, reads, nr) || Hits(e_c, &e_x, 1) || (out != X && Hits(e_out, &e_x, 1)))
    return -1;
  if (!DeadStore(c, idx, idx + 2, e_c, 2)) return -1;
  a.relaxed = Relaxed(c, ins);
  a.addend = X;
  a.C = out;
  if (int rc = Gemm(c, a, what)) return rc;
  c->done[0] = at + 64;
  c->ndone = 1;
  ++c->fused;
  return SEEAI_OK;
}

// Two adjacent exact TN products that read nothing the first writes and
// write apart from each other and from what the first reads (a LoRA
// site's dB = t^T dC and dA = X^T dt) run as one launch where each alone
// would leave CUs idle (GemmExactPairFits): the same sums, bit for bit.
int TryFuseGemmPair(seeai_ctx* c, const Instruction& ins, const uint8_t* at) {
  if (!c->allow_fusion || !c->cur_at || !c->prog || at != c->cur_at || ins.opcode != 3) return -1;
  const uint64_t idx = CurIndex(c);
  if (idx + 1 >= c->range_end) return -1;
  Instruction nx;
  std::memcpy(&nx, c->prog + (idx + 1) * 64, sizeof nx);
  if (nx.opcode != 3) return -1;
  const auto relaxed = [&](const Instruction& i) {
    return (i.flags & kFlagRelaxed) && c->allow_relaxed;
  };
  if (relaxed(ins) || relaxed(nx)) return -1;
  GemmArgs a{}, b{};
  const char* what = DecodeGemm(c, ins, &a);
  if (!what || !DecodeGemm(c, nx, &b)) return -1;
  a.policy = b.policy = &c->policy;
  if (!GemmExactPairFits(a, b)) return -1;
  Extent ra[8], rb[8];
  const int nra = GemmReads(a, ra), nrb = GemmReads(b, rb);
  const Extent wa = GemmWrites(a), wb = GemmWrites(b);
  if (Hits(wa, rb, nrb) || Hits(wb, ra, nra) || Hits(wb, &wa, 1)) return -1;
  SEEAI_TRY(c, LaunchGemmExactPair(a, b, c->stream), what);
  c->done[0] = at + 64;
  c->ndone = 1;
  ++c->fused;
  return SEEAI_OK;
}

// The residual add behind a normalisation's gradient: LayerNorm / RMSNorm
// backward writing dx, then kAddEW of dx and a residual gradient R, runs as
// one pass writing R + dx into the add's output (with the add's conversion
// sink when a relaxed product follows), when dx is read by nothing after
// the add and the add's output misses the normalisation's inputs (it may
// be R itself).
int TryFuseNormAdd(seeai_ctx* c, const Instruction& ins, const uint8_t* at) {
  if (!c->allow_fusion || !c->prog || (ins.opcode != 27 && ins.opcode != 32) || at < c->prog ||
      at >= c->prog + c->prog_count * 64 || (at - c->prog) % 64 != 0)
    return -1;
  const uint64_t idx = static_cast<uint64_t>(at - c->prog) / 64;
  if (idx + 1 >= c->range_end) return -1;
  Instruction nx;
  std::memcpy(&nx, c->prog + (idx + 1) * 64, sizeof nx);
  if (nx.opcode != 5) return -1;
  const Ptrs R{c};
  const bool ln = ins.opcode == 27;
  const uint64_t shape = ln ? ins.out[2] : ins.out[1];
  const uint64_t rows = shape >> 32, cols = shape & 0xFFFFFFFFu, n = rows * cols;
  const float *dy = R.f(ins.in[0]), *x = R.f(ins.in[1]), *g = R.f(ins.in[2]);
  const float* mean = ln ? R.f(ins.out[0]) : nullptr;
  const float* rstd = R.f(ln ? ins.out[1] : ins.out[0]);
  const float* dx = R.f(ins.in[3]);
  const float *x0 = R.f(nx.in[0]), *x1 = R.f(nx.in[1]);
  float* out = R.f(nx.in[2]);
  if (n == 0 || nx.out[0] != n || (x0 == dx) == (x1 == dx)) return -1;
  const float* res = x0 == dx ? x1 : x0;
  const uint64_t nb = n * 4;
  const auto ext = [](const void* p, uint64_t bytes) {
    return Extent{static_cast<const uint8_t*>(p), bytes};
  };
  const Extent reads[] = {ext(dy, nb), ext(x, nb), ext(g, cols * 4), ext(rstd, rows * 4),
                          ext(mean ? mean : rstd, rows * 4)};
  const Extent e_out = ext(out, nb), e_dx = ext(dx, nb), e_res = ext(res, nb);
  if (Hits(e_out, reads, 5) || Hits(e_dx, &e_res, 1) || (out != res && Hits(e_out, &e_res, 1)) ||
      Hits(e_res, reads, 2))
    return -1;
  if (!NormSinkFits(cols, {dy, x, g, out, res})) return -1;
  if (!DeadStore(c, idx, idx + 2, e_dx, 3)) return -1;
  Bf16Sink sink;
  GemmArgs ga{};
  const bool sunk = PlanSink(c, idx + 1, idx + 1, out, n, &sink, &ga);
  if (ln)
    SEEAI_TRY(c, LaunchLayerNormBwd(dy, x, g, mean, rstd, out, rows, cols, c->stream, sink, res),
              "layernorm.bwd+add");
  else
    SEEAI_TRY(c, LaunchRmsNormBwd(dy, x, g, rstd, out, rows, cols, c->stream, sink, res),
              "rmsnorm.bwd+add");
  if (sunk) SinkDone(c, idx + 1, ga);
  c->done[0] = at + 64;
  c->ndone = 1;
  ++c->fused;
  return SEEAI_OK;
}

// The loss at the turn of a train program: softmax-xent forward, the fill of
// its seed, softmax-xent backward over the same probabilities and labels
// (plain or masked).  The fill runs first (it touches nothing the forward
// reads or writes; a few rows run the whole turn in one workgroup), then
// one pass forms the probabilities and, from them,
// the gradient -- the backward's expression on the same f32 values, with
// its conversion sink -- storing the probabilities only where something
// after the backward reads them.  One read of the logits and no read of
// the probabilities instead of a write and a read.
int TryFuseXEnt(seeai_ctx* c, const Instruction& ins, const uint8_t* at,
                const seeai_step_params& P) {
  if (!c->allow_fusion || !c->prog || (ins.opcode != 11 && ins.opcode != 51) || at < c->prog ||
      at >= c->prog + c->prog_count * 64 || (at - c->prog) % 64 != 0)
    return -1;
  const uint64_t idx = static_cast<uint64_t>(at - c->prog) / 64;
  if (idx + 2 >= c->range_end) return -1;
  Instruction f, b;
  std::memcpy(&f, c->prog + (idx + 1) * 64, sizeof f);
  std::memcpy(&b, c->prog + (idx + 2) * 64, sizeof b);
  if (f.opcode != 19 || b.opcode != ins.opcode + 1 || b.in[0] != ins.in[3] ||
      b.in[1] != ins.in[1] || b.out[0] != ins.out[0] || b.out[1] != ins.out[1])
    return -1;
  const Ptrs R{c};
  const uint64_t N = ins.out[0], C = ins.out[1];
  const float* logits = R.f(ins.in[0]);
  const int32_t* labels = R.i32(ins.in[1]);
  float *loss = R.f(ins.in[2]), *probs = R.f(ins.in[3]);
  const float* seed = R.f(b.in[2]);
  float* dl = R.f(b.in[3]);
  const auto ext = [](const void* p, uint64_t bytes) {
    return Extent{static_cast<const uint8_t*>(p), bytes};
  };
  const Extent fwd[] = {ext(logits, N * C * 4), ext(labels, N * 4), ext(loss, 4),
                        ext(probs, N * C * 4)};
  const Extent e_fill = ext(R.f(f.in[0]), f.out[0] * 4), e_dl = ext(dl, N * C * 4),
               e_seed = ext(seed, 4);
  if (Hits(e_fill, fwd, 4) || Hits(e_dl, fwd, 4) || Hits(e_dl, &e_seed, 1) ||
      Hits(e_seed, fwd + 2, 2))
    return -1;
  float* keep = DeadStore(c, idx, idx + 3, fwd[3]) ? nullptr : probs;
  if (!XEntFusedFits(logits, keep, dl, C)) return -1;
  void* ws;
  if (int rc = Scratch(c, XEntFwdScratchBytes(N), &ws)) return rc;
  Bf16Sink sink;
  GemmArgs ga{};
  const bool sunk = PlanSink(c, idx + 2, idx + 2, dl, N * C, &sink, &ga);
  // The product just before left the logits' partial row maxima.
  const auto& pk = c->pmax_key;
  const float* parts = pk.C == logits && pk.M == N && pk.N == C && pk.at == idx &&
                               pk.epoch == c->a16_epoch
                           ? c->pmax
                           : nullptr;
  c->pmax_key.C = nullptr;
  SEEAI_TRY(c,
            LaunchXEntFwdBwd(logits, labels, loss, keep, R.f(f.in[0]), f.out[0],
                             BitsToF32(f.in[1]), seed, dl, N, C, ins.opcode == 51, ws, c->stream,
                             sink, parts),
            "softmax_xent.fwd+bwd");
  if (sunk) SinkDone(c, idx + 2, ga);
  c->done[0] = at + 64;
  c->done[1] = at + 128;
  c->ndone = 2;
  ++c->fused;
  return SEEAI_OK;
}

// A 64-bit hash of a program's words (FNV-1a over 8-byte words, then a
// final avalanche): what the per-program dead-store decisions are keyed on
// besides the program's address and length.
uint64_t ProgramHash(const uint8_t* prog, uint64_t count) {
  uint64_t h = 0xcbf29ce484222325ULL;
  for (uint64_t i = 0; i < count * 8; ++i) {
    uint64_t w;
    std::memcpy(&w, prog + i * 8, 8);
    h = (h ^ w) * 0x100000001b3ULL;
  }
  h ^= h >> 33;
  h *= 0xff51afd7ed558ccdULL;
  h ^= h >> 33;
  return h;
}

}  // namespace

int seeai_execute(seeai_ctx* c, const void* instruction, const seeai_step_params* params) {
  if (!c || !instruction) return SEEAI_INVALID;
  const auto* at = static_cast<const uint8_t*>(instruction);
  if (c->ndone > 0 && at == c->done[0]) {  // ran with an earlier instruction
    for (int i = 1; i < c->ndone; ++i) c->done[i - 1] = c->done[i];
    --c->ndone;
    return SEEAI_OK;
  }
  c->ndone = 0;  // any other order runs every instruction as given
  Instruction ins;
  std::memcpy(&ins, instruction, sizeof ins);
  if (!c->arena) return Fail(c, SEEAI_INVALID, "execute: no arena is bound");
  seeai_step_params P{};
  if (params) P = *params;
  const bool in_range = c->prog && at >= c->prog && at < c->prog + c->prog_count * 64 &&
                        (at - c->prog) % 64 == 0;
  c->cur_at = in_range ? at : nullptr;
  int rc = TryFuseLowRank(c, ins, at, P);
  if (rc < 0) rc = TryFuseAdamW(c, ins, at, P);
  if (rc < 0) rc = TryFuseAttnBwd(c, ins, at);
  if (rc < 0) rc = TryFuseElementwise(c, ins, at);
  if (rc < 0) rc = TryFuseNormAdd(c, ins, at);
  if (rc < 0) rc = TryFuseXEnt(c, ins, at, P);
  if (rc < 0) rc = TryFuseGemmPair(c, ins, at);
  if (rc < 0) rc = TryFuseAddend(c, ins, at);
  if (rc < 0) rc = ExecuteOne(c, ins, P);
  c->cur_at = nullptr;
  return rc;
}

namespace {
// A range's workspaces at their largest before its first instruction runs:
// the exact family's reduction scratch, the relaxed products' conversion
// buffer and their weights' bf16 shadows are sized (and the shadows made)
// here, so no instruction of the range drains the stream to allocate.
int PresizeWorkspaces(seeai_ctx* c, const uint8_t* prog, uint64_t begin, uint64_t end) {
  size_t scratch = 0, cvt = 0;
  for (uint64_t i = begin; i < end; ++i) {
    Instruction ins;
    std::memcpy(&ins, prog + i * sizeof(Instruction), sizeof ins);
    if (ins.opcode == 11 || ins.opcode == 51)  // softmax-xent forward (+masked): row partials
      scratch = std::max(scratch, XEntFwdScratchBytes(ins.out[0]));
    if ((ins.opcode == 47 || ins.opcode == 57) && (ins.flags & kFlagRelaxed)) {
      uint64_t B, S, H, d;
      if (ins.opcode == 47) {
        B = ins.out[1] >> 32, S = ins.out[1] & 0xFFFFFFFFu, H = ins.out[2] >> 32,
        d = ins.out[2] & 0xFFFFFFFFu;
      } else {
        const uint64_t g = ins.out[1];
        B = g >> 48, S = (g >> 32) & 0xFFFF, H = (g >> 16) & 0xFFFF, d = g & 0xFFFF;
      }
      if (Attn16Plan(c, B, S, H, d)) {
        const Ptrs R{c};
        if (int rc = MakeSavedCopies(c, R.f(ins.in[0]), R.f(ins.in[1]), R.f(ins.in[2]),
                                     B * S * H * d))
          return rc;
      }
    }
    GemmArgs a{};
    if (!DecodeGemm(c, ins, &a)) continue;
    a.relaxed = (ins.flags & kFlagRelaxed) && c->allow_relaxed ? 1 : 0;
    a.policy = &c->policy;
    if (a.relaxed && c->allow_dma && Bf16DmaFits(a) && Immutable(c, a.B)) {
      cvt = std::max(cvt, static_cast<size_t>(a.M * Bf16DmaKp(a.K) * 2));
      const auto key = std::make_tuple(a.B, a.layout, a.b_kind, static_cast<uint64_t>(a.N),
                                       static_cast<uint64_t>(a.K));
      if (c->shadows.find(key) == c->shadows.end()) {
        void* shadow = nullptr;
        SEEAI_TRY(c, hipMalloc(&shadow, a.N * Bf16DmaKp(a.K) * 2), "weight shadow alloc");
        c->shadows[key] = shadow;
        SEEAI_TRY(c, LaunchWeightShadow(a, shadow, c->stream), "weight shadow");
      }
    } else if (!a.relaxed) {
      scratch = std::max(scratch, GemmExactScratchBytes(a));
    }
  }
  {  // at least the initial size: the norm and clip partials take 8 KiB
    void* ws;
    if (int rc = Scratch(c, std::max(scratch, kInitialScratch), &ws)) return rc;
  }
  if (cvt > c->cvt_bytes) {
    DropGraphs(c);
    SEEAI_TRY(c, hipStreamSynchronize(c->stream), "conversion buffer drain");
    if (c->cvt) SEEAI_TRY(c, hipFree(c->cvt), "conversion buffer free");
    c->cvt = nullptr;
    c->cvt_bytes = 0;
    SEEAI_TRY(c, hipMalloc(&c->cvt, cvt), "conversion buffer alloc");
    c->cvt_bytes = cvt;
  }
  if (cvt > c->xcvt_bytes) {
    DropGraphs(c);
    SEEAI_TRY(c, hipStreamSynchronize(c->stream), "conversion buffer drain");
    c->xcvt_bytes = 0;
    for (int s = 0; s < seeai_ctx::kXSlots; ++s) {
      c->xcvt_key[s].at = nullptr;
      if (c->xcvt[s]) SEEAI_TRY(c, hipFree(c->xcvt[s]), "conversion buffer free");
      c->xcvt[s] = nullptr;
    }
    for (int s = 0; s < seeai_ctx::kXSlots; ++s)
      SEEAI_TRY(c, hipMalloc(&c->xcvt[s], cvt), "conversion buffer alloc");
    c->xcvt_bytes = cvt;
  }
  return SEEAI_OK;
}
}  // namespace

int seeai_begin_range(seeai_ctx* c, const void* program, uint64_t count, uint64_t begin,
                      uint64_t end) {
  if (!c || (!program && count) || begin > end || end > count) return SEEAI_INVALID;
  if (c->arena)
    if (int rc = PresizeWorkspaces(c, static_cast<const uint8_t*>(program), begin, end)) return rc;
  c->prog_hash = ProgramHash(static_cast<const uint8_t*>(program), count);
  c->prog = static_cast<const uint8_t*>(program);
  c->prog_count = count;
  c->range_end = end;
  c->ndone = 0;
  ForgetCopies(c);
  return SEEAI_OK;
}

int seeai_end_range(seeai_ctx* c) {
  if (!c) return SEEAI_INVALID;
  c->prog = nullptr;
  c->prog_count = c->range_end = 0;
  c->ndone = 0;
  ForgetCopies(c);
  return SEEAI_OK;
}

int seeai_set_fusion(seeai_ctx* c, int allow) {
  if (!c) return SEEAI_INVALID;
  DropGraphs(c);
  c->allow_fusion = allow ? 1 : 0;
  return SEEAI_OK;
}

uint64_t seeai_fused_dispatches(const seeai_ctx* c) { return c ? c->fused : 0; }
uint64_t seeai_dropped_stores(const seeai_ctx* c) { return c ? c->dropped_stores : 0; }
uint64_t seeai_fused_conversions(const seeai_ctx* c) { return c ? c->sinks : 0; }

int seeai_configure(seeai_ctx* c, const seeai_tile_policy* p) {
  if (!c) return SEEAI_INVALID;
  TilePolicy t;  // defaults
  if (p) {
    // CheckEntry's role (kernel_policy_table.cc:280-289): refuse what no
    // kernel implements, leave the previous policy in force.
    if (p->w8a8_large_kernel > 3)
      return Fail(c, SEEAI_INVALID, "tile policy: w8a8_large_kernel %u is not 1, 2 or 3",
                  p->w8a8_large_kernel);
    if (p->exact_longk_first > 2)
      return Fail(c, SEEAI_INVALID, "tile policy: exact_longk_first %u is not 1 or 2",
                  p->exact_longk_first);
    if (p->relaxed_tile_192 > 3)
      return Fail(c, SEEAI_INVALID, "tile policy: relaxed_tile_192 %u is not 1, 2 or 3",
                  p->relaxed_tile_192);
    if (p->relaxed_min_fill_256 > 100)
      return Fail(c, SEEAI_INVALID, "tile policy: relaxed_min_fill_256 %u exceeds 100 percent",
                  p->relaxed_min_fill_256);
    if (p->convert_wgs_per_cu > 64)
      return Fail(c, SEEAI_INVALID, "tile policy: convert_wgs_per_cu %u exceeds 64",
                  p->convert_wgs_per_cu);
    if (p->quantize_waves_per_cu > 32)
      return Fail(c, SEEAI_INVALID, "tile policy: quantize_waves_per_cu %u exceeds 32 waves per CU",
                  p->quantize_waves_per_cu);
    if (p->w8a8_large_kernel) t.w8a8_large_kernel = static_cast<int>(p->w8a8_large_kernel);
    if (p->w8a8_large_min) t.w8a8_large_min = p->w8a8_large_min;
    if (p->quantize_waves_per_cu) t.quantize_waves_per_cu = static_cast<int>(p->quantize_waves_per_cu);
    if (p->relaxed_min_tiles_256) t.relaxed_min_tiles_256 = p->relaxed_min_tiles_256;
    if (p->relaxed_min_fill_256) t.relaxed_min_fill_256 = static_cast<int>(p->relaxed_min_fill_256);
    if (p->relaxed_nt_dma_min_k) t.relaxed_nt_dma_min_k = p->relaxed_nt_dma_min_k;
    if (p->convert_wgs_per_cu) t.convert_wgs_per_cu = static_cast<int>(p->convert_wgs_per_cu);
    if (p->exact_longk_first) t.exact_longk_first = static_cast<int>(p->exact_longk_first);
    if (p->relaxed_tile_192) t.relaxed_tile_192 = static_cast<int>(p->relaxed_tile_192);
  }
  DropGraphs(c);
  c->policy = t;
  return SEEAI_OK;
}

int seeai_policy(const seeai_ctx* c, seeai_tile_policy* out) {
  if (!c || !out) return SEEAI_INVALID;
  out->w8a8_large_kernel = static_cast<uint32_t>(c->policy.w8a8_large_kernel);
  out->w8a8_large_min = static_cast<uint32_t>(c->policy.w8a8_large_min);
  out->quantize_waves_per_cu = static_cast<uint32_t>(c->policy.quantize_waves_per_cu);
  out->relaxed_min_tiles_256 = static_cast<uint32_t>(c->policy.relaxed_min_tiles_256);
  out->relaxed_min_fill_256 = static_cast<uint32_t>(c->policy.relaxed_min_fill_256);
  out->relaxed_nt_dma_min_k = static_cast<uint32_t>(c->policy.relaxed_nt_dma_min_k);
  out->convert_wgs_per_cu = static_cast<uint32_t>(c->policy.convert_wgs_per_cu);
  out->exact_longk_first = static_cast<uint32_t>(c->policy.exact_longk_first);
  out->relaxed_tile_192 = static_cast<uint32_t>(c->policy.relaxed_tile_192);
  return SEEAI_OK;
}

int seeai_device_key(int device, char* buf, uint64_t bytes) {
  if (!buf || bytes == 0) return SEEAI_INVALID;
  hipDeviceProp_t p{};
  if (hipGetDeviceProperties(&p, device) != hipSuccess) return SEEAI_HIP_ERROR;
  std::string arch(p.gcnArchName);
  if (const size_t colon = arch.find(':'); colon != std::string::npos) arch.resize(colon);
  char key[512];
  std::snprintf(key, sizeof key, "%s;%s;cus=%d;lds=%zu;l2=%d;wave=%d", arch.c_str(), p.name,
                p.multiProcessorCount, static_cast<size_t>(p.maxSharedMemoryPerMultiProcessor),
                p.l2CacheSize, p.warpSize);
  const size_t n = std::strlen(key);
  if (n + 1 > bytes) return SEEAI_INVALID;
  std::memcpy(buf, key, n + 1);
  return SEEAI_OK;
}

int seeai_execute_range(seeai_ctx* c, const void* instructions, uint64_t count,
                        const seeai_step_params* params, uint64_t* failed_at) {
  if (!c || (!instructions && count)) return SEEAI_INVALID;
  const auto* base = static_cast<const uint8_t*>(instructions);
  if (int rc = seeai_begin_range(c, instructions, count, 0, count)) return rc;
  for (uint64_t i = 0; i < count; ++i) {
    if (int rc = seeai_execute(c, base + i * 64, params)) {
      if (failed_at) *failed_at = i;
      seeai_end_range(c);
      return rc;
    }
  }
  seeai_end_range(c);
  return SEEAI_OK;
}

int seeai_set_graph_replay(seeai_ctx* c, int on) {
  if (!c) return SEEAI_INVALID;
  DropGraphs(c);
  c->graph_replay = on ? 1 : 0;
  return SEEAI_OK;
}

int seeai_run_range(seeai_ctx* c, const void* program, uint64_t count, uint64_t begin,
                    uint64_t end, const seeai_step_params* params, uint64_t* failed_at) {
  if (!c || (!program && count) || begin > end || end > count) return SEEAI_INVALID;
  const auto* base = static_cast<const uint8_t*>(program);
  auto eager = [&]() -> int {
    if (int rc = seeai_begin_range(c, program, count, begin, end)) return rc;
    for (uint64_t i = begin; i < end; ++i) {
      if (int rc = seeai_execute(c, base + i * 64, params)) {
        if (failed_at) *failed_at = i;
        seeai_end_range(c);
        return rc;
      }
    }
    seeai_end_range(c);
    return SEEAI_OK;
  };
  if (!c->graph_replay || begin == end || !c->arena) return eager();
  const uint64_t hash = ProgramHash(base, count);
  // The entry of this range (found again after anything that may have
  // dropped the list: a workspace growth clears it).
  auto find = [&]() -> seeai_ctx::RangeGraph* {
    for (auto& g : c->graphs)
      if (g.prog == base && g.count == count && g.begin == begin && g.end == end && g.hash == hash)
        return &g;
    return nullptr;
  };
  seeai_ctx::RangeGraph* e = find();
  if (!e) {
    if (c->graphs.size() >= 8) {  // a few ranges per plan: keep the newest
      if (c->graphs.front().exec) {
        SEEAI_TRY(c, hipStreamSynchronize(c->stream), "graph retire");
        (void)hipGraphExecDestroy(c->graphs.front().exec);
      }
      c->graphs.erase(c->graphs.begin());
    }
    c->graphs.push_back({});
    e = &c->graphs.back();
    e->prog = base, e->count = count, e->begin = begin, e->end = end, e->hash = hash;
    e->gen = c->graph_gen;
  }
  if (e->ungraphable) return eager();
  if (!e->exec) {
    if (e->runs == 0) {  // eager first: makes the shadows, sizes the workspaces
      const uint64_t gen = c->graph_gen;
      const int rc = eager();
      if (auto* g = find(); g && rc == SEEAI_OK && c->graph_gen == gen) g->runs = 1;
      return rc;
    }
    // Capture: the range's launches recorded, not run (nothing in it waits
    // on the host or allocates once its first run has sized everything).
    const uint64_t gen = c->graph_gen;
    if (int rc = seeai_begin_range(c, program, count, begin, end)) return rc;
    if (c->graph_gen != gen) {  // the range start grew a workspace: run it as it is
      seeai_end_range(c);
      return eager();
    }
    const uint64_t relaxed0 = c->relaxed, fused0 = c->fused, dropped0 = c->dropped_stores,
                   sinks0 = c->sinks;
    int rc = SEEAI_OK;
    if (!c->capture_stream)
      rc = Hip(c, hipStreamCreateWithFlags(&c->capture_stream, hipStreamNonBlocking), "capture stream");
    const hipStream_t stream = c->stream;
    if (rc == SEEAI_OK)
      rc = Hip(c, hipStreamBeginCapture(c->capture_stream, hipStreamCaptureModeThreadLocal), "capture");
    const bool began = rc == SEEAI_OK;
    c->stream = c->capture_stream;  // every launch of the range records into the capture
    c->capturing = true;
    for (uint64_t i = begin; rc == SEEAI_OK && i < end; ++i) rc = seeai_execute(c, base + i * 64, params);
    c->capturing = false;
    hipGraph_t graph = nullptr;
    hipError_t ec = began ? hipStreamEndCapture(c->capture_stream, &graph) : hipErrorUnknown;
    c->stream = stream;
    seeai_end_range(c);
    const uint64_t d_relaxed = c->relaxed - relaxed0, d_fused = c->fused - fused0,
                   d_dropped = c->dropped_stores - dropped0, d_sinks = c->sinks - sinks0;
    c->relaxed = relaxed0, c->fused = fused0, c->dropped_stores = dropped0;  // nothing ran yet
    c->sinks = sinks0;
    hipGraphExec_t exec = nullptr;
    if (rc == SEEAI_OK && ec == hipSuccess && graph && c->graph_gen == gen)
      ec = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    else
      ec = hipErrorUnknown;
    if (graph) (void)hipGraphDestroy(graph);
    (void)hipGetLastError();  // a refused capture leaves nothing to report
    e = find();
    if (ec != hipSuccess || !exec || !e) {
      if (exec) (void)hipGraphExecDestroy(exec);
      if (e) e->ungraphable = true;  // instruction by instruction, now and from here on
      return eager();
    }
    e->exec = exec;
    e->relaxed = d_relaxed, e->fused = d_fused, e->dropped = d_dropped, e->sinks = d_sinks;
  }
  // Replay: the step's optimizer values land in hyper() first.
  float hy[3] = {0.0f, 0.0f, 0.0f};
  if (params) StepHyper(*params, hy);
  SEEAI_TRY(c, hipEventSynchronize(c->hyper_copied), "step values");  // the last copy has read them
  std::memcpy(c->host_hyper, hy, sizeof hy);
  SEEAI_TRY(c, hipMemcpyAsync(c->hyper(), c->host_hyper, sizeof hy, hipMemcpyHostToDevice, c->stream),
            "step values");
  SEEAI_TRY(c, hipEventRecord(c->hyper_copied, c->stream), "step values");
  SEEAI_TRY(c, hipGraphLaunch(e->exec, c->stream), "graph launch");
  c->relaxed += e->relaxed, c->fused += e->fused, c->dropped_stores += e->dropped;
  c->sinks += e->sinks;
  ++c->graph_launches;
  return SEEAI_OK;
}

uint64_t seeai_graph_launches(const seeai_ctx* c) { return c ? c->graph_launches : 0; }

int seeai_attn_dkdv(seeai_ctx* c, const float* q, const float* k, const float* v,
                    const float* dout, const float* stats, float* dk, float* dv, uint64_t B,
                    uint64_t S, uint64_t H, uint64_t d) {
  if (!c) return SEEAI_INVALID;
  if (!AttnDKDVFusable(q, k, v, dout, dk, dv, B, S, H, d))
    return Fail(c, SEEAI_INVALID, "attn_dkdv: the fused pass takes d = 64 with 16-byte aligned "
                                  "operands and slices under 2 GiB");
  SEEAI_TRY(c, LaunchAttnDKDVFused(q, k, v, dout, stats, dk, dv, B, S, H, d, c->stream),
            "attn_dkdv");
  return SEEAI_OK;
}

int seeai_flush_download(seeai_ctx* c, uint64_t off, void* dst, uint64_t bytes) {
  if (!c || !c->arena || off + bytes > c->arena_bytes || (bytes && !dst))
    return Fail(c, SEEAI_INVALID, "flush_download: extent outside the arena");
  SEEAI_TRY(c, hipMemcpyAsync(c->host_flag, c->flag(), sizeof(int), hipMemcpyDeviceToHost, c->stream),
            "flush flag");
  if (bytes)
    SEEAI_TRY(c, hipMemcpyAsync(dst, c->arena + off, bytes, hipMemcpyDeviceToHost, c->stream),
              "flush download");
  SEEAI_TRY(c, hipStreamSynchronize(c->stream), "flush");
  if (*c->host_flag) {
    SEEAI_TRY(c, hipMemsetAsync(c->flag(), 0, sizeof(int), c->stream), "flush reset");
    SEEAI_TRY(c, hipStreamSynchronize(c->stream), "flush reset sync");
    return Fail(c, SEEAI_REFUSED, "%s", kNonFiniteNormRefusal);
  }
  return SEEAI_OK;
}

int seeai_flush(seeai_ctx* c) {
  if (!c) return SEEAI_INVALID;
  SEEAI_TRY(c, hipMemcpyAsync(c->host_flag, c->flag(), sizeof(int), hipMemcpyDeviceToHost, c->stream),
            "flush flag");
  SEEAI_TRY(c, hipStreamSynchronize(c->stream), "flush");
  if (*c->host_flag) {
    SEEAI_TRY(c, hipMemsetAsync(c->flag(), 0, sizeof(int), c->stream), "flush reset");
    SEEAI_TRY(c, hipStreamSynchronize(c->stream), "flush reset sync");
    return Fail(c, SEEAI_REFUSED, "%s", kNonFiniteNormRefusal);
  }
  return SEEAI_OK;
}

int seeai_gemm_f32(seeai_ctx* c, int layout, const float* A, const float* B, float* C, uint64_t M,
                   uint64_t N, uint64_t K, const float* bias, int act, const float* addend,
                   float alpha, int accumulate) {
  if (!c || layout < 0 || layout > 2 || act < 0 || act > 3) return Fail(c, SEEAI_INVALID, "gemm_f32: bad layout/act");
  GemmArgs a{};
  a.layout = layout;
  a.A = A;
  a.B = B;
  a.C = C;
  a.M = M;
  a.N = N;
  a.K = K;
  a.alpha_a = layout == 1 ? 1.0f : alpha;
  a.alpha_dot = layout == 1 ? alpha : 1.0f;
  a.addend = addend;
  a.bias = bias;
  a.act = act;
  a.accumulate = accumulate;
  return Gemm(c, a, "gemm_f32");
}

int seeai_gemm_q8(seeai_ctx* c, int nt, const float* A, const int8_t* B, float* C, uint64_t M,
                  uint64_t N, uint64_t K, float scale, const float* col_scale, int act) {
  if (!c || act < 0 || act > 3 || (nt && act)) return Fail(c, SEEAI_INVALID, "gemm_q8: bad act");
  GemmArgs a{};
  a.layout = nt ? 1 : 0;
  a.b_kind = 1;
  a.A = A;
  a.B = B;
  a.C = C;
  a.M = M;
  a.N = N;
  a.K = K;
  const float sc = col_scale ? 1.0f : scale;
  a.alpha_a = nt ? 1.0f : sc;
  a.alpha_dot = nt ? sc : 1.0f;
  if (col_scale) {
    if (nt)
      a.a_k_scale = col_scale;
    else
      a.b_col_scale = col_scale;
  }
  a.act = act;
  return Gemm(c, a, "gemm_q8");
}

int seeai_gemm_bf16w(seeai_ctx* c, int nt, const float* A, const uint16_t* B, float* C, uint64_t M,
                     uint64_t N, uint64_t K, const float* bias, int act) {
  if (!c || act < 0 || act > 3 || (nt && (act || bias))) return Fail(c, SEEAI_INVALID, "gemm_bf16w: NT takes no epilogue");
  GemmArgs a{};
  a.layout = nt ? 1 : 0;
  a.b_kind = 2;
  a.A = A;
  a.B = B;
  a.C = C;
  a.M = M;
  a.N = N;
  a.K = K;
  a.alpha_a = 1.0f;
  a.alpha_dot = 1.0f;
  a.bias = bias;
  a.act = act;
  return Gemm(c, a, "gemm_bf16w");
}

int seeai_w8a8_quantize_rows(seeai_ctx* c, const float* X, int8_t* Q, float* scale, uint64_t rows,
                             uint64_t cols) {
  if (!c) return SEEAI_INVALID;
  SEEAI_TRY(c, LaunchQuantizeRows(X, Q, scale, rows, cols, c->policy.quantize_waves_per_cu, c->stream), "quantize_rows");
  return SEEAI_OK;
}

int seeai_w8a8_pack_weights(seeai_ctx* c, const float* W, int8_t* Qt, float* scale, uint64_t K,
                            uint64_t N) {
  if (!c) return SEEAI_INVALID;
  SEEAI_TRY(c, LaunchPackWeightsI8(W, Qt, scale, K, N, c->stream), "pack_weights");
  return SEEAI_OK;
}

int seeai_w8a8_gemm(seeai_ctx* c, const int8_t* QA, const float* sa, const int8_t* QWt,
                    const float* sw, float* C, int32_t* acc, uint64_t M, uint64_t N, uint64_t K) {
  if (!c) return SEEAI_INVALID;
  if (K > 133144) return Fail(c, SEEAI_INVALID, "w8a8_gemm: K = %llu could overflow the int32 accumulator",
                             static_cast<unsigned long long>(K));
  SEEAI_TRY(c, LaunchGemmW8A8(QA, sa, QWt, sw, C, acc, M, N, K, c->policy, c->stream), "w8a8_gemm");
  return SEEAI_OK;
}

int seeai_attn_fwd(seeai_ctx* c, int dtype, const float* q, const float* k, const float* v, float* o,
                   float* stats, uint64_t B, uint64_t S, uint64_t H, uint64_t d,
                   const int32_t* starts) {
  if (!c || dtype < 0 || dtype > 1) return Fail(c, SEEAI_INVALID, "attn_fwd: dtype is 0 or 1");
  SEEAI_TRY(c, LaunchAttnFwdTiled(dtype, q, k, v, o, stats, B, S, H, d, starts, c->stream), "attn_fwd");
  return SEEAI_OK;
}
int seeai_attn_fwd_bf16(seeai_ctx* c, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                        float* o, float* stats, uint64_t B, uint64_t S, uint64_t H, uint64_t d,
                        const int32_t* starts) {
  if (!c) return SEEAI_INVALID;
  if (!Attn16Fits(B, S, H, d))
    return Fail(c, SEEAI_INVALID, "attn_fwd_bf16: head width %llu (64 only) or slice too large",
                static_cast<unsigned long long>(d));
  SEEAI_TRY(c, LaunchAttn16Fwd(q, k, v, o, stats, B, S, H, starts, c->stream), "attn_fwd_bf16");
  return SEEAI_OK;
}
int seeai_attn_dq_bf16(seeai_ctx* c, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                       const uint16_t* dout, float* stats, float* dq, uint64_t B, uint64_t S,
                       uint64_t H, uint64_t d) {
  if (!c) return SEEAI_INVALID;
  if (!Attn16Fits(B, S, H, d))
    return Fail(c, SEEAI_INVALID, "attn_dq_bf16: head width %llu (64 only) or slice too large",
                static_cast<unsigned long long>(d));
  SEEAI_TRY(c, LaunchAttn16DQ(q, k, v, dout, stats, dq, B, S, H, c->stream), "attn_dq_bf16");
  return SEEAI_OK;
}
int seeai_attn_dkdv_bf16(seeai_ctx* c, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                         const uint16_t* dout, const float* stats, float* dk, float* dv,
                         uint64_t B, uint64_t S, uint64_t H, uint64_t d) {
  if (!c) return SEEAI_INVALID;
  if (!Attn16Fits(B, S, H, d) || (!dk && !dv))
    return Fail(c, SEEAI_INVALID,
                "attn_dkdv_bf16: head width %llu (64 only), slice too large or no output",
                static_cast<unsigned long long>(d));
  SEEAI_TRY(c, LaunchAttn16DKDV(q, k, v, dout, stats, dk, dv, B, S, H, c->stream),
            "attn_dkdv_bf16");
  return SEEAI_OK;
}
int seeai_attn_dq(seeai_ctx* c, int dtype, const float* q, const float* k, const float* v,
                  const float* dout, float* stats, float* dq, uint64_t B, uint64_t S, uint64_t H,
                  uint64_t d) {
  if (!c || dtype < 0 || dtype > 1) return Fail(c, SEEAI_INVALID, "attn_dq: dtype is 0 or 1");
  SEEAI_TRY(c, LaunchAttnDQTiled(dtype, q, k, v, dout, stats, dq, B, S, H, d, c->stream), "attn_dq");
  return SEEAI_OK;
}
int seeai_attn_dk(seeai_ctx* c, int dtype, const float* q, const float* k, const float* v,
                  const float* dout, const float* stats, float* dk, uint64_t B, uint64_t S,
                  uint64_t H, uint64_t d) {
  if (!c || dtype < 0 || dtype > 1) return Fail(c, SEEAI_INVALID, "attn_dk: dtype is 0 or 1");
  SEEAI_TRY(c, LaunchAttnDKTiled(dtype, q, k, v, dout, stats, dk, B, S, H, d, c->stream), "attn_dk");
  return SEEAI_OK;
}
int seeai_attn_dv(seeai_ctx* c, int dtype, const float* q, const float* k, const float* dout,
                  const float* stats, float* dv, uint64_t B, uint64_t S, uint64_t H, uint64_t d) {
  if (!c || dtype < 0 || dtype > 1) return Fail(c, SEEAI_INVALID, "attn_dv: dtype is 0 or 1");
  SEEAI_TRY(c, LaunchAttnDVTiled(dtype, q, k, dout, stats, dv, B, S, H, d, c->stream), "attn_dv");
  return SEEAI_OK;
}
int seeai_attn_dkdv_f32(seeai_ctx* c, const float* q, const float* k, const float* v,
                        const float* dout, const float* stats, float* dk, float* dv, uint64_t B,
                        uint64_t S, uint64_t H, uint64_t d) {
  if (!c) return SEEAI_INVALID;
  if (!dk || !dv || !AttnDKDVExactFusable(q, k, v, dout, stats, dk, dv, B, S, H, d))
    return Fail(c, SEEAI_INVALID, "attn_dkdv_f32: the exact pass takes d = 64 or 128 with "
                                  "16-byte aligned operands and both outputs");
  SEEAI_TRY(c, LaunchAttnDKDVExact(q, k, v, dout, stats, dk, dv, B, S, H, d, c->stream),
            "attn_dkdv_f32");
  return SEEAI_OK;
}

int seeai_xent_fwd(seeai_ctx* c, const float* logits, const int32_t* labels, float* loss,
                   float* probs, uint64_t N, uint64_t C, int masked) {
  if (!c) return SEEAI_INVALID;
  void* ws;
  if (int rc = Scratch(c, XEntFwdScratchBytes(N), &ws)) return rc;
  SEEAI_TRY(c, LaunchXEntFwd(logits, labels, loss, probs, N, C, masked, ws, c->stream), "xent_fwd");
  return SEEAI_OK;
}
int seeai_xent_fwd_noalloc(seeai_ctx* c, const float* logits, const int32_t* labels, float* loss,
                           float* probs, uint64_t N, uint64_t C, int masked) {
  if (!c) return SEEAI_INVALID;
  if (N > SEEAI_XENT_NOALLOC_MAX_ROWS)
    return Fail(c, SEEAI_INVALID,
                "xent_fwd_noalloc: %llu rows exceed the %llu-row workspace (%zu bytes); use "
                "seeai_xent_fwd",
                static_cast<unsigned long long>(N),
                static_cast<unsigned long long>(SEEAI_XENT_NOALLOC_MAX_ROWS), kNoAllocScratchBytes);
  if (XEntFwdScratchBytes(N) > kNoAllocScratchBytes)
    return Fail(c, SEEAI_INVALID, "xent_fwd_noalloc: workspace too small");
  void* ws = g_noalloc[c->device].ptr;
  if (!ws) return Fail(c, SEEAI_HIP_ERROR, "xent_fwd_noalloc: no workspace address on this device");
  // Every word of the workspace the kernels read (row maxima, sums and
  // losses) is written by them first in this call: nothing to clear.
  SEEAI_TRY(c, LaunchXEntFwd(logits, labels, loss, probs, N, C, masked, ws, c->stream),
            "xent_fwd_noalloc");
  return SEEAI_OK;
}
int seeai_xent_bwd(seeai_ctx* c, const float* probs, const int32_t* labels, const float* seed,
                   float* dlogits, uint64_t N, uint64_t C, int masked) {
  if (!c) return SEEAI_INVALID;
  void* ws;
  if (int rc = Scratch(c, 64, &ws)) return rc;
  SEEAI_TRY(c, LaunchXEntBwd(probs, labels, seed, dlogits, N, C, masked, ws, c->stream), "xent_bwd");
  return SEEAI_OK;
}
int seeai_adamw_step(seeai_ctx* c, float* p, const float* g, float* m, float* v, uint64_t n,
                     const seeai_step_params* params, float clip_norm) {
  if (!c || !params) return SEEAI_INVALID;
  return AdamWLaunch(c, p, g, m, v, n, *params, clip_norm);
}
int seeai_argmax_rows(seeai_ctx* c, const float* probs, uint64_t rows, uint64_t cols, int32_t* out) {
  if (!c) return SEEAI_INVALID;
  SEEAI_TRY(c, LaunchArgmaxRows(probs, rows, cols, out, c->stream), "argmax");
  return SEEAI_OK;
}
int seeai_argmax_tally(seeai_ctx* c, const float* probs, const int32_t* labels, uint64_t rows,
                       uint64_t cols, uint64_t* hits, uint64_t* judged) {
  if (!c || !hits || !judged || (rows && (!probs || !labels)))
    return Fail(c, SEEAI_INVALID, "argmax_tally: null operand");
  if (rows > 0x7FFFFFFFull) return Fail(c, SEEAI_INVALID, "argmax_tally: too many rows");
  SEEAI_TRY(c, LaunchArgmaxTally(probs, labels, rows, cols, c->counts(), c->stream), "argmax_tally");
  uint64_t host[2];
  SEEAI_TRY(c, hipMemcpyAsync(host, c->counts(), sizeof host, hipMemcpyDeviceToHost, c->stream),
            "argmax_tally counts");
  SEEAI_TRY(c, hipStreamSynchronize(c->stream), "argmax_tally sync");
  *hits = host[0];
  *judged = host[1];
  return SEEAI_OK;
}

}  // extern "C"
