// ref_shim.cc -- C entry points over the reference kernel library.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile compiles this file together
// with the reference's own kernel sources, where they lie under
// /root/reference (runtime/executor/{gemm,attention,loss,optimizer,
// elementwise,activation,normalization}.cc and
// source/parallel/parallel_for.cc), into oracle/_ref/libseeref.so.  The
// tests use it to pin the C restatement (oracle.c) bit-for-bit and to write
// the golden fixtures under tests/golden/.  Only this file's code is ours;
// it forwards plain pointers to the functions declared in the reference's
// runtime/executor/update_kernels.h:34-294.
#include <cstddef>
#include <cstdint>

#include "runtime/executor/update_kernels.h"
#include "source/identity/hash.h"
#include "source/parallel/parallel_for.h"

namespace k = seeml::update_rt::kernels;
namespace up = seeml::update;

static up::EpilogueAct Act(int act) { return static_cast<up::EpilogueAct>(act); }

extern "C" {

void ref_set_threads(size_t n) { up::SetParallelThreadCount(n); }

void ref_gemm_nn(const float* A, const float* B, float* C, size_t M, size_t N,
                 size_t K, const float* bias, int act, const float* addend,
                 float alpha) {
  k::GemmNN(A, B, C, M, N, K, bias, Act(act), k::kDefaultGemmTiles, addend,
            alpha);
}
void ref_gemm_nt(const float* A, const float* B, float* C, size_t M, size_t N,
                 size_t K, const float* addend, float alpha) {
  k::GemmNT(A, B, C, M, N, K, k::kDefaultGemmTiles, addend, alpha);
}
void ref_gemm_tn(const float* A, const float* B, float* C, size_t M, size_t N,
                 size_t K, const float* addend, float alpha) {
  k::GemmTN(A, B, C, M, N, K, k::kDefaultGemmTiles, addend, alpha);
}
void ref_gemm_acc_nn(const float* A, const float* B, float* C, size_t M,
                     size_t N, size_t K, float alpha) {
  k::GemmAccNN(A, B, C, M, N, K, alpha);
}
void ref_gemm_nn_q8(const float* A, const int8_t* B, float* C, size_t M,
                    size_t N, size_t K, float scale, int act,
                    const float* col_scale) {
  k::GemmNNQ8(A, B, C, M, N, K, scale, Act(act), k::kDefaultGemmTiles,
              col_scale);
}
void ref_gemm_nt_q8(const float* A, const int8_t* B, float* C, size_t M,
                    size_t N, size_t K, float scale, const float* k_scale) {
  k::GemmNTQ8(A, B, C, M, N, K, scale, k::kDefaultGemmTiles, k_scale);
}
void ref_gemm_nn_bf16(const float* A, const uint16_t* B, float* C, size_t M,
                      size_t N, size_t K, const float* bias, int act) {
  k::GemmNNBF16(A, B, C, M, N, K, bias, Act(act));
}
void ref_gemm_nt_bf16(const float* A, const uint16_t* B, float* C, size_t M,
                      size_t N, size_t K) {
  k::GemmNTBF16(A, B, C, M, N, K);
}

void ref_add_ew(const float* x, const float* y, float* o, size_t n) { k::AddEW(x, y, o, n); }
void ref_mul_ew(const float* x, const float* y, float* o, size_t n) { k::MulEW(x, y, o, n); }
void ref_add_bias(const float* x, const float* b, float* o, size_t r, size_t c) {
  k::AddBias(x, b, o, r, c);
}
void ref_relu_fwd(const float* x, float* o, size_t n) { k::ReluFwd(x, o, n); }
void ref_relu_bwd(const float* dy, const float* x, float* dx, size_t n) { k::ReluBwd(dy, x, dx, n); }
void ref_gelu_fwd(const float* x, float* o, size_t n) { k::GeluFwd(x, o, n); }
void ref_gelu_bwd(const float* dy, const float* x, float* dx, size_t n) { k::GeluBwd(dy, x, dx, n); }
void ref_silu_fwd(const float* x, float* o, size_t n) { k::SiluFwd(x, o, n); }
void ref_silu_bwd(const float* dy, const float* x, float* dx, size_t n) { k::SiluBwd(dy, x, dx, n); }
void ref_scale(const float* x, float* o, float a, size_t n) { k::Scale(x, o, a, n); }
void ref_reduce_rows(const float* dy, float* db, size_t r, size_t c) { k::ReduceRows(dy, db, r, c); }
void ref_accumulate(float* d, const float* s, size_t n) { k::Accumulate(d, s, n); }
void ref_embed_fwd(const int32_t* t, const float* table, float* o, size_t rows, size_t dim) {
  k::EmbedFwd(t, table, o, rows, dim);
}
void ref_fused_map(const float* x, const float* o1, const float* o2, float* out,
                   size_t n, uint64_t stages, float imm0, float imm1) {
  const float* others[3] = {nullptr, o1, o2};
  const float imm[2] = {imm0, imm1};
  k::FusedMap(x, others, out, n, stages, imm);
}
void ref_layernorm_fwd(const float* x, const float* g, const float* b, float* y,
                       float* mean, float* rstd, size_t r, size_t c, float eps) {
  k::LayerNormFwd(x, g, b, y, mean, rstd, r, c, eps);
}
void ref_layernorm_bwd(const float* dy, const float* x, const float* g,
                       const float* mean, const float* rstd, float* dx, size_t r,
                       size_t c) {
  k::LayerNormBwd(dy, x, g, mean, rstd, dx, r, c);
}
void ref_rmsnorm_fwd(const float* x, const float* g, float* y, float* rstd,
                     size_t r, size_t c, float eps) {
  k::RmsNormFwd(x, g, y, rstd, r, c, eps);
}
void ref_rmsnorm_bwd(const float* dy, const float* x, const float* g,
                     const float* rstd, float* dx, size_t r, size_t c) {
  k::RmsNormBwd(dy, x, g, rstd, dx, r, c);
}
void ref_rope(const float* x, float* y, size_t B, size_t S, size_t H, size_t d,
              float base, const float* table, int backward) {
  if (backward)
    k::RopeBwd(x, y, B, S, H, d, base, table);
  else
    k::RopeFwd(x, y, B, S, H, d, base, table);
}
void ref_rope_table(float* t, size_t S, size_t d, float base) { k::RopeTable(t, S, d, base); }

void ref_segment_starts(const int32_t* t, int32_t* s, size_t B, size_t S, int32_t eos) {
  k::SegmentStarts(t, s, B, S, eos);
}
void ref_attn_fwd(const float* q, const float* kk, const float* v, float* o,
                  float* p, size_t B, size_t S, size_t H, size_t d,
                  const int32_t* starts) {
  k::AttnFwd(q, kk, v, o, p, B, S, H, d, starts);
}
void ref_attn_dp(const float* dout, const float* v, float* dp, size_t B, size_t S,
                 size_t H, size_t d) {
  k::AttnDP(dout, v, dp, B, S, H, d);
}
void ref_attn_dv(const float* p, const float* dout, float* dv, size_t B, size_t S,
                 size_t H, size_t d) {
  k::AttnDV(p, dout, dv, B, S, H, d);
}
void ref_softmax_rows_bwd(const float* p, const float* dp, float* ds, size_t r, size_t c) {
  k::SoftmaxRowsBwd(p, dp, ds, r, c);
}
void ref_attn_dq(const float* ds, const float* kk, float* dq, size_t B, size_t S,
                 size_t H, size_t d) {
  k::AttnDQ(ds, kk, dq, B, S, H, d);
}
void ref_attn_dk(const float* ds, const float* q, float* dk, size_t B, size_t S,
                 size_t H, size_t d) {
  k::AttnDK(ds, q, dk, B, S, H, d);
}
void ref_attn_fwd_tiled(const float* q, const float* kk, const float* v, float* o,
                        float* st, size_t B, size_t S, size_t H, size_t d,
                        const int32_t* starts) {
  k::AttnFwdTiled(q, kk, v, o, st, B, S, H, d, starts);
}
void ref_attn_dq_tiled(const float* q, const float* kk, const float* v,
                       const float* dout, float* st, float* dq, size_t B, size_t S,
                       size_t H, size_t d) {
  k::AttnDQTiled(q, kk, v, dout, st, dq, B, S, H, d);
}
void ref_attn_dk_tiled(const float* q, const float* kk, const float* v,
                       const float* dout, const float* st, float* dk, size_t B,
                       size_t S, size_t H, size_t d) {
  k::AttnDKTiled(q, kk, v, dout, st, dk, B, S, H, d);
}
void ref_attn_dv_tiled(const float* q, const float* kk, const float* dout,
                       const float* st, float* dv, size_t B, size_t S, size_t H,
                       size_t d) {
  k::AttnDVTiled(q, kk, dout, st, dv, B, S, H, d);
}

void ref_xent_fwd(const float* l, const int32_t* y, float* loss, float* p, size_t N, size_t C) {
  k::SoftmaxXEntFwd(l, y, loss, p, N, C);
}
void ref_xent_bwd(const float* p, const int32_t* y, const float* seed, float* dl,
                  size_t N, size_t C) {
  k::SoftmaxXEntBwd(p, y, seed, dl, N, C);
}
void ref_xent_masked_fwd(const float* l, const int32_t* y, float* loss, float* p,
                         size_t N, size_t C) {
  k::SoftmaxXEntMaskedFwd(l, y, loss, p, N, C);
}
void ref_xent_masked_bwd(const float* p, const int32_t* y, const float* seed,
                         float* dl, size_t N, size_t C) {
  k::SoftmaxXEntMaskedBwd(p, y, seed, dl, N, C);
}

int ref_clip_norm(float* g, size_t n, float mx) { return k::ClipNorm(g, n, mx) ? 1 : 0; }
void ref_sqnorm_accum(const float* g, size_t n, float* acc) { k::SqNormAccum(g, n, acc); }
int ref_clip_global(float* g, size_t n, const float* acc, float mx) {
  return k::ClipGlobal(g, n, acc, mx) ? 1 : 0;
}
int ref_sgd_step(float* p, const float* g, size_t n, float lr, float wd, float clip) {
  return k::SgdStep(p, g, n, lr, wd, clip) ? 1 : 0;
}
int ref_adamw_step(float* p, const float* g, float* m, float* v, size_t n, float lr,
                   float b1, float b2, float eps, float wd, uint64_t step,
                   float clip) {
  return k::AdamWStep(p, g, m, v, n, lr, b1, b2, eps, wd, step, clip) ? 1 : 0;
}

uint64_t ref_plan_self_hash(const uint8_t* plan, size_t size, size_t hash_offset) {
  return seeml::update::PlanSelfHash(plan, size, hash_offset);
}

}  // extern "C"
