// hip_backend.cc -- ExecutorBackend over the C ABI (see hip_backend.h).
#include "hip_backend.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstring>
#include <thread>
#include <vector>

#include "seeai_hip.h"

namespace seeai::host {

Result<std::unique_ptr<HipBackend>> HipBackend::Create(int device) {
  seeai_ctx* ctx = nullptr;
  if (seeai_create(device, &ctx) != SEEAI_OK) {
    std::string why = ctx ? seeai_last_error(ctx) : "no HIP device";
    if (ctx) seeai_destroy(ctx);
    return Fail("hip backend: " + why);
  }
  return std::unique_ptr<HipBackend>(new HipBackend(ctx));
}

HipBackend::~HipBackend() { seeai_destroy(ctx_); }

std::string HipBackend::device() const {
  int dev = 0;
  hipDeviceProp_t prop{};
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess)
    return "AMD GPU";
  return std::string(prop.name) + " (" + prop.gcnArchName + ")";
}

Result<void> HipBackend::Check(int status) const {
  if (status == SEEAI_OK) return {};
  return Fail(seeai_last_error(ctx_));  // refusals carry the reference's exact words
}

Result<void> HipBackend::Bind(uint8_t* arena, uint64_t arena_bytes, const uint8_t* rodata,
                              uint64_t rodata_bytes, uint64_t /*rodata_mapped_bytes*/) {
  if (auto r = Check(seeai_bind(ctx_, arena_bytes, rodata, rodata_bytes)); !r) return r;
  host_ = arena;
  host_bytes_ = arena_bytes;
  // The device arena starts as the caller's copy.  seeai_bind hands it over
  // zeroed, so only the blocks of the caller's arena that hold a nonzero
  // byte are uploaded (a plan's arena is its persistent image followed by
  // zeros: C5's 23.6 GB arena uploads its few hundred MB of image).
  return UploadNonZero(arena, arena_bytes);
}

namespace {
bool AllZero(const uint8_t* p, uint64_t n) {
  uint64_t i = 0;
  for (; i < n && (reinterpret_cast<uintptr_t>(p + i) & 7) != 0; ++i)
    if (p[i]) return false;
  for (; i + 64 <= n; i += 64) {  // eight words per test
    uint64_t w[8];
    std::memcpy(w, p + i, sizeof w);
    if ((w[0] | w[1] | w[2] | w[3] | w[4] | w[5] | w[6] | w[7]) != 0) return false;
  }
  for (; i < n; ++i)
    if (p[i]) return false;
  return true;
}
}  // namespace

Result<void> HipBackend::UploadNonZero(const uint8_t* arena, uint64_t bytes) {
  constexpr uint64_t kBlock = uint64_t{4} << 20;
  const uint64_t nblocks = (bytes + kBlock - 1) / kBlock;
  if (nblocks == 0) return {};
  // The scan: blocks dealt round-robin to at most 16 host threads.
  std::vector<uint8_t> nonzero(nblocks, 0);
  const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
  const unsigned nt = static_cast<unsigned>(std::min<uint64_t>({hw, 16, nblocks}));
  auto scan = [&](unsigned t) {
    for (uint64_t b = t; b < nblocks; b += nt) {
      const uint64_t off = b * kBlock;
      nonzero[b] = !AllZero(arena + off, std::min(kBlock, bytes - off));
    }
  };
  std::vector<std::thread> pool;
  for (unsigned t = 1; t < nt; ++t) pool.emplace_back(scan, t);
  scan(0);
  for (auto& th : pool) th.join();
  // Each run of nonzero blocks goes up as one copy.
  for (uint64_t b = 0; b < nblocks;) {
    if (!nonzero[b]) {
      ++b;
      continue;
    }
    uint64_t e = b;
    while (e < nblocks && nonzero[e]) ++e;
    const uint64_t off = b * kBlock, n = std::min(e * kBlock, bytes) - off;
    if (auto r = Check(seeai_upload(ctx_, off, arena + off, n)); !r) return r;
    b = e;
  }
  return {};
}

Result<void> HipBackend::BindSource(const uint8_t* data, uint64_t bytes) {
  return Check(seeai_bind_source(ctx_, data, bytes));
}

Result<void> HipBackend::Configure(const seeai_tile_policy* policy) {
  return Check(seeai_configure(ctx_, policy));
}

Result<void> HipBackend::Execute(const Instruction& ins, const StepParams& p) {
  const seeai_step_params sp{p.lr, p.beta1, p.beta2, p.eps, p.weight_decay, 0, p.step};
  return Check(seeai_execute(ctx_, &ins, &sp));
}

void HipBackend::BeginRange(std::span<const Instruction> program, size_t begin, size_t end) {
  static_assert(sizeof(Instruction) == 64);
  (void)seeai_begin_range(ctx_, program.data(), program.size(), begin, end);
}

void HipBackend::EndRange() { (void)seeai_end_range(ctx_); }

Result<void> HipBackend::RunRange(std::span<const Instruction> program, size_t begin, size_t end,
                                  const StepParams& p, size_t* failed_at) {
  const seeai_step_params sp{p.lr, p.beta1, p.beta2, p.eps, p.weight_decay, 0, p.step};
  uint64_t at = begin;
  auto r = Check(seeai_run_range(ctx_, program.data(), program.size(), begin, end, &sp, &at));
  if (failed_at) *failed_at = static_cast<size_t>(at);
  return r;
}

uint64_t HipBackend::fused_dispatches() const { return seeai_fused_dispatches(ctx_); }

Result<void> HipBackend::Flush() { return Check(seeai_flush(ctx_)); }

Result<void> HipBackend::FlushSyncToHost(uint64_t offset, uint64_t bytes) {
  if (!host_ || offset > host_bytes_ || bytes > host_bytes_ - offset)
    return Fail("hip backend: sync range outside the bound arena");
  return Check(seeai_flush_download(ctx_, offset, host_ + offset, bytes));
}

uint64_t HipBackend::relaxed_executions() const { return seeai_relaxed_executions(ctx_); }

void HipBackend::SetRelaxed(bool allow) { seeai_set_relaxed(ctx_, allow ? 1 : 0); }

void HipBackend::SetAttentionBf16(bool on) { seeai_set_attention_bf16(ctx_, on ? 1 : 0); }

Result<void> HipBackend::SyncToDevice(uint64_t offset, uint64_t bytes) {
  if (!host_ || offset > host_bytes_ || bytes > host_bytes_ - offset)
    return Fail("hip backend: sync range outside the bound arena");
  return Check(seeai_upload(ctx_, offset, host_ + offset, bytes));
}

Result<void> HipBackend::SyncToHost(uint64_t offset, uint64_t bytes) {
  if (!host_ || offset > host_bytes_ || bytes > host_bytes_ - offset)
    return Fail("hip backend: sync range outside the bound arena");
  return Check(seeai_download(ctx_, offset, host_ + offset, bytes));
}

}  // namespace seeai::host
