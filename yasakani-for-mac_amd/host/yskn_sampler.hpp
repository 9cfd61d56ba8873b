// yskn_sampler.hpp -- C++ host interface of the MI355X sampler, mirroring the
// reference's Rust sampler API over the C ABI of include/yskn_smp.h.
//
//   Rust (crates/yskn-ref)                          here
//   SamplingVersion (output_head_sampler.rs:14-18)  yskn::SamplingVersion
//   SamplingParameters (:21-75)                     yskn::SamplingParameters
//   Sampler::{Greedy, Sampled} (:77-92)             yskn::Sampler::greedy() / sampled(p)
//   greedy / top_tokens (:103-134)                  yskn::greedy / yskn::top_tokens
//   negative_log_likelihood (:230-250)              yskn::negative_log_likelihood
//   trait Selector (speculation.rs:123-139)         yskn::Selector
//   Error::{InvalidInput, NonFinite} (lib.rs:37-45) yskn::Error::Kind
//   accept loop of generate (speculation.rs:483-523) yskn::verify_block
//
// Every call runs on the GPU (the C ABI has no CPU path). Host slices are
// copied to device memory first, as Selector::select's signature requires;
// engines that already hold logits in HBM call yskn_smp_sample directly.
// Results are Result<T> values, never exceptions, like the Rust API.
#pragma once

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "../../include/yskn_smp.h"

namespace yskn {

enum class SamplingVersion { InverseCumulative, Gumbel };

struct Error {
  enum class Kind { InvalidInput, NonFinite, Device };
  Kind kind;
  std::string message;
};

struct Unit {};

// Rust's Result<T, Error>.
template <class T>
class Result {
 public:
  Result(T value) : ok_(true), value_(std::move(value)) {}
  Result(Error error) : ok_(false), error_(std::move(error)) {}
  bool is_ok() const { return ok_; }
  bool is_err() const { return !ok_; }
  const T& value() const { return value_; }
  const Error& error() const { return error_; }

 private:
  bool ok_;
  T value_{};
  Error error_{Error::Kind::InvalidInput, ""};
};

namespace detail {

inline Error from_status(int status) {
  if (status == YSKN_SMP_ENONFINITE) return {Error::Kind::NonFinite, "logits"};
  if (status == YSKN_SMP_EDEVICE) return {Error::Kind::Device, yskn_smp_last_error()};
  return {Error::Kind::InvalidInput, yskn_smp_last_error()};
}

inline Error invalid(const char* message) { return {Error::Kind::InvalidInput, message}; }

// validate_logits (output_head_sampler.rs:94-101): nonempty, u32-indexed. The
// finite check runs on the device, with the same error.
inline bool vocabulary_ok(size_t n) { return n > 0 && n <= (size_t)INT32_MAX; }

// Device buffers that live as long as a handle.
struct Device {
  void* p = nullptr;
  explicit Device(size_t bytes) {
    if (hipMalloc(&p, bytes) != hipSuccess) p = nullptr;
  }
  ~Device() {
    if (p) (void)hipFree(p);
  }
  Device(const Device&) = delete;
  Device& operator=(const Device&) = delete;
};

struct Handle {
  yskn_smp_handle h = nullptr;
  int32_t max_vocab = 0;
  ~Handle() { yskn_smp_destroy(h); }
};

inline Result<std::shared_ptr<Handle>> make_handle(int32_t rows, int32_t vocab, uint32_t flags) {
  auto hd = std::make_shared<Handle>();
  const int st = yskn_smp_create(rows, vocab, flags, &hd->h);
  if (st != YSKN_SMP_OK) return from_status(st);
  hd->max_vocab = vocab;
  return hd;
}

}  // namespace detail

struct SamplingParameters {
  double temperature = 1.0;
  double top_p = 0.95;
  size_t top_k = 20;
  double min_p = 0.0;
  uint64_t seed = 0;
  SamplingVersion version = SamplingVersion::Gumbel;

  // Thousandths divided in binary64 (output_head_sampler.rs:43-54), then
  // validated against a vocabulary of 20 like the reference.
  static Result<SamplingParameters> from_thousandths(uint32_t temperature, uint32_t top_p, uint32_t min_p) {
    SamplingParameters p;
    p.temperature = (double)temperature / 1000.0;
    p.top_p = (double)top_p / 1000.0;
    p.min_p = (double)min_p / 1000.0;
    const Result<Unit> v = p.validate(20);
    if (v.is_err()) return v.error();
    return p;
  }

  // SamplingParameters::validate (output_head_sampler.rs:56-75).
  Result<Unit> validate(size_t vocabulary_size) const {
    const yskn_smp_params_f64 c = to_c(false);
    const int32_t v = (int32_t)std::min(vocabulary_size, (size_t)INT32_MAX);
    const int st = yskn_smp_validate_params_f64(&c, v, 0);
    if (st != YSKN_SMP_OK) return detail::from_status(st);
    return Unit{};
  }

  yskn_smp_params_f64 to_c(bool greedy) const {
    yskn_smp_params_f64 c;
    std::memset(&c, 0, sizeof c);
    c.temperature = temperature;
    c.top_p = top_p;
    c.min_p = min_p;
    c.top_k = (uint32_t)std::min(top_k, (size_t)UINT32_MAX);
    c.greedy = greedy ? 1 : 0;
    c.seed = seed;
    c.version = version == SamplingVersion::Gumbel ? YSKN_SMP_VERSION_GUMBEL : YSKN_SMP_VERSION_INVERSE_CDF;
    c.repetition_penalty = 1.0f;
    return c;
  }
};

// trait Selector (speculation.rs:123-139): the selection depends only on the
// logits and the absolute prediction position (input position + 1).
class Selector {
 public:
  virtual ~Selector() = default;
  virtual Result<uint32_t> select(const std::vector<float>& logits, uint64_t prediction_position) = 0;
};

// Sampler::{Greedy, Sampled(SamplingParameters)} (output_head_sampler.rs:77-92).
class Sampler final : public Selector {
 public:
  static Sampler greedy() { return Sampler(true, SamplingParameters{}); }
  static Sampler sampled(SamplingParameters p) { return Sampler(false, p); }

  bool is_greedy() const { return greedy_; }
  const SamplingParameters& parameters() const { return params_; }

  // `prediction_position` is the absolute input position plus one.
  Result<uint32_t> sample(const std::vector<float>& logits, uint64_t prediction_position) const {
    if (!detail::vocabulary_ok(logits.size()))
      return detail::invalid("invalid input: logits must contain a nonempty u32-indexed vocabulary");
    const int32_t V = (int32_t)logits.size();
    if (!handle_ || handle_->max_vocab < V) {
      Result<std::shared_ptr<detail::Handle>> hd = detail::make_handle(1, V, 0);
      if (hd.is_err()) return hd.error();
      const yskn_smp_params_f64 c = params_.to_c(greedy_);
      const int st = yskn_smp_set_params_f64(hd.value()->h, &c, 1);
      if (st != YSKN_SMP_OK) return detail::from_status(st);
      handle_ = hd.value();
    }
    uint32_t token = 0;
    const int st = yskn_smp_select_host(handle_->h, logits.data(), V, prediction_position, &token);
    if (st != YSKN_SMP_OK) return detail::from_status(st);
    return token;
  }

  Result<uint32_t> select(const std::vector<float>& logits, uint64_t prediction_position) override {
    return sample(logits, prediction_position);
  }

 private:
  Sampler(bool greedy, SamplingParameters p) : greedy_(greedy), params_(p) {}
  bool greedy_;
  SamplingParameters params_;
  mutable std::shared_ptr<detail::Handle> handle_;
};

namespace detail {

// One host row on the device for the pure functions of the logits.
struct HostRow {
  std::shared_ptr<Handle> hd;
  Device logits, out;
  HostRow(std::shared_ptr<Handle> h, size_t n, size_t out_bytes) : hd(std::move(h)), logits(n * 4), out(out_bytes) {}
};

inline Result<std::shared_ptr<HostRow>> host_row(const std::vector<float>& logits, size_t out_bytes) {
  if (!vocabulary_ok(logits.size()))
    return invalid("invalid input: logits must contain a nonempty u32-indexed vocabulary");
  Result<std::shared_ptr<Handle>> hd = make_handle(1, (int32_t)logits.size(), 0);
  if (hd.is_err()) return hd.error();
  auto row = std::make_shared<HostRow>(hd.value(), logits.size(), out_bytes);
  if (!row->logits.p || !row->out.p) return Error{Error::Kind::Device, "hipMalloc failed"};
  if (hipMemcpy(row->logits.p, logits.data(), logits.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
    return Error{Error::Kind::Device, "hipMemcpy failed"};
  return row;
}

inline Result<Unit> finish(const HostRow& row, int launch_status, void* host_out, size_t bytes) {
  if (launch_status != YSKN_SMP_OK) return from_status(launch_status);
  const int st = yskn_smp_sync(row.hd->h, nullptr);
  if (st != YSKN_SMP_OK) return from_status(st);
  if (hipMemcpy(host_out, row.out.p, bytes, hipMemcpyDeviceToHost) != hipSuccess)
    return Error{Error::Kind::Device, "hipMemcpy failed"};
  return Unit{};
}

}  // namespace detail

// greedy (output_head_sampler.rs:103-113): larger logit, then smaller id.
inline Result<uint32_t> greedy(const std::vector<float>& logits) {
  auto row = detail::host_row(logits, 4);
  if (row.is_err()) return row.error();
  const auto& r = *row.value();
  const int32_t V = (int32_t)logits.size();
  uint32_t id = 0;
  Result<Unit> f = detail::finish(r, yskn_smp_argmax(r.hd->h, r.logits.p, YSKN_SMP_F32, 1, V, V, (uint32_t*)r.out.p, nullptr), &id, 4);
  if (f.is_err()) return f.error();
  return id;
}

// top_tokens (output_head_sampler.rs:115-134): the first `count` ids in
// (logit desc, id asc) order, any count up to the vocabulary.
inline Result<std::vector<uint32_t>> top_tokens(const std::vector<float>& logits, size_t count) {
  if (!detail::vocabulary_ok(logits.size()))
    return detail::invalid("invalid input: logits must contain a nonempty u32-indexed vocabulary");
  if (count > logits.size()) return detail::invalid("invalid input: top-token count exceeds vocabulary");
  if (count == 0) {
    // the reference still validates the logits: one argmax pass does
    Result<uint32_t> g = greedy(logits);
    if (g.is_err()) return g.error();
    return std::vector<uint32_t>{};
  }
  auto row = detail::host_row(logits, count * 4);
  if (row.is_err()) return row.error();
  const auto& r = *row.value();
  const int32_t V = (int32_t)logits.size();
  std::vector<uint32_t> ids(count);
  Result<Unit> f = detail::finish(r, yskn_smp_top_tokens(r.hd->h, r.logits.p, YSKN_SMP_F32, 1, V, V, (int32_t)count,
                                                         (uint32_t*)r.out.p, nullptr, nullptr),
                                  ids.data(), count * 4);
  if (f.is_err()) return f.error();
  return ids;
}

// negative_log_likelihood (output_head_sampler.rs:230-250), within 1e-5
// relative of the reference's serial binary64 sum.
inline Result<double> negative_log_likelihood(const std::vector<float>& logits, uint32_t target) {
  if (!detail::vocabulary_ok(logits.size()))
    return detail::invalid("invalid input: logits must contain a nonempty u32-indexed vocabulary");
  if ((size_t)target >= logits.size()) return detail::invalid("invalid input: target token is outside the vocabulary");
  auto row = detail::host_row(logits, 8 + 4);
  if (row.is_err()) return row.error();
  const auto& r = *row.value();
  const int32_t V = (int32_t)logits.size();
  uint32_t* d_target = (uint32_t*)((char*)r.out.p + 8);
  if (hipMemcpy(d_target, &target, 4, hipMemcpyHostToDevice) != hipSuccess)
    return Error{Error::Kind::Device, "hipMemcpy failed"};
  double loss = 0.0;
  Result<Unit> f = detail::finish(r, yskn_smp_nll(r.hd->h, r.logits.p, YSKN_SMP_F32, 1, V, V, d_target, (double*)r.out.p, nullptr),
                                  &loss, 8);
  if (f.is_err()) return f.error();
  if (!(loss - loss == 0.0)) return Error{Error::Kind::NonFinite, "negative log-likelihood"};
  return loss;
}

// One verified block of speculative decoding (speculation.rs:483-523): row j
// of `target_logits` (M rows of V) is selected at prediction position
// base_position + j + 1; drafts[j] (j < M - 1) is accepted while it equals
// the selection; the first mismatch's selection, or the bonus row's, ends the
// block; an EOS id among the emitted tokens stops it.
struct VerifyResult {
  uint32_t accepted = 0;
  uint32_t emitted = 0;
  uint32_t token = 0;
  bool stop_eos = false;
  std::vector<uint32_t> selected;  // per row
};

inline Result<VerifyResult> verify_block(const SamplingParameters& params, bool greedy_rows,
                                         const std::vector<float>& target_logits, size_t rows,
                                         const std::vector<uint32_t>& drafts, uint64_t base_position,
                                         const std::vector<uint32_t>& eos_ids) {
  if (rows == 0 || target_logits.size() % rows != 0 || drafts.size() + 1 != rows)
    return detail::invalid("invalid input: M rows of logits and M - 1 drafts");
  const size_t V = target_logits.size() / rows;
  if (!detail::vocabulary_ok(V)) return detail::invalid("invalid input: logits must contain a nonempty u32-indexed vocabulary");
  Result<std::shared_ptr<detail::Handle>> hd = detail::make_handle((int32_t)rows, (int32_t)V, 0);
  if (hd.is_err()) return hd.error();
  const yskn_smp_params_f64 c = params.to_c(greedy_rows);
  int st = yskn_smp_set_params_f64(hd.value()->h, &c, 1);
  if (st != YSKN_SMP_OK) return detail::from_status(st);
  const size_t n_eos = eos_ids.size();
  detail::Device d_logits(target_logits.size() * 4), d_drafts((drafts.size() + 1) * 4), d_pos(8),
      d_eos((n_eos + 1) * 4), d_ids(rows * 4), d_res(sizeof(yskn_smp_verify_result));
  if (!d_logits.p || !d_drafts.p || !d_pos.p || !d_eos.p || !d_ids.p || !d_res.p)
    return Error{Error::Kind::Device, "hipMalloc failed"};
  bool ok = hipMemcpy(d_logits.p, target_logits.data(), target_logits.size() * 4, hipMemcpyHostToDevice) == hipSuccess;
  if (!drafts.empty()) ok = ok && hipMemcpy(d_drafts.p, drafts.data(), drafts.size() * 4, hipMemcpyHostToDevice) == hipSuccess;
  ok = ok && hipMemcpy(d_pos.p, &base_position, 8, hipMemcpyHostToDevice) == hipSuccess;
  if (n_eos) ok = ok && hipMemcpy(d_eos.p, eos_ids.data(), n_eos * 4, hipMemcpyHostToDevice) == hipSuccess;
  if (!ok) return Error{Error::Kind::Device, "hipMemcpy failed"};
  st = yskn_smp_verify(hd.value()->h, d_logits.p, YSKN_SMP_F32, (int32_t)rows, (int32_t)V, (int64_t)V,
                       (const uint32_t*)d_drafts.p, (const uint64_t*)d_pos.p, n_eos ? (const uint32_t*)d_eos.p : nullptr,
                       (int32_t)n_eos, (uint32_t*)d_ids.p, (yskn_smp_verify_result*)d_res.p, nullptr, nullptr,
                       nullptr);
  if (st != YSKN_SMP_OK) return detail::from_status(st);
  st = yskn_smp_sync(hd.value()->h, nullptr);
  if (st != YSKN_SMP_OK) return detail::from_status(st);
  yskn_smp_verify_result r;
  VerifyResult out;
  out.selected.resize(rows);
  ok = hipMemcpy(&r, d_res.p, sizeof r, hipMemcpyDeviceToHost) == hipSuccess &&
       hipMemcpy(out.selected.data(), d_ids.p, rows * 4, hipMemcpyDeviceToHost) == hipSuccess;
  if (!ok) return Error{Error::Kind::Device, "hipMemcpy failed"};
  out.accepted = r.accepted;
  out.emitted = r.emitted;
  out.token = r.token;
  out.stop_eos = r.stop_eos != 0;
  return out;
}

}  // namespace yskn
