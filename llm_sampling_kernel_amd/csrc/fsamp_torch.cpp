// fsamp_torch.cpp -- the torch extension module of the sampler (import name _fsamp_torch,
// re-exported as llm_sampling_kernel_amd.fused_sampling).
//
// The same functions, argument order and error messages as the reference's pybind11 module
// `fused_sampling` (csrc/bindings.cpp:16-25, csrc/fused_sampling.cu:341-540), plus the
// explicit-uniform, per-row and shard entries.  Every sampler call is one fsamp_run (the C ABI
// of include/fsamp.h, in libfsamp.so) on torch's current HIP stream:
//   - out (and the split candidates when a row is split) come from torch's caching allocator,
//     so a call allocates nothing that launches, and a captured HIP graph keeps its own;
//   - the split-row arrival counters live in one buffer per device, zeroed once when it is
//     created and left zero by every call; it never shares memory with the candidates, so calls
//     of any batch size, captured or not, can follow one another in any order;
//   - offset < 0 takes (seed, offset) from torch's default generator of the logits' device with
//     philox_cuda_state(4) under the generator's lock, as csrc/fused_sampling.cu:441-447 does.
//     Outside capture that is the generator's values; under capture the graph's seed and offset
//     pointers plus the offset within the graph, which the kernel reads, so eager calls and
//     every replay draw from the one generator stream.
// Written directly against torch's HIP headers (c10/hip, ATen/hip); no hipify step.

#include <torch/extension.h>

#include <ATen/hip/HIPGeneratorImpl.h>
#include <c10/hip/HIPGuard.h>
#include <c10/hip/HIPStream.h>

#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "fsamp.h"

namespace {

void check_status(int rc) {
  TORCH_CHECK(rc == FSAMP_OK, fsamp_error_string(rc));
}

int dtype_of(const at::Tensor& logits) {
  TORCH_CHECK(logits.is_cuda() && logits.dim() == 2 && logits.is_contiguous(),
              "logits must be a contiguous cuda [B, V] tensor");
  TORCH_CHECK(logits.scalar_type() == at::kBFloat16 || logits.scalar_type() == at::kHalf,
              "logits must be float16 or bfloat16");
  return logits.scalar_type() == at::kBFloat16 ? FSAMP_DTYPE_BF16 : FSAMP_DTYPE_F16;
}

void check_top_k(int64_t top_k, int64_t V) {
  TORCH_CHECK(top_k >= 1, "top_k must be >= 1");
  TORCH_CHECK(std::min(top_k, V) <= FSAMP_K_MAX, "top_k must be <= ", FSAMP_K_MAX);
}

void check_top_p(double top_p) {
  TORCH_CHECK(top_p > 0.0 && top_p <= 1.0, "top_p must be in (0, 1]");
}

hipStream_t stream_of(const at::Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

// Per-device arrival counters.  A buffer is never freed: a captured graph may hold its address.
constexpr int64_t kCounterRows = 4096;
std::mutex g_counter_mu;
std::vector<at::Tensor> g_counters;  // by device index (undefined: none yet)
std::vector<at::Tensor> g_retired;

void* counters_for(const at::Tensor& logits, int64_t B, size_t* bytes) {
  const size_t need = fsamp_counter_bytes(B);
  const int dev = logits.device().index();
  std::lock_guard<std::mutex> lock(g_counter_mu);
  if ((int)g_counters.size() <= dev) g_counters.resize(dev + 1);
  at::Tensor& buf = g_counters[dev];
  if (!buf.defined() || (size_t)buf.numel() < need) {
    TORCH_CHECK(c10::hip::currentStreamCaptureStatusMayInitCtx() ==
                    c10::hip::CaptureStatus::None,
                "the sampler's row counters for batch ", B, " do not exist yet on this device: "
                "call the sampler once outside graph capture (a warm-up call) first");
    const size_t cap = std::max(need, fsamp_counter_bytes(kCounterRows));
    if (buf.defined()) g_retired.push_back(buf);
    buf = at::zeros({(int64_t)cap}, logits.options().dtype(at::kByte));
  }
  *bytes = (size_t)buf.numel();
  return buf.data_ptr();
}

struct Draw {
  uint64_t seed = 0, offset = 0;
  const int64_t* seed_ptr = nullptr;
  const int64_t* offset_ptr = nullptr;
};

// The reference's generator path, csrc/fused_sampling.cu:441-447 (+ philox::unpack, :296-300).
Draw generator_draw(const at::Tensor& logits) {
  auto gen = at::cuda::detail::getDefaultCUDAGenerator(logits.device().index());
  at::PhiloxCudaState st;
  {
    std::lock_guard<std::mutex> lock(gen.mutex());
    st = at::check_generator<at::CUDAGeneratorImpl>(gen)->philox_cuda_state(4);
  }
  Draw d;
  if (st.captured_) {
    d.seed_ptr = st.seed_.ptr;
    d.offset_ptr = st.offset_.ptr;
    d.offset = st.offset_intragraph_;
  } else {
    d.seed = st.seed_.val;
    d.offset = st.offset_.val;
  }
  return d;
}

const float* u_ptr(const c10::optional<at::Tensor>& u, const at::Tensor& logits) {
  if (!u.has_value()) return nullptr;
  const at::Tensor& t = *u;
  TORCH_CHECK(t.is_cuda() && t.scalar_type() == at::kFloat && t.is_contiguous() &&
                  t.numel() == logits.size(0) && t.device() == logits.device(),
              "u must be a contiguous float32 cuda tensor with one value per row");
  return t.data_ptr<float>();
}

template <typename T>
const T* row_ptr(const c10::optional<at::Tensor>& a, const at::Tensor& logits, at::ScalarType st,
                 const char* name) {
  if (!a.has_value()) return nullptr;
  const at::Tensor& t = *a;
  TORCH_CHECK(t.is_cuda() && t.scalar_type() == st && t.is_contiguous() &&
                  t.numel() == logits.size(0) && t.device() == logits.device(),
              name, " must be a contiguous ", c10::toString(st),
              " cuda tensor with one value per row");
  return static_cast<const T*>(t.data_ptr());
}

// Fills the workspace fields of `c` (counters and, for split rows, per-call scratch that must
// outlive the launch: returned so the caller holds it until the call is enqueued).
at::Tensor attach_workspace(fsamp_call& c, const at::Tensor& logits) {
  at::Tensor scratch;
  const size_t sb = fsamp_scratch_bytes(logits.data_ptr(), c.batch, c.vocab, c.top_k,
                                        c.splits_override);
  if (sb == 0) return scratch;
  c.counters = counters_for(logits, c.batch, &c.counter_bytes);
  scratch = at::empty({(int64_t)sb}, logits.options().dtype(at::kByte));
  c.scratch = scratch.data_ptr();
  c.scratch_bytes = sb;
  return scratch;
}

fsamp_call base_call(const at::Tensor& logits, int dtype, int64_t top_k, double top_p,
                     int64_t splits_override) {
  fsamp_call c;
  memset(&c, 0, sizeof(c));
  c.struct_bytes = sizeof(c);
  c.logits = logits.data_ptr();
  c.dtype = dtype;
  c.batch = logits.size(0);
  c.vocab = logits.size(1);
  c.ld = logits.size(1);
  c.top_k = top_k;
  c.top_p = top_p;
  c.splits_override = splits_override;
  return c;
}

std::vector<at::Tensor> run_sample(const at::Tensor& logits, int64_t top_k, double top_p,
                                   int64_t seed, int64_t offset, int64_t splits_override,
                                   const c10::optional<at::Tensor>& u, bool stages,
                                   const c10::optional<at::Tensor>& top_k_row,
                                   const c10::optional<at::Tensor>& top_p_row,
                                   const c10::optional<at::Tensor>& temperature) {
  const int dtype = dtype_of(logits);
  const int64_t B = logits.size(0), V = logits.size(1);
  check_top_k(top_k, V);
  check_top_p(top_p);
  const c10::hip::HIPGuard guard(logits.device().index());
  fsamp_call c = base_call(logits, dtype, top_k, top_p, splits_override);
  c.u = u_ptr(u, logits);
  if (c.u == nullptr) {
    if (offset < 0) {
      const Draw d = generator_draw(logits);
      c.seed = d.seed;
      c.offset = d.offset;
      c.seed_ptr = d.seed_ptr;
      c.offset_ptr = d.offset_ptr;
    } else {
      c.seed = (uint64_t)seed;
      c.offset = (uint64_t)offset;
    }
  }
  c.top_k_row = row_ptr<int32_t>(top_k_row, logits, at::kInt, "top_k_row");
  c.top_p_row = row_ptr<float>(top_p_row, logits, at::kFloat, "top_p_row");
  c.temperature_row = row_ptr<float>(temperature, logits, at::kFloat, "temperature");
  at::Tensor out = at::empty({B}, logits.options().dtype(at::kLong));
  c.out = out.data_ptr<int64_t>();
  at::Tensor keep, renormed;
  if (stages) {
    const int64_t K = std::min(top_k, V);
    keep = at::empty({B, K}, logits.options().dtype(at::kBool));
    renormed = at::empty({B, K}, logits.options().dtype(at::kFloat));
    c.keep = reinterpret_cast<uint8_t*>(keep.data_ptr());
    c.renormed = renormed.data_ptr<float>();
  }
  const at::Tensor scratch = attach_workspace(c, logits);
  check_status(fsamp_run(&c, stream_of(logits)));
  if (stages) return {out, keep, renormed};
  return {out};
}

// ---- the reference's functions (csrc/bindings.cpp:16-25) ----------------------------------

at::Tensor sample_fused(at::Tensor logits, int64_t top_k, double top_p, int64_t seed,
                        int64_t offset, int64_t splits_override) {
  return run_sample(logits, top_k, top_p, seed, offset, splits_override, c10::nullopt, false,
                    c10::nullopt, c10::nullopt, c10::nullopt)[0];
}

std::vector<at::Tensor> stages_fused(at::Tensor logits, int64_t top_k, double top_p, int64_t seed,
                                     int64_t offset, int64_t splits_override) {
  TORCH_CHECK(offset >= 0, "stages_fused takes an explicit offset >= 0");
  return run_sample(logits, top_k, top_p, seed, offset, splits_override, c10::nullopt, true,
                    c10::nullopt, c10::nullopt, c10::nullopt);
}

at::Tensor topk_fused(at::Tensor logits, int64_t top_k, int64_t splits_override) {
  const int dtype = dtype_of(logits);
  const int64_t B = logits.size(0), V = logits.size(1);
  check_top_k(top_k, V);
  const c10::hip::HIPGuard guard(logits.device().index());
  fsamp_call c = base_call(logits, dtype, top_k, 1.0, splits_override);
  at::Tensor ids = at::empty({B, std::min(top_k, V)}, logits.options().dtype(at::kLong));
  c.ids = ids.data_ptr<int64_t>();
  const at::Tensor scratch = attach_workspace(c, logits);
  check_status(fsamp_run(&c, stream_of(logits)));
  return ids;
}

at::Tensor probe_phase(at::Tensor logits, int64_t top_k, double top_p, int64_t phase,
                       int64_t splits_override) {
  const int dtype = dtype_of(logits);
  const int64_t B = logits.size(0), V = logits.size(1);
  check_top_k(top_k, V);
  check_top_p(top_p);
  TORCH_CHECK(phase >= 1 && phase <= 7, "phase must be in [1, 7]");
  const c10::hip::HIPGuard guard(logits.device().index());
  // the ablation keeps the classic single-buffer workspace: counters, then candidates
  const size_t wb = fsamp_workspace_bytes(logits.data_ptr(), B, V, top_k, splits_override);
  at::Tensor ws = at::zeros({(int64_t)wb}, logits.options().dtype(at::kByte));
  at::Tensor out = at::zeros({B}, logits.options().dtype(at::kLong));
  check_status(fsamp_probe_phase(logits.data_ptr(), dtype, B, V, top_k, top_p, phase,
                                 out.data_ptr<int64_t>(), ws.data_ptr(), wb, splits_override,
                                 stream_of(logits)));
  return out;
}

at::Tensor probe_noop(at::Tensor logits) {
  dtype_of(logits);
  const c10::hip::HIPGuard guard(logits.device().index());
  at::Tensor out = at::empty({logits.size(0)}, logits.options().dtype(at::kLong));
  check_status(fsamp_probe_noop(logits.size(0), out.data_ptr<int64_t>(), stream_of(logits)));
  return out;
}

at::Tensor probe_scan_rowblock(at::Tensor logits) {
  const int dtype = dtype_of(logits);
  const c10::hip::HIPGuard guard(logits.device().index());
  at::Tensor out = at::empty({logits.size(0)}, logits.options().dtype(at::kLong));
  check_status(fsamp_probe_scan_rowblock(logits.data_ptr(), dtype, logits.size(0),
                                         logits.size(1), out.data_ptr<int64_t>(),
                                         stream_of(logits)));
  return out;
}

at::Tensor probe_scan_split(at::Tensor logits, int64_t splits) {
  const int dtype = dtype_of(logits);
  TORCH_CHECK(splits >= 1, "splits must be >= 1");
  const c10::hip::HIPGuard guard(logits.device().index());
  const int64_t B = logits.size(0);
  at::Tensor partial = at::empty({B, splits}, logits.options().dtype(at::kLong));
  at::Tensor out = at::empty({B}, logits.options().dtype(at::kLong));
  check_status(fsamp_probe_scan_split(logits.data_ptr(), dtype, B, logits.size(1), splits,
                                      out.data_ptr<int64_t>(), partial.data_ptr(),
                                      (size_t)partial.numel() * 8, stream_of(logits)));
  return out;
}

std::vector<std::tuple<std::string, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t>>
kernel_attrs() {
  int32_t n = 0;
  check_status(fsamp_kernel_attrs(nullptr, 0, &n));
  std::vector<fsamp_attr_row> rows(n);
  check_status(fsamp_kernel_attrs(rows.data(), n, &n));
  std::vector<std::tuple<std::string, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t>> res;
  for (const auto& r : rows)
    res.emplace_back(r.name, r.chunks, r.threads, r.vgprs, r.scratch_bytes, r.lds_bytes,
                     r.blocks_per_cu);
  return res;
}

// ---- additions: explicit u, per-row controls, probes, shards --------------------------------

at::Tensor sample_fused_u(at::Tensor logits, int64_t top_k, double top_p, at::Tensor u,
                          int64_t splits_override) {
  return run_sample(logits, top_k, top_p, 0, 0, splits_override, u, false, c10::nullopt,
                    c10::nullopt, c10::nullopt)[0];
}

std::vector<at::Tensor> stages_fused_u(at::Tensor logits, int64_t top_k, double top_p,
                                       at::Tensor u, int64_t splits_override) {
  return run_sample(logits, top_k, top_p, 0, 0, splits_override, u, true, c10::nullopt,
                    c10::nullopt, c10::nullopt);
}

py::object sample_fused_ex(at::Tensor logits, int64_t top_k, double top_p,
                           c10::optional<at::Tensor> u, int64_t seed, int64_t offset,
                           c10::optional<at::Tensor> top_k_row,
                           c10::optional<at::Tensor> top_p_row,
                           c10::optional<at::Tensor> temperature, int64_t splits_override,
                           bool stages) {
  auto r = run_sample(logits, top_k, top_p, seed, offset, splits_override, u, stages, top_k_row,
                      top_p_row, temperature);
  if (stages) return py::cast(r);
  return py::cast(r[0]);
}

at::Tensor probe_load(at::Tensor logits, c10::optional<at::Tensor> wave_max) {
  const int dtype = dtype_of(logits);
  const int64_t B = logits.size(0);
  const c10::hip::HIPGuard guard(logits.device().index());
  at::Tensor wm = wave_max.has_value() ? *wave_max
                                       : at::empty({B * 8}, logits.options().dtype(at::kInt));
  TORCH_CHECK(wm.is_cuda() && wm.scalar_type() == at::kInt && wm.is_contiguous() &&
                  wm.numel() >= B * 8,
              "wave_max must be a contiguous int32 cuda tensor of B*8 entries");
  check_status(fsamp_probe_load(logits.data_ptr(), dtype, B, logits.size(1),
                                reinterpret_cast<uint32_t*>(wm.data_ptr()), stream_of(logits)));
  return wm.narrow(0, 0, B * 8).view({B, 8});
}

at::Tensor probe_stream(at::Tensor logits, c10::optional<at::Tensor> wave_max) {
  const int dtype = dtype_of(logits);
  TORCH_CHECK(logits.is_contiguous(), "logits must be a contiguous cuda [B, V] tensor");
  const int64_t B = logits.size(0), V = logits.size(1);
  const int64_t n = fsamp_probe_stream_words(B, V);
  const c10::hip::HIPGuard guard(logits.device().index());
  at::Tensor wm = wave_max.has_value() ? *wave_max
                                       : at::empty({n}, logits.options().dtype(at::kInt));
  TORCH_CHECK(wm.is_cuda() && wm.scalar_type() == at::kInt && wm.is_contiguous(),
              "wave_max must be a contiguous int32 cuda tensor");
  check_status(fsamp_probe_stream(logits.data_ptr(), dtype, B, V,
                                  reinterpret_cast<uint32_t*>(wm.data_ptr()), wm.numel(),
                                  stream_of(logits)));
  return wm.narrow(0, 0, n);
}

// logits_shard: [B, V_shard] with any row stride (a column slice of the whole logits is fine)
at::Tensor topk_shard(at::Tensor logits_shard, int64_t top_k, int64_t id_offset,
                      int64_t splits_override) {
  TORCH_CHECK(logits_shard.is_cuda() && logits_shard.dim() == 2 && logits_shard.stride(1) == 1,
              "logits must be a cuda [B, V] tensor with unit column stride");
  TORCH_CHECK(logits_shard.scalar_type() == at::kBFloat16 ||
                  logits_shard.scalar_type() == at::kHalf,
              "logits must be float16 or bfloat16");
  const int dtype = logits_shard.scalar_type() == at::kBFloat16 ? FSAMP_DTYPE_BF16
                                                                 : FSAMP_DTYPE_F16;
  const int64_t B = logits_shard.size(0), V = logits_shard.size(1);
  check_top_k(top_k, V);
  TORCH_CHECK(top_k <= V, "top_k must be <= the shard's vocabulary");
  const c10::hip::HIPGuard guard(logits_shard.device().index());
  fsamp_call c = base_call(logits_shard, dtype, top_k, 1.0, splits_override);
  c.ld = logits_shard.stride(0);
  c.id_offset = id_offset;
  at::Tensor words = at::empty({B, top_k}, logits_shard.options().dtype(at::kLong));
  c.words = reinterpret_cast<uint64_t*>(words.data_ptr());
  const at::Tensor scratch = attach_workspace(c, logits_shard);
  check_status(fsamp_run(&c, stream_of(logits_shard)));
  return words;
}

// words: [B, N, k] int64 (uint64 words); returns token ids [B], or [ids, keep, renormed]
py::object merge_sample(at::Tensor words, int64_t dtype_code, double top_p,
                        c10::optional<at::Tensor> u, int64_t seed, int64_t offset, bool stages,
                        bool ids_only) {
  TORCH_CHECK(words.is_cuda() && words.dim() == 3 && words.is_contiguous() &&
                  words.scalar_type() == at::kLong,
              "words must be a contiguous int64 cuda [B, N, k] tensor");
  check_top_p(top_p);
  const int64_t B = words.size(0), N = words.size(1), K = words.size(2);
  TORCH_CHECK(K >= 1 && K <= FSAMP_K_MAX, "top_k must be <= ", FSAMP_K_MAX);
  const c10::hip::HIPGuard guard(words.device().index());
  const float* up = nullptr;
  if (u.has_value()) {
    TORCH_CHECK(u->is_cuda() && u->scalar_type() == at::kFloat && u->is_contiguous() &&
                    u->numel() == B,
                "u must be a contiguous float32 cuda tensor with one value per row");
    up = u->data_ptr<float>();
  }
  auto opts = words.options();
  hipStream_t st = c10::hip::getCurrentHIPStream(words.device().index()).stream();
  if (ids_only) {
    at::Tensor ids = at::empty({B, K}, opts.dtype(at::kLong));
    check_status(fsamp_merge_sample(reinterpret_cast<const uint64_t*>(words.data_ptr()),
                                    (int)dtype_code, B, N, K, top_p, up, (uint64_t)seed,
                                    (uint64_t)offset, nullptr, nullptr, nullptr,
                                    ids.data_ptr<int64_t>(), st));
    return py::cast(ids);
  }
  at::Tensor out = at::empty({B}, opts.dtype(at::kLong));
  at::Tensor keep, renormed;
  if (stages) {
    keep = at::empty({B, K}, opts.dtype(at::kBool));
    renormed = at::empty({B, K}, opts.dtype(at::kFloat));
  }
  check_status(fsamp_merge_sample(
      reinterpret_cast<const uint64_t*>(words.data_ptr()), (int)dtype_code, B, N, K, top_p, up,
      (uint64_t)seed, (uint64_t)offset, out.data_ptr<int64_t>(),
      stages ? reinterpret_cast<uint8_t*>(keep.data_ptr()) : nullptr,
      stages ? renormed.data_ptr<float>() : nullptr, nullptr, st));
  if (stages) return py::cast(std::vector<at::Tensor>{out, keep, renormed});
  return py::cast(out);
}

}  // namespace

PYBIND11_MODULE(_fsamp_torch, m) {
  m.doc() = "MI355X fused top-k + top-p sampler (libfsamp.so through its C ABI)";
  m.def("sample_fused", &sample_fused, "fused top-k + top-p + sample, [B, V] -> [B]");
  m.def("topk_fused", &topk_fused, "debug: the selected candidate ids, descending");
  m.def("stages_fused", &stages_fused, "debug: (token_ids, keep, renormed) for Gate A");
  m.def("probe_phase", &probe_phase, "ablation: run phases 1..n of the pipeline and stop");
  m.def("probe_noop", &probe_noop, "launch floor: allocate [B] and write it");
  m.def("probe_scan_rowblock", &probe_scan_rowblock, "one full pass, one workgroup per row");
  m.def("probe_scan_split", &probe_scan_split, "one full pass split over workgroups, then a merge");
  m.def("kernel_attrs", &kernel_attrs, "debug: registers, spills, LDS, occupancy per kernel");
  m.def("sample_fused_u", &sample_fused_u, "sample with one fp32 uniform per row",
        py::arg("logits"), py::arg("top_k"), py::arg("top_p"), py::arg("u"),
        py::arg("splits_override") = 0);
  m.def("stages_fused_u", &stages_fused_u, "stages_fused with one fp32 uniform per row",
        py::arg("logits"), py::arg("top_k"), py::arg("top_p"), py::arg("u"),
        py::arg("splits_override") = 0);
  m.def("sample_fused_ex", &sample_fused_ex, "per-row top_k / top_p / temperature",
        py::arg("logits"), py::arg("top_k"), py::arg("top_p"), py::kw_only(),
        py::arg("u") = py::none(), py::arg("seed") = 0, py::arg("offset") = -1,
        py::arg("top_k_row") = py::none(), py::arg("top_p_row") = py::none(),
        py::arg("temperature") = py::none(), py::arg("splits_override") = 0,
        py::arg("stages") = false);
  m.def("probe_stream", &probe_stream,
        "streaming-read floor of the whole batch: per-wave maximum keys of 4 KB blocks",
        py::arg("logits"), py::arg("wave_max") = py::none());
  m.def("probe_load", &probe_load, "load-only floor: per-wave maximum keys [B, 8]",
        py::arg("logits"), py::arg("wave_max") = py::none());
  m.def("topk_shard", &topk_shard, "one vocabulary shard: sorted candidate words [B, k]",
        py::arg("logits_shard"), py::arg("top_k"), py::arg("id_offset"),
        py::arg("splits_override") = 0);
  m.def("merge_sample", &merge_sample, "merge N shard lists per row and sample",
        py::arg("words"), py::arg("dtype_code"), py::arg("top_p"), py::arg("u") = py::none(),
        py::arg("seed") = 0, py::arg("offset") = 0, py::arg("stages") = false,
        py::arg("ids_only") = false);
}
