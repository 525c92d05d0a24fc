// Host-side helper of the operator mirrors (whallm_amd/operators.py), built as a CPython
// extension against torch (no device code): the pool check of a resident expert set, which
// in Python spends most of a resident-expert call reading tensor metadata attribute by
// attribute.
//
// pool_regions(flat, n): flat holds n experts' four region tensors, expert-major
// (gate_up, gate_up_scales, down, down_scales of expert 0, then expert 1, ...). When every
// region r of every expert is a 2-D view of the storage of expert 0's region r, with the
// same shape, strides and dtype, at offsets that are slot * step from the lowest one (the
// slot views of a pool, or [i] of region-major tensors: how the reference's get_many hands
// out resident experts, expert_cache.py:488-497), it returns (fields, slot_of): the four
// regions as [max slot + 1, rows, cols] views from the lowest offset on, and each expert's
// slot (its offset in the first region over the gcd of the offset differences). Else None.
// The rules are those of operators._pool_regions, the same check in Python, which is also
// the fallback when this module is not built.
#include <torch/extension.h>

#include <algorithm>
#include <numeric>
#include <vector>

namespace {

py::object pool_regions(const std::vector<at::Tensor>& flat, int64_t n) {
  if (n <= 0 || (int64_t)flat.size() != 4 * n) return py::none();
  std::vector<int64_t> slot_of;
  std::vector<at::Tensor> fields;
  std::vector<int64_t> offs((size_t)n);
  for (int r = 0; r < 4; ++r) {
    const at::Tensor& t0 = flat[r];
    if (t0.dim() != 2) return py::none();
    const auto shape = t0.sizes();
    const auto stride = t0.strides();
    const auto dtype = t0.scalar_type();
    const int64_t size = (int64_t)t0.element_size();
    const auto& storage = t0.storage();
    const auto base = reinterpret_cast<intptr_t>(storage.data());
    const auto nbytes = (int64_t)storage.nbytes();
    for (int64_t e = 0; e < n; ++e) {
      const at::Tensor& t = flat[4 * e + r];
      if (t.sizes() != shape || t.strides() != stride || t.scalar_type() != dtype) return py::none();
      const int64_t at = (int64_t)(reinterpret_cast<intptr_t>(t.data_ptr()) - base);
      if (at < 0 || at >= nbytes || at % size) return py::none();
      offs[(size_t)e] = at / size;
    }
    const int64_t lo = *std::min_element(offs.begin(), offs.end());
    const int64_t numel = t0.numel();
    if (slot_of.empty()) {  // slot numbers from the first region's offsets
      int64_t unit = 0;
      for (int64_t o : offs) unit = std::gcd(unit, o - lo);
      if (unit == 0) unit = numel;
      slot_of.resize((size_t)n);
      for (int64_t e = 0; e < n; ++e) slot_of[(size_t)e] = (offs[(size_t)e] - lo) / unit;
      std::vector<int64_t> sorted = slot_of;
      std::sort(sorted.begin(), sorted.end());
      if (std::adjacent_find(sorted.begin(), sorted.end()) != sorted.end()) return py::none();
    }
    const auto top_it = std::max_element(slot_of.begin(), slot_of.end());
    const int64_t top_slot = *top_it;
    const int64_t top = top_it - slot_of.begin();
    const int64_t step = top_slot ? (offs[(size_t)top] - lo) / top_slot : numel;
    if (step < numel) return py::none();
    for (int64_t e = 0; e < n; ++e)
      if (offs[(size_t)e] - lo != slot_of[(size_t)e] * step) return py::none();
    fields.push_back(t0.as_strided({top_slot + 1, shape[0], shape[1]}, {step, stride[0], stride[1]}, lo));
  }
  return py::make_tuple(fields, slot_of);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("pool_regions", &pool_regions, "the pool check of a resident expert set (operators._pool_regions)");
}
