// Feature entry points of `_C`: the output-stationary, weight-stationary
// (fused and gather-GEMM-scatter) and hybrid dataflows, the selector's timing
// probes and the buffer / error utilities.
// Reference: torch/cuda_sparse_convolution_forward.cu:7-507,
// torch/cuda_memory_buffer.cu:7-16.
#include "host_common.h"

#include <c10/hip/HIPCachingAllocator.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <tuple>
#include <unordered_map>

namespace spira_host {

static int dtype_of(const torch::Tensor &t) {
  if (t.scalar_type() == torch::kHalf) return SPIRA_F16;
  if (t.scalar_type() == torch::kFloat) return SPIRA_F32;
  fail("Cannot find implementation for feature dtype ", t.scalar_type());
}

// Cached device tensors are allocated from the caching allocator's pool of
// the stream that made them, and go back to that pool when their entry is
// dropped.  A kernel that reads them on another stream must be recorded on
// them, or a later allocation on the making stream could reuse the memory
// while that kernel still reads it (an order overwritten under a running
// convolution indexes its output rows out of bounds).
static void record_use(hipStream_t made_on, std::initializer_list<const torch::Tensor *> ts) {
  const auto cur = c10::hip::getCurrentHIPStream();
  if (cur.stream() == made_on) return;
  for (const torch::Tensor *t : ts)
    if (t->defined()) const_cast<torch::Tensor *>(t)->record_stream(cur);
}

// Prepared (MFMA-ready) weights, cached per weight tensor.  An entry is valid
// while the same TensorImpl is alive with the same storage pointer and
// version counter, so an optimizer step or `param.data = ...` invalidates it;
// the weak reference keeps a freed tensor's address from being reused by a
// different tensor while its entry exists.
struct PreparedEntry {
  explicit PreparedEntry(const torch::Tensor &w) : impl(w.getIntrusivePtr()) {}
  c10::weak_intrusive_ptr<c10::TensorImpl> impl;
  const void *data = nullptr;
  uint32_t version = 0;
  torch::Tensor prepared;
  hipStream_t stream = nullptr;  // the stream that allocated and wrote `prepared`
};

static std::unordered_map<const c10::TensorImpl *, PreparedEntry> &prepared_cache() {
  static std::unordered_map<const c10::TensorImpl *, PreparedEntry> cache;
  return cache;
}

// Returns the prepared copy of W (or an undefined tensor when the dtype needs none).
static torch::Tensor prepared_weights(const torch::Tensor &W) {
  const int dtype = dtype_of(W);
  size_t bytes = 0;
  check_rc(spira_hip_prepared_weights_bytes(W.size(0), W.size(1), W.size(2), dtype, &bytes), "prepare_weights");
  if (bytes == 0) return torch::Tensor();
  auto &cache = prepared_cache();
  const c10::TensorImpl *key = W.unsafeGetTensorImpl();
  auto it = cache.find(key);
  if (it != cache.end()) {
    auto &e = it->second;
    if (!e.impl.expired() && e.data == W.data_ptr() && e.version == W._version() &&
        e.prepared.device() == W.device()) {
      record_use(e.stream, {&e.prepared});
      return e.prepared;
    }
    cache.erase(it);
  }
  // drop the entries of freed weight tensors (one entry per live layer)
  for (auto i = cache.begin(); i != cache.end();) i = i->second.impl.expired() ? cache.erase(i) : std::next(i);
  PreparedEntry e(W);
  e.data = W.data_ptr();
  e.version = W._version();
  e.prepared = workspace(bytes, W.device());
  e.stream = current_stream();
  check_rc(spira_hip_prepare_weights(W.data_ptr(), W.size(0), W.size(1), W.size(2), dtype, e.prepared.data_ptr(),
                                     current_stream()),
           "prepare_weights");
  auto out = e.prepared;
  cache.emplace(key, std::move(e));
  return out;
}

// pointer to weight row `k` of W, and of its prepared copy
static const void *wrow_ptr(const torch::Tensor &W, int k) {
  return static_cast<const char *>(W.data_ptr()) + static_cast<int64_t>(k) * W.size(1) * W.size(2) * W.element_size();
}
static const void *prow_ptr(const torch::Tensor &P, const torch::Tensor &W, int k) {
  if (!P.defined()) return nullptr;
  const int64_t cinp = (W.size(1) + 15) / 16 * 16, coutp = (W.size(2) + 31) / 32 * 32;
  return static_cast<const char *>(P.data_ptr()) + static_cast<int64_t>(k) * cinp * coutp * 2;
}

// Row orders of output-stationary maps, cached per map tensor like the
// prepared weights (valid while the same map tensor is alive and unchanged).
struct OrderEntry {
  explicit OrderEntry(const torch::Tensor &m) : impl(m.getIntrusivePtr()) {}
  c10::weak_intrusive_ptr<c10::TensorImpl> impl;
  const void *data = nullptr;
  uint32_t version = 0;
  int64_t T = 0;
  bool free = false;  // made with the map at no sorting cost (convert_transposed_os_ordered)
  torch::Tensor order, masks, ordered_map;
  hipStream_t stream = nullptr;  // the stream the tensors were allocated and written on
};


static std::unordered_map<const c10::TensorImpl *, OrderEntry> &order_cache() {
  static std::unordered_map<const c10::TensorImpl *, OrderEntry> cache;
  return cache;
}

// Drops the entries whose map tensor has been freed, so that their device
// tensors (order, ordered map, masks: ~7 MB for a 200k-row k = 2 inverse) go
// back to the allocator with the map instead of piling up across steps.  Run
// on every insert: the cache holds one entry per live map, a few dozen.
static void purge_expired_orders() {
  auto &cache = order_cache();
  for (auto i = cache.begin(); i != cache.end();) i = i->second.impl.expired() ? cache.erase(i) : std::next(i);
}

static bool &row_order_flag() {
  static bool on = true;
  return on;
}
static bool row_order_enabled() { return row_order_flag(); }
void set_row_order(bool on) { row_order_flag() = on; }

// Default rule for walking an output-stationary map in row order (fp16):
// maps of at least 100k targets and 27 to 57 offsets.  Below 100k targets
// the sort costs more than the few small blocks it saves; a k = 2 down /
// up-sampling map (8 offsets) serves a single layer, and its sort cost more
// than that layer saved (config-4 network: 3.28 -> 3.07 ms per step without
// the order of its two k = 2 maps); above 57 offsets the sort keys cannot
// hold the column mask, the order takes 64-bit keys and a second pass over
// the map, and for the 125-offset maps of config 5 it cost more than it saved
// (SparseResNetLarge on the 300k-voxel scene: 6.61 ms per step with it, 5.87
// ms without).  A layer's tuning may ask for it on (1) or off (0) instead.
static bool row_order_applies(int64_t T, int64_t K, int request = -1) {
  if (!row_order_enabled() || T <= 0 || K > 128) return false;
  if (request >= 0) return request == 1;
  return T >= 100000 && K >= 27 && K <= 57;
}

static const OrderEntry &row_order_of(const torch::Tensor &map, int64_t T) {
  auto &cache = order_cache();
  const c10::TensorImpl *key = map.unsafeGetTensorImpl();
  auto it = cache.find(key);
  if (it != cache.end()) {
    auto &e = it->second;
    if (!e.impl.expired() && e.data == map.data_ptr() && e.version == map._version() && e.T == T) return e;
    cache.erase(it);
  }
  purge_expired_orders();
  OrderEntry e(map);
  e.data = map.data_ptr();
  e.version = map._version();
  e.T = T;
  e.stream = current_stream();
  const int64_t K = map.size(1);
  e.order = empty_i32({std::max<int64_t>(T, 1)}, map.device());
  // 128-bit valid-column unions per 128 ordered rows (maps of <= 128 offsets)
  if (K <= 128)
    e.masks = torch::empty({(T + 127) / 128 * 2}, torch::TensorOptions(map.device()).dtype(torch::kInt64));
  e.ordered_map = empty_i32({std::max<int64_t>(T, 1), K}, map.device());
  size_t wsb = 0;
  check_rc(spira_hip_kmap_row_order_workspace(T, &wsb), "row_order");
  auto ws = workspace(wsb, map.device());
  check_rc(spira_hip_kmap_row_order(map.data_ptr<int32_t>(), T, static_cast<int>(K), e.order.data_ptr<int32_t>(),
                                    e.masks.defined() ? reinterpret_cast<uint64_t *>(e.masks.data_ptr<int64_t>()) : nullptr,
                                    e.ordered_map.data_ptr<int32_t>(), ws.data_ptr(), wsb, current_stream()),
           "row_order");
  return cache.emplace(key, std::move(e)).first->second;
}

// The order cached for `map` (same tensor, unchanged, same T), or null.
static const OrderEntry *cached_order(const torch::Tensor &map, int64_t T) {
  auto &cache = order_cache();
  auto it = cache.find(map.unsafeGetTensorImpl());
  if (it == cache.end()) return nullptr;
  const OrderEntry &e = it->second;
  if (e.impl.expired() || e.data != map.data_ptr() || e.version != map._version() || e.T != T) return nullptr;
  return &e;
}

// The inverse of a map whose entries partition its sources (a k = 2 or 1
// down-sampling map with its stride) for a transposed layer, with the
// inverse's row order made in the same pass (no sort) and cached for it:
// the fp16 kernel then walks the inverse grouped by column, one offset per
// 128-row group but at the group boundaries, instead of visiting every
// offset with one row in K valid.  No reference counterpart (a special case
// of cuda_convert_transposed_os, torch/cuda_sparse_convolution_mapping.cu:1809-1830).
torch::Tensor convert_transposed_os_ordered(const torch::Tensor &map, int64_t num_coarse, int64_t num_sources) {
  SPIRA_CHECK_ARG(map.dim() == 2 && map.scalar_type() == torch::kInt32, "out_in_map must be a 2-D int32 tensor");
  require_device(map, "out_in_map");
  SPIRA_CHECK_ARG(num_coarse >= 0 && num_coarse <= map.size(0) && num_sources >= 0, "bad map sizes");
  const int64_t K = map.size(1);
  const int64_t Sp = (num_sources + 127) / 128 * 128;
  auto inverse = empty_i32({Sp, K}, map.device());
  const int64_t ntiles = (std::max<int64_t>(num_coarse, 1) + 255) / 256;
  if (!row_order_enabled() || K > 8 || K * ntiles > 16384 || num_sources == 0) {
    // the general inverse (a -1 fill, then one scatter per entry): it does
    // not rely on the entries partitioning the sources
    check_rc(spira_hip_convert_transposed_os(map.data_ptr<int32_t>(), map.size(0), static_cast<int>(K), Sp,
                                             inverse.data_ptr<int32_t>(), current_stream()),
             "convert_transposed_os_ordered");
    return inverse;
  }
  OrderEntry e(inverse);
  e.data = inverse.data_ptr();
  e.version = inverse._version();
  e.T = num_sources;
  e.free = true;
  e.stream = current_stream();
  e.order = empty_i32({num_sources}, map.device());
  e.masks = torch::empty({(num_sources + 127) / 128 * 2}, torch::TensorOptions(map.device()).dtype(torch::kInt64));
  e.ordered_map = empty_i32({num_sources, K}, map.device());
  size_t wsb = 0;
  check_rc(spira_hip_convert_transposed_os_partition_order_workspace(num_coarse, static_cast<int>(K), &wsb),
           "convert_transposed_os_ordered");
  auto ws = workspace(wsb, map.device());
  check_rc(spira_hip_convert_transposed_os_partition_order(
               map.data_ptr<int32_t>(), num_coarse, static_cast<int>(K), num_sources, Sp, inverse.data_ptr<int32_t>(),
               e.order.data_ptr<int32_t>(), e.ordered_map.data_ptr<int32_t>(),
               reinterpret_cast<uint64_t *>(e.masks.data_ptr<int64_t>()), ws.data_ptr(), wsb, current_stream()),
           "convert_transposed_os_ordered");
  purge_expired_orders();
  auto &cache = order_cache();
  cache.erase(inverse.unsafeGetTensorImpl());
  cache.emplace(inverse.unsafeGetTensorImpl(), std::move(e));
  return inverse;
}

// Queue the row order of an output-stationary map now, on the current
// stream, if the fp16 kernel would use one for it (same rule as run_os), so
// that it is computed before the first layer needs it.  Returns its tensors
// (order, group masks, ordered map; for a caller that made them on another
// stream than the one that will read them), or nothing if the kernel uses
// no row order for this map.  No reference counterpart (the row order is
// this build's own).
std::vector<torch::Tensor> prepare_row_order(const torch::Tensor &map, int64_t T, int64_t request) {
  SPIRA_CHECK_ARG(map.dim() == 2 && map.scalar_type() == torch::kInt32, "out_in_map must be 2-D int32");
  require_device(map, "out_in_map");
  SPIRA_CHECK_ARG(map.size(0) >= T, "out_in_map has fewer rows than targets");
  const int64_t K = map.size(1);
  SPIRA_CHECK_ARG(request >= -1 && request <= 1, "row order request must be -1, 0 or 1");
  if (!row_order_applies(T, K, static_cast<int>(request))) return {};
  const OrderEntry &e = row_order_of(map, T);
  std::vector<torch::Tensor> out{e.order, e.ordered_map};
  if (e.masks.defined()) out.push_back(e.masks);
  return out;
}

// prepare_row_order for several maps at once: the maps that take a row
// order and have none cached get it from one batched chain of launches
// (spira_hip_kmap_row_order_batch: one sort over all maps' rows) when they
// have 9 to 27 offsets, else one by one.  No reference counterpart.
void prepare_row_orders(const std::vector<torch::Tensor> &maps, const std::vector<int64_t> &Ts,
                        const std::vector<int64_t> &requests) {
  SPIRA_CHECK_ARG(maps.size() == Ts.size() && maps.size() == requests.size(),
                  "maps, target counts and requests must have the same length");
  std::vector<size_t> batch;
  for (size_t i = 0; i < maps.size(); ++i) {
    const torch::Tensor &map = maps[i];
    SPIRA_CHECK_ARG(map.dim() == 2 && map.scalar_type() == torch::kInt32, "out_in_map must be 2-D int32");
    require_device(map, "out_in_map");
    SPIRA_CHECK_ARG(map.size(0) >= Ts[i], "out_in_map has fewer rows than targets");
    SPIRA_CHECK_ARG(requests[i] >= -1 && requests[i] <= 1, "row order request must be -1, 0 or 1");
    const int64_t K = map.size(1);
    if (!row_order_applies(Ts[i], K, static_cast<int>(requests[i])) || cached_order(map, Ts[i])) continue;
    bool dup = false;  // (one map listed twice)
    for (size_t j : batch) dup |= maps[j].unsafeGetTensorImpl() == map.unsafeGetTensorImpl();
    if (dup) continue;
    // (maps of at most 8 offsets take their own counting sort)
    if (K > 8 && K <= 27) batch.push_back(i);
    else row_order_of(map, Ts[i]);
  }
  for (size_t b0 = 0; b0 < batch.size(); b0 += 16) {
    const size_t nb = std::min<size_t>(16, batch.size() - b0);
    if (nb == 1) {
      row_order_of(maps[batch[b0]], Ts[batch[b0]]);
      continue;
    }
    purge_expired_orders();
    std::vector<OrderEntry> entries;
    std::vector<spira_hip_row_order_job_t> jobs;
    entries.reserve(nb);
    for (size_t q = 0; q < nb; ++q) {
      const torch::Tensor &map = maps[batch[b0 + q]];
      const int64_t T = Ts[batch[b0 + q]], K = map.size(1);
      OrderEntry e(map);
      e.data = map.data_ptr();
      e.version = map._version();
      e.T = T;
      e.stream = current_stream();
      e.order = empty_i32({T}, map.device());
      e.masks = torch::empty({(T + 127) / 128 * 2}, torch::TensorOptions(map.device()).dtype(torch::kInt64));
      e.ordered_map = empty_i32({T, K}, map.device());
      jobs.push_back(spira_hip_row_order_job_t{map.data_ptr<int32_t>(), T, static_cast<int>(K),
                                                e.order.data_ptr<int32_t>(),
                                                reinterpret_cast<uint64_t *>(e.masks.data_ptr<int64_t>()),
                                                e.ordered_map.data_ptr<int32_t>()});
      entries.push_back(std::move(e));
    }
    size_t wsb = 0;
    check_rc(spira_hip_kmap_row_order_batch_workspace(static_cast<int>(nb), jobs.data(), &wsb), "row_order_batch");
    auto ws = workspace(wsb, maps[batch[b0]].device());
    check_rc(spira_hip_kmap_row_order_batch(static_cast<int>(nb), jobs.data(), ws.data_ptr(), wsb, current_stream()),
             "row_order_batch");
    auto &cache = order_cache();
    for (size_t q = 0; q < nb; ++q) {
      const c10::TensorImpl *key = maps[batch[b0 + q]].unsafeGetTensorImpl();
      cache.erase(key);
      cache.emplace(key, std::move(entries[q]));
    }
  }
}

// The row order of an output-stationary map as the fp16 kernel uses it:
// (order, group masks as int64 [ceil(T / 128) * 2], ordered map).  No
// reference counterpart: exposed for tests.
std::tuple<torch::Tensor, torch::Tensor, torch::Tensor> kmap_row_order(const torch::Tensor &map, int64_t T) {
  require_device(map, "out_in_map");
  SPIRA_CHECK_ARG(map.dim() == 2 && map.scalar_type() == torch::kInt32 && map.size(0) >= T,
                  "out_in_map must be int32 [>= T, K]");
  const OrderEntry &e = row_order_of(map, T);
  return {e.order.narrow(0, 0, T), e.masks, e.ordered_map.narrow(0, 0, T)};
}

// (X2: the second part of a channel concatenation [X | X2], or null)
static void check_features(const torch::Tensor &X, const torch::Tensor &W, const torch::Tensor *X2 = nullptr) {
  SPIRA_CHECK_ARG(X.dim() == 2, "sources must be [N, C_in]");
  SPIRA_CHECK_ARG(W.dim() == 3, "weights must be [K, C_in, C_out]");
  require_device(X, "sources");
  require_device(W, "weights");
  SPIRA_CHECK_ARG(X.scalar_type() == W.scalar_type(), "sources and weights must share a dtype");
  int64_t c = X.size(1);
  if (X2) {
    SPIRA_CHECK_ARG(X2->dim() == 2 && X2->size(0) == X.size(0) && X2->scalar_type() == X.scalar_type(),
                    "the second source part must be [N, C2] of the sources' dtype");
    require_device(*X2, "sources2");
    c += X2->size(1);
  }
  SPIRA_CHECK_ARG(c == W.size(1), "sources have ", c, " channels, weights expect ", W.size(1));
  dtype_of(X);
}

// Output-stationary pass over weight rows W[w0 : w0+K] into `out` (mode:
// SPIRA_OUT_*).  A missing map is the identity map (a submanifold layer whose
// only dense offset is the centre: sparse_convolution.cu:1368-1380).
struct Epi {
  const float *scale = nullptr, *shift = nullptr;
  const void *residual = nullptr;
  int relu = 0;
};

// Epilogue operands from the optional tensors of the torch API
// (scale / shift fp32 [C], residual [T, C] in the feature dtype).
static Epi epi_of(const std::optional<torch::Tensor> &scale, const std::optional<torch::Tensor> &shift,
                  const std::optional<torch::Tensor> &residual, bool relu, int64_t T, int64_t C,
                  const torch::Tensor &X) {
  Epi e;
  auto vec = [&](const std::optional<torch::Tensor> &v, const char *name) -> const float * {
    if (!v.has_value() || !v->defined()) return nullptr;
    SPIRA_CHECK_ARG(v->scalar_type() == torch::kFloat && v->numel() == C && v->is_contiguous(), name,
                    " must be a contiguous fp32 vector of ", C, " channels");
    require_device(*v, name);
    return v->data_ptr<float>();
  };
  e.scale = vec(scale, "scale");
  e.shift = vec(shift, "shift");
  if (residual.has_value() && residual->defined()) {
    SPIRA_CHECK_ARG(residual->scalar_type() == X.scalar_type() && residual->dim() == 2 && residual->size(0) == T &&
                        residual->size(1) == C && residual->is_contiguous(),
                    "residual must be a contiguous [", T, ", ", C, "] tensor of the feature dtype");
    require_device(*residual, "residual");
    e.residual = residual->data_ptr();
  }
  e.relu = relu ? 1 : 0;
  return e;
}

// The output-stationary workspace holds fp32 accumulators that every call
// leaves zeroed; one zero-filled buffer per (device, stream) is kept and
// grown (calls on one stream run in order, so they share it safely).
static torch::Tensor zeroed_workspace(size_t bytes, const torch::Device &dev) {
  static std::unordered_map<uint64_t, torch::Tensor> pool;
  if (bytes == 0) return torch::Tensor();
  const hipStream_t s = current_stream();
  const uint64_t key = (reinterpret_cast<uint64_t>(s) << 8) ^ static_cast<uint64_t>(dev.index() & 0xff);
  auto &t = pool[key];
  if (!t.defined() || static_cast<size_t>(t.numel()) < bytes)
    t = torch::zeros({static_cast<int64_t>((bytes + 255) / 256 * 256)},
                     torch::TensorOptions(dev).dtype(torch::kUInt8));
  return t;
}

// A layer's output-stationary launch choices: the kernel's
// (spira_hip_os_tuning_t, 0 = automatic) and the row order (-1 automatic,
// 0 off, 1 on).  From Python: a 6-tuple (col_tile, step_channels,
// offset_splits, offset_pack, block_order, row_order), optionally followed
// by row_walk, balance_offsets and blocks_per_cu.
struct OsTune {
  spira_hip_os_tuning_t k{};
  int row_order = -1;
};
using TuneArg = std::optional<std::vector<int64_t>>;
static OsTune tune_of(const TuneArg &t) {
  OsTune r;
  if (!t.has_value()) return r;
  const auto &v = *t;
  SPIRA_CHECK_ARG(v.size() >= 6 && v.size() <= 9, "tuning must have 6 to 9 fields");
  r.k.col_tile = static_cast<int>(v[0]);
  r.k.step_channels = static_cast<int>(v[1]);
  r.k.offset_splits = static_cast<int>(v[2]);
  r.k.offset_pack = static_cast<int>(v[3]);
  r.k.block_order = static_cast<int>(v[4]);
  r.row_order = static_cast<int>(v[5]);
  r.k.row_walk = v.size() > 6 ? static_cast<int>(v[6]) : 0;
  r.k.balance_offsets = v.size() > 7 ? static_cast<int>(v[7]) : 0;
  r.k.blocks_per_cu = v.size() > 8 ? static_cast<int>(v[8]) : 0;
  SPIRA_CHECK_ARG(r.row_order >= -1 && r.row_order <= 1, "row_order must be -1, 0 or 1");
  return r;
}

static bool epi_empty(const Epi &e) { return !e.scale && !e.shift && !e.residual && !e.relu; }

static void run_os(const torch::Tensor *map, int64_t S, int64_t T, const torch::Tensor &X0, const torch::Tensor &W,
                   int w0, int K, void *out, int mode, const Epi &epi = Epi(), const torch::Tensor *X2 = nullptr,
                   const OsTune &tn = OsTune()) {
  const auto dev = X0.device();
  const int dtype = dtype_of(X0);
  // a channel concatenation [X0 | X2] is gathered from its two parts when
  // the split falls on a 16-channel slice (fp16), else materialised here
  const bool split = X2 && dtype == SPIRA_F16 && X0.size(1) % 32 == 0 && X2->size(1) % 8 == 0;
  const torch::Tensor X = (X2 && !split) ? torch::cat({X0, *X2}, 1) : X0;
  const int32_t *mp = nullptr;
  if (map) {
    SPIRA_CHECK_ARG(map->dim() == 2 && map->scalar_type() == torch::kInt32, "out_in_map must be 2-D int32");
    require_device(*map, "out_in_map");
    SPIRA_CHECK_ARG(map->size(0) >= T, "out_in_map has fewer rows than targets");
    SPIRA_CHECK_ARG(map->size(1) == K, "out_in_map has ", map->size(1), " columns, expected ", K);
    mp = map->data_ptr<int32_t>();
  } else {
    // no map: the identity map (targets[t] reads sources[t], one offset)
    SPIRA_CHECK_ARG(S == T && K == 1, "the identity map needs as many sources as targets and one offset");
  }
  // the row walk (few input channels): the map as it is and the rows unpadded
  const bool walk = tn.k.row_walk == 1 && map && dtype == SPIRA_F16 && !X2 && W.size(1) <= 16 &&
                    mode == SPIRA_OUT_STORE && K <= 128;
  auto P = prepared_weights(W);
  size_t wsb = 0;
  const int64_t cin_run =
      (!split && dtype == SPIRA_F16 && W.size(1) % 8 != 0) ? (W.size(1) + 7) / 8 * 8 : W.size(1);
  check_rc(spira_hip_conv_os_workspace(T, K, cin_run, W.size(2), dtype, mode, &tn.k, &wsb), "conv_os");
  auto ws = zeroed_workspace(wsb, dev);
  const int32_t *order = nullptr;
  const uint64_t *masks = nullptr;
  if (map && dtype == SPIRA_F16 && !walk) {
    // the library's rule (or the tuning's request) for a sorted order; an
    // order made at no cost with the map (convert_transposed_os_ordered)
    // is taken unless the tuning asks against it
    const OrderEntry *oe = nullptr;
    if (row_order_applies(T, K, tn.row_order)) oe = &row_order_of(*map, T);
    else if (tn.row_order != 0 && row_order_enabled()) {
      oe = cached_order(*map, T);
      if (oe && !oe->free) oe = nullptr;  // (a sorted order only by the rule or on request)
    }
    if (oe) {
      record_use(oe->stream, {&oe->order, &oe->masks, &oe->ordered_map});
      order = oe->order.data_ptr<int32_t>();
      masks = oe->masks.defined() ? reinterpret_cast<const uint64_t *>(oe->masks.data_ptr<int64_t>()) : nullptr;
      mp = oe->ordered_map.data_ptr<int32_t>();
    }
  }
  // fp16 rows whose width is not a multiple of 8 channels (the 3-channel
  // stem) are padded with zero channels to 16-byte rows, which the MMA
  // kernel gathers with one vector load each; the prepared weights already
  // hold zeros there (they are padded to 16 input channels)
  void *wsp = ws.defined() ? ws.data_ptr() : nullptr;
  if (split) {
    check_rc(spira_hip_conv_os_concat(T, K, mp, order, masks, X.data_ptr(), X2->data_ptr(), S, X.size(1), X2->size(1),
                                      prow_ptr(P, W, w0), W.size(2), out, mode, epi.scale, epi.shift, epi.residual,
                                      epi.relu, &tn.k, wsp, wsb, current_stream()),
             "sparse_convolution_forward_os");
    return;
  }
  const int64_t cin = walk ? W.size(1) : cin_run;
  torch::Tensor Xp = X;
  if (cin != W.size(1)) Xp = torch::constant_pad_nd(X.narrow(0, 0, S), {0, cin - W.size(1)});
  check_rc(spira_hip_conv_os(T, K, mp, order, masks, Xp.data_ptr(), S, cin, wrow_ptr(W, w0), prow_ptr(P, W, w0), W.size(2),
                             dtype, out, mode, epi.scale, epi.shift, epi.residual, epi.relu, &tn.k, wsp, wsb,
                             current_stream()),
           "sparse_convolution_forward_os");
}

// (reference: CUDASparseConvolutionForward_OS, :448-496)
// (x2: the second part of a channel-concatenated input [X | x2], or None)
torch::Tensor forward_os(int64_t S, int64_t T, const torch::Tensor &out_in_map, const torch::Tensor &X,
                         const torch::Tensor &W, const std::optional<torch::Tensor> &scale,
                         const std::optional<torch::Tensor> &shift, const std::optional<torch::Tensor> &residual,
                         bool relu, const std::optional<torch::Tensor> &x2, const TuneArg &tuning) {
  const torch::Tensor *X2 = x2.has_value() ? &*x2 : nullptr;
  check_features(X, W, X2);
  SPIRA_CHECK_ARG(out_in_map.dim() == 2, "out_in_map must be 2-D");
  SPIRA_CHECK_ARG(W.size(0) == out_in_map.size(1), "weights have ", W.size(0), " offsets, map has ",
                  out_in_map.size(1));
  auto Y = torch::empty({T, W.size(2)}, X.options());
  run_os(&out_in_map, S, T, X, W, 0, static_cast<int>(W.size(0)), Y.data_ptr(), SPIRA_OUT_STORE,
         epi_of(scale, shift, residual, relu, T, W.size(2), X), X2, tune_of(tuning));
  return Y;
}

// 1x1x1 / stride-1 layers: targets = sources @ W[0] with the fused epilogue,
// on the output-stationary kernel with the identity map (reference:
// the torch.mm path of SparseConv.forward, source/spira/nn/conv.py:310-313).
torch::Tensor forward_dense(const torch::Tensor &X, const torch::Tensor &W, const std::optional<torch::Tensor> &scale,
                            const std::optional<torch::Tensor> &shift, const std::optional<torch::Tensor> &residual,
                            bool relu, const std::optional<torch::Tensor> &x2, const TuneArg &tuning) {
  const torch::Tensor *X2 = x2.has_value() ? &*x2 : nullptr;
  check_features(X, W, X2);
  SPIRA_CHECK_ARG(W.size(0) == 1, "a dense layer has one weight offset, got ", W.size(0));
  const int64_t T = X.size(0);
  auto Y = torch::empty({T, W.size(2)}, X.options());
  run_os(nullptr, T, T, X, W, 0, 1, Y.data_ptr(), SPIRA_OUT_STORE, epi_of(scale, shift, residual, relu, T, W.size(2), X),
         X2, tune_of(tuning));
  return Y;
}

// Host sizes of the per-offset lists, the mirrored half filled in when only
// the first half was compacted (sparse_convolution.cu:1020-1037, 1150-1157).
static std::vector<int32_t> host_sizes(const torch::Tensor &nbsizes, int Km, bool half) {
  auto h = nbsizes.to(torch::kCPU).to(torch::kInt32).contiguous();
  const int32_t *p = h.data_ptr<int32_t>();
  std::vector<int32_t> s(Km, 0);
  const int nh = half ? (Km + 1) / 2 : Km;
  SPIRA_CHECK_ARG(h.numel() >= nh, "kernel_map_sizes has ", h.numel(), " entries, expected ", nh);
  for (int i = 0; i < nh; ++i) s[i] = p[i];
  for (int i = nh; i < Km; ++i) s[i] = s[Km - 1 - i];
  return s;
}

// Greedy bucketing of adjacent offsets while the padding redundancy stays
// within `threshold` (nullopt: merge all, negative: never merge), returning
// each offset's first row in the padded buffer (Km + 1 entries)
// (reference: GeneratePaddingBuckets / ComputeCumsumKernelPaddedSizes,
// cuda/functions/sparse_convolution.cu:488-515, 744-764).
static std::vector<int64_t> padded_offsets(const std::vector<int32_t> &sizes, const std::optional<double> &threshold) {
  const int K = static_cast<int>(sizes.size());
  std::vector<int> bounds{0};
  for (int i = 0; i < K; ++i) {
    const int j = i;
    uint64_t actual = sizes[i], summit = sizes[i];
    while (i + 1 < K) {
      actual += sizes[i + 1];
      summit = std::max<uint64_t>(summit, sizes[i + 1]);
      const uint64_t padded = summit * static_cast<uint64_t>((i + 1) - j + 1);
      const double red = static_cast<double>(padded - actual) / static_cast<double>(actual);
      if (threshold.has_value() && (*threshold < 0 || red > *threshold)) break;
      ++i;
    }
    bounds.push_back(i + 1);
  }
  std::vector<int64_t> off(K + 1, 0);
  for (size_t b = 0; b + 1 < bounds.size(); ++b) {
    int64_t summit = 0;
    for (int k = bounds[b]; k < bounds[b + 1]; ++k) summit = std::max<int64_t>(summit, sizes[k]);
    for (int k = bounds[b]; k < bounds[b + 1]; ++k) off[k + 1] = off[k] + summit;
  }
  return off;
}

// A planned gather -> GEMM -> scatter over Km offsets.
struct GsPlan {
  int Km = 0;
  int64_t S = 0, T = 0;
  std::vector<int32_t> sizes;
  std::vector<int64_t> off;
  const int32_t *smask = nullptr, *tmask = nullptr;
  torch::Tensor bin, bout;
};

static GsPlan plan_gs(int64_t S, int64_t T, const torch::Tensor &source_masks, const torch::Tensor &target_masks,
                      const torch::Tensor &nbsizes, bool half, const std::optional<double> &threshold, int cin,
                      int cout, const torch::TensorOptions &fopt) {
  SPIRA_CHECK_ARG(source_masks.dim() == 2 && target_masks.dim() == 2, "masks must be 2-D");
  SPIRA_CHECK_ARG(source_masks.scalar_type() == torch::kInt32 && target_masks.scalar_type() == torch::kInt32,
                  "masks must be int32");
  require_device(source_masks, "source_masks");
  require_device(target_masks, "target_masks");
  SPIRA_CHECK_ARG(source_masks.size(0) == target_masks.size(0), "source and target masks disagree on offsets");
  SPIRA_CHECK_ARG(source_masks.size(1) == S && target_masks.size(1) == T, "masks do not match S / T");
  GsPlan p;
  p.Km = static_cast<int>(target_masks.size(0));
  p.S = S;
  p.T = T;
  p.sizes = host_sizes(nbsizes, p.Km, half);
  p.off = padded_offsets(p.sizes, threshold);
  p.smask = source_masks.data_ptr<int32_t>();
  p.tmask = target_masks.data_ptr<int32_t>();
  const int64_t total = std::max<int64_t>(p.off[p.Km], 1);
  p.bin = torch::empty({total, cin}, fopt);
  p.bout = torch::empty({total, cout}, fopt.dtype(torch::kFloat));
  return p;
}

static void gs_gather(GsPlan &p, const torch::Tensor &X, hipStream_t s) {
  check_rc(spira_hip_ws_gather(p.S, X.size(1), p.Km, dtype_of(X), X.data_ptr(), p.smask, p.off.data(),
                               p.bin.data_ptr(), s),
           "gather");
}

static void gs_gemm(GsPlan &p, const torch::Tensor &W, int woff, hipStream_t s) {
  const int dtype = dtype_of(W);
  auto P = prepared_weights(W);
  check_rc(spira_hip_ws_gemm(p.Km, p.sizes.data(), p.off.data(), W.size(1), W.size(2), dtype, p.bin.data_ptr(),
                             wrow_ptr(W, woff), prow_ptr(P, W, woff), p.bout.data_ptr<float>(), s),
           "gemm");
}

static void gs_scatter(GsPlan &p, int cout, int dtype, const float *base, void *Y, hipStream_t s,
                       const Epi &e = Epi()) {
  check_rc(spira_hip_ws_scatter(p.T, cout, p.Km, dtype, p.tmask, p.off.data(), p.bout.data_ptr<float>(), base,
                                e.scale, e.shift, e.residual, e.relu, Y, s),
           "scatter");
}

// (reference: CUDASparseConvolutionForward_WS, :130-184)
torch::Tensor forward_ws(int64_t S, int64_t T, int64_t gather_tile, int64_t scatter_tile, int64_t parallel,
                         const std::optional<double> &threshold, const torch::Tensor &X, const torch::Tensor &W,
                         const torch::Tensor &source_masks, const torch::Tensor &target_masks,
                         const torch::Tensor &nbsizes, const std::optional<torch::Tensor> &scale,
                         const std::optional<torch::Tensor> &shift, const std::optional<torch::Tensor> &residual,
                         bool relu) {
  (void)gather_tile;
  (void)scatter_tile;
  (void)parallel;
  check_features(X, W);
  SPIRA_CHECK_ARG(W.size(0) == target_masks.size(0), "weights have ", W.size(0), " offsets, masks have ",
                  target_masks.size(0));
  const int Km = static_cast<int>(target_masks.size(0));
  const bool half = (Km % 2 == 1) && S == T;
  auto p = plan_gs(S, T, source_masks, target_masks, nbsizes, half, threshold, W.size(1), W.size(2), X.options());
  auto Y = torch::empty({T, W.size(2)}, X.options());
  auto s = current_stream();
  gs_gather(p, X, s);
  gs_gemm(p, W, 0, s);
  gs_scatter(p, W.size(2), dtype_of(X), nullptr, Y.data_ptr(), s, epi_of(scale, shift, residual, relu, T, W.size(2), X));
  return Y;
}

// fused pass + fp32 -> storage dtype
static void ws_fused_into(int64_t S, int64_t T, const torch::Tensor &X, const torch::Tensor &W,
                          const torch::Tensor &naddrs, const torch::Tensor &qnaddrs, const torch::Tensor &nbmaps,
                          int64_t mapsize, int64_t qmapsize, bool transpose, int woff, int mirror_rows,
                          float *acc) {
  SPIRA_CHECK_ARG(nbmaps.dim() == 2 && nbmaps.size(0) == 2, "nbmaps must be [2, P]");
  SPIRA_CHECK_ARG(nbmaps.size(1) == mapsize, "nbmaps holds ", nbmaps.size(1), " pairs, mapsize is ", mapsize);
  require_device(nbmaps, "nbmaps");
  require_device(naddrs, "naddrs");
  require_device(qnaddrs, "qnaddrs");
  const int rows = static_cast<int>(naddrs.size(0) - 1);
  const int32_t *base = nbmaps.data_ptr<int32_t>();
  const int32_t *imap = transpose ? base + mapsize : base;
  const int32_t *omap = transpose ? base : base + mapsize;
  const int dtype = dtype_of(X);
  auto P = prepared_weights(W);
  check_rc(spira_hip_conv_ws_fused(S, T, imap, omap, rows, naddrs.data_ptr<int32_t>(), qnaddrs.data_ptr<int32_t>(),
                                   mapsize, qmapsize, woff, mirror_rows, X.data_ptr(), W.size(1), W.data_ptr(),
                                   P.defined() ? P.data_ptr() : nullptr, W.size(0), W.size(2), dtype, acc,
                                   current_stream()),
           "sparse_convolution_forward_ws_merged");
}

static torch::Tensor finish_acc(const torch::Tensor &acc, const torch::Tensor &X, const Epi &e = Epi()) {
  if (X.scalar_type() == torch::kFloat && epi_empty(e)) return acc;
  auto Y = torch::empty(acc.sizes(), X.options());
  check_rc(spira_hip_finalize(acc.data_ptr<float>(), acc.size(0), acc.size(1), dtype_of(X), e.scale, e.shift,
                              e.residual, e.relu, Y.data_ptr(), current_stream()),
           "finalize");
  return Y;
}

// (reference: CUDASparseConvolutionForward_WS_Merged, :186-250)
torch::Tensor forward_ws_merged(int64_t S, int64_t T, const torch::Tensor &X, const torch::Tensor &W,
                                const torch::Tensor &naddrs, const torch::Tensor &qnaddrs, const torch::Tensor &nbmaps,
                                int64_t mapsize, int64_t qmapsize, bool transpose,
                                const std::optional<torch::Tensor> &scale, const std::optional<torch::Tensor> &shift,
                                const std::optional<torch::Tensor> &residual, bool relu) {
  check_features(X, W);
  const int K = static_cast<int>(W.size(0));
  // mirrored pass for submanifold maps with an odd kernel volume
  // (sparse_convolution.cu:1287-1293)
  const int mirror = (S == T && K % 2 == 1) ? K : 0;
  auto acc = torch::zeros({T, W.size(2)}, X.options().dtype(torch::kFloat));
  ws_fused_into(S, T, X, W, naddrs, qnaddrs, nbmaps, mapsize, qmapsize, transpose, 0, mirror, acc.data_ptr<float>());
  return finish_acc(acc, X, epi_of(scale, shift, residual, relu, T, W.size(2), X));
}

// (reference: CUDASparseConvolutionForward_HS, :254-342)
torch::Tensor forward_hs(int64_t S, int64_t T, int64_t gather_tile, int64_t scatter_tile, int64_t parallel,
                         const std::optional<double> &threshold, const torch::Tensor &X, const torch::Tensor &W,
                         const torch::Tensor &source_masks, const torch::Tensor &target_masks,
                         const torch::Tensor &nbsizes, const std::optional<torch::Tensor> &out_in_map,
                         const std::optional<torch::Tensor> &scale, const std::optional<torch::Tensor> &shift,
                         const std::optional<torch::Tensor> &residual, bool relu) {
  (void)gather_tile;
  (void)scatter_tile;
  (void)parallel;
  check_features(X, W);
  const int Kws = static_cast<int>(target_masks.size(0));
  const int Kos = out_in_map.has_value() ? static_cast<int>(out_in_map->size(1)) : 1;
  SPIRA_CHECK_ARG(W.size(0) == Kws + Kos, "weights have ", W.size(0), " offsets, expected ", Kws + Kos);
  auto acc = torch::empty({T, W.size(2)}, X.options().dtype(torch::kFloat));
  run_os(out_in_map.has_value() ? &*out_in_map : nullptr, S, T, X, W, 0, Kos, acc.data_ptr<float>(),
         SPIRA_OUT_STORE_F32);
  auto p = plan_gs(S, T, source_masks, target_masks, nbsizes, true, threshold, W.size(1), W.size(2), X.options());
  auto Y = torch::empty({T, W.size(2)}, X.options());
  auto s = current_stream();
  gs_gather(p, X, s);
  gs_gemm(p, W, Kos, s);
  gs_scatter(p, W.size(2), dtype_of(X), acc.data_ptr<float>(), Y.data_ptr(), s,
             epi_of(scale, shift, residual, relu, T, W.size(2), X));
  return Y;
}

// (reference: CUDASparseConvolutionForward_HS_Merged, :346-443)
torch::Tensor forward_hs_merged(int64_t S, int64_t T, const torch::Tensor &X, const torch::Tensor &W,
                                const torch::Tensor &naddrs, const torch::Tensor &qnaddrs, const torch::Tensor &nbmaps,
                                const std::optional<torch::Tensor> &out_in_map, int64_t mapsize, int64_t qmapsize,
                                bool transpose, const std::optional<torch::Tensor> &scale,
                                const std::optional<torch::Tensor> &shift,
                                const std::optional<torch::Tensor> &residual, bool relu) {
  check_features(X, W);
  const int Kws = static_cast<int>((naddrs.size(0) - 1) * 2);
  const int Kos = out_in_map.has_value() ? static_cast<int>(out_in_map->size(1)) : 1;
  SPIRA_CHECK_ARG(W.size(0) == Kws + Kos, "weights have ", W.size(0), " offsets, expected ", Kws + Kos);
  auto acc = torch::empty({T, W.size(2)}, X.options().dtype(torch::kFloat));
  run_os(out_in_map.has_value() ? &*out_in_map : nullptr, S, T, X, W, 0, Kos, acc.data_ptr<float>(),
         SPIRA_OUT_STORE_F32);
  ws_fused_into(S, T, X, W, naddrs, qnaddrs, nbmaps, mapsize, qmapsize, transpose, Kos, Kws, acc.data_ptr<float>());
  return finish_acc(acc, X, epi_of(scale, shift, residual, relu, T, W.size(2), X));
}

// ---- selector probes: time one phase of the gather-GEMM-scatter path ----

enum class Phase { kGather, kGemm, kScatter };

static float time_phase(Phase ph, const std::optional<double> &threshold, bool is_hybrid, const torch::Tensor &W,
                        const torch::Tensor &source_masks, const torch::Tensor &target_masks,
                        const torch::Tensor &nbsizes) {
  SPIRA_CHECK_ARG(W.dim() == 3, "weights must be [K, C_in, C_out]");
  require_device(W, "weights");
  const int64_t S = source_masks.size(1), T = target_masks.size(1);
  const int Km = static_cast<int>(target_masks.size(0));
  const bool half = is_hybrid || (Km % 2 == 1 && S == T);
  auto p = plan_gs(S, T, source_masks, target_masks, nbsizes, half, threshold, W.size(1), W.size(2), W.options());
  auto X = torch::zeros({S, W.size(1)}, W.options());
  auto Y = torch::empty({T, W.size(2)}, W.options());
  auto s = current_stream();
  // the weights probed are the last Km offsets (the WS part of a hybrid map)
  const int woff = static_cast<int>(W.size(0)) - Km;
  SPIRA_CHECK_ARG(woff >= 0, "weights have fewer offsets than the masks");
  hipEvent_t a, b;
  SPIRA_CHECK_ARG(hipEventCreate(&a) == hipSuccess && hipEventCreate(&b) == hipSuccess, "event creation failed");
  if (ph != Phase::kGather) gs_gather(p, X, s);
  if (ph == Phase::kScatter) gs_gemm(p, W, woff, s);
  SPIRA_CHECK_ARG(hipEventRecord(a, s) == hipSuccess, "event record failed");
  if (ph == Phase::kGather) gs_gather(p, X, s);
  else if (ph == Phase::kGemm) gs_gemm(p, W, woff, s);
  else gs_scatter(p, W.size(2), dtype_of(W), nullptr, Y.data_ptr(), s);
  SPIRA_CHECK_ARG(hipEventRecord(b, s) == hipSuccess, "event record failed");
  SPIRA_CHECK_ARG(hipEventSynchronize(b) == hipSuccess, "event synchronisation failed");
  float ms = 0.f;
  (void)hipEventElapsedTime(&ms, a, b);
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  return ms;
}

// (reference: CUDATimeGEMM / CUDATimeGather / CUDATimeScatter, :7-128)
float time_gemm(int64_t parallel, const std::optional<double> &threshold, bool is_hybrid, const torch::Tensor &W,
                const torch::Tensor &sm, const torch::Tensor &tm, const torch::Tensor &nb) {
  (void)parallel;
  return time_phase(Phase::kGemm, threshold, is_hybrid, W, sm, tm, nb);
}
float time_gather(int64_t tile, const std::optional<double> &threshold, bool is_hybrid, const torch::Tensor &W,
                  const torch::Tensor &sm, const torch::Tensor &tm, const torch::Tensor &nb) {
  (void)tile;
  return time_phase(Phase::kGather, threshold, is_hybrid, W, sm, tm, nb);
}
float time_scatter(int64_t tile, const std::optional<double> &threshold, bool is_hybrid, const torch::Tensor &W,
                   const torch::Tensor &sm, const torch::Tensor &tm, const torch::Tensor &nb) {
  (void)tile;
  return time_phase(Phase::kScatter, threshold, is_hybrid, W, sm, tm, nb);
}

// Kernel-only timing of the output-stationary layer: `reps` back-to-back
// launches on the current stream between two HIP events, after the row
// order (cached per map) and the prepared weights exist; returns ms per
// launch.  No reference counterpart: a measurement probe for the roofline
// report (the reference times its layers from Python,
// scripts/layerwise_experiment.py:100-186).
float time_conv_os(int64_t S, int64_t T, const std::optional<torch::Tensor> &out_in_map, const torch::Tensor &X,
                   const torch::Tensor &W, int64_t reps, const std::optional<torch::Tensor> &x2,
                   const TuneArg &tuning) {
  const torch::Tensor *X2 = x2.has_value() ? &*x2 : nullptr;
  check_features(X, W, X2);
  SPIRA_CHECK_ARG(reps >= 1, "reps must be positive");
  auto Y = torch::empty({T, W.size(2)}, X.options());
  const int K = static_cast<int>(W.size(0));
  const torch::Tensor *map = out_in_map.has_value() ? &*out_in_map : nullptr;
  const OsTune tn = tune_of(tuning);
  run_os(map, S, T, X, W, 0, K, Y.data_ptr(), SPIRA_OUT_STORE, Epi(), X2, tn);  // warm: order, weights
  auto s = current_stream();
  hipEvent_t a, b;
  SPIRA_CHECK_ARG(hipEventCreate(&a) == hipSuccess && hipEventCreate(&b) == hipSuccess, "event creation failed");
  SPIRA_CHECK_ARG(hipEventRecord(a, s) == hipSuccess, "event record failed");
  for (int64_t i = 0; i < reps; ++i) run_os(map, S, T, X, W, 0, K, Y.data_ptr(), SPIRA_OUT_STORE, Epi(), X2, tn);
  SPIRA_CHECK_ARG(hipEventRecord(b, s) == hipSuccess, "event record failed");
  SPIRA_CHECK_ARG(hipEventSynchronize(b) == hipSuccess, "event synchronisation failed");
  float ms = 0.f;
  (void)hipEventElapsedTime(&ms, a, b);
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  return ms / static_cast<float>(reps);
}

// The launch the output-stationary kernel would make (spira_hip_conv_os_plan):
// (col_tile, step_channels, offset_splits, offsets_per_step, grid_x, grid_y,
// block_order).
// No reference counterpart: it shows what a layer's tuning changes.
std::vector<int64_t> conv_os_plan(int64_t T, int64_t K, int64_t cin, int64_t cin2, int64_t cout, bool has_map,
                                  const TuneArg &tuning) {
  const OsTune tn = tune_of(tuning);
  int32_t plan[7] = {};
  check_rc(spira_hip_conv_os_plan(T, static_cast<int>(K), static_cast<int>(cin), static_cast<int>(cin2),
                                  static_cast<int>(cout), has_map ? 1 : 0, SPIRA_OUT_STORE, &tn.k, plan),
           "conv_os_plan");
  return std::vector<int64_t>(plan, plan + 7);
}

// (reference: cuda_free_buffers / cuda_reset_error, torch/cuda_memory_buffer.cu:7-16)
void free_buffers() { c10::hip::HIPCachingAllocator::emptyCache(); }
void reset_error() { (void)hipGetLastError(); }

void register_conv(pybind11::module_ &m) {
  // The reference binds these without defaults (cuda_sparse_convolution_forward.cu:130-448) and its
  // callers pass exactly the reference arguments (nn/functional/convolution.py:78-172); the fused
  // epilogue and the launch tuning of this build are trailing keyword arguments with neutral defaults,
  // so a call at the reference's arity runs the plain convolution.
  namespace py = pybind11;
  const auto epi_args = [](auto... head) {
    return std::make_tuple(head..., py::arg("scale") = py::none(), py::arg("shift") = py::none(),
                           py::arg("residual") = py::none(), py::arg("relu") = false);
  };
  const auto def_with = [&](const char *name, auto fn, auto args, auto... extra) {
    std::apply([&](auto... a) { m.def(name, fn, a..., extra...); }, args);
  };
  def_with("cuda_sparse_convolution_forward_os", &forward_os,
           epi_args(py::arg("S"), py::arg("T"), py::arg("out_in_map"), py::arg("X"), py::arg("W")),
           py::arg("x2") = py::none(), py::arg("tuning") = py::none());
  def_with("cuda_dense_forward", &forward_dense, epi_args(py::arg("X"), py::arg("W")), py::arg("x2") = py::none(),
           py::arg("tuning") = py::none());
  m.def("time_conv_os", &time_conv_os, pybind11::arg("S"), pybind11::arg("T"), pybind11::arg("out_in_map"),
        pybind11::arg("X"), pybind11::arg("W"), pybind11::arg("reps"), pybind11::arg("x2") = pybind11::none(),
        pybind11::arg("tuning") = pybind11::none());
  def_with("cuda_sparse_convolution_forward_ws", &forward_ws,
           epi_args(py::arg("S"), py::arg("T"), py::arg("gather_tile"), py::arg("scatter_tile"), py::arg("parallel"),
                    py::arg("threshold"), py::arg("X"), py::arg("W"), py::arg("source_masks"),
                    py::arg("target_masks"), py::arg("nbsizes")));
  def_with("cuda_sparse_convolution_forward_ws_merged", &forward_ws_merged,
           epi_args(py::arg("S"), py::arg("T"), py::arg("X"), py::arg("W"), py::arg("naddrs"), py::arg("qnaddrs"),
                    py::arg("nbmaps"), py::arg("mapsize"), py::arg("qmapsize"), py::arg("transpose")));
  def_with("cuda_sparse_convolution_forward_hs", &forward_hs,
           epi_args(py::arg("S"), py::arg("T"), py::arg("gather_tile"), py::arg("scatter_tile"), py::arg("parallel"),
                    py::arg("threshold"), py::arg("X"), py::arg("W"), py::arg("source_masks"),
                    py::arg("target_masks"), py::arg("nbsizes"), py::arg("out_in_map")));
  def_with("cuda_sparse_convolution_forward_hs_merged", &forward_hs_merged,
           epi_args(py::arg("S"), py::arg("T"), py::arg("X"), py::arg("W"), py::arg("naddrs"), py::arg("qnaddrs"),
                    py::arg("nbmaps"), py::arg("out_in_map"), py::arg("mapsize"), py::arg("qmapsize"),
                    py::arg("transpose")));
  m.def("cuda_time_gemm", &time_gemm);
  m.def("cuda_time_gather", &time_gather);
  m.def("cuda_time_scatter", &time_scatter);
  m.def("cuda_free_buffers", &free_buffers);
  m.def("cuda_reset_error", &reset_error);
  m.def("set_os_row_order", &set_row_order);
  m.def("kmap_row_order", &kmap_row_order);
  // an order made with the map (no sort), as a partition inverse carries one
  // number of cached row orders (for tests: entries of freed maps are dropped)
  m.def("row_order_cache_size", [] { return static_cast<int64_t>(order_cache().size()); });
  m.def("has_free_row_order", [](const torch::Tensor &map, int64_t T) {
    const OrderEntry *e = cached_order(map, T);
    return e != nullptr && e->free;
  });
  m.def("convert_transposed_os_ordered", &convert_transposed_os_ordered, pybind11::arg("out_in_map"),
        pybind11::arg("num_coarse"), pybind11::arg("num_sources"));
  m.def("conv_os_plan", &conv_os_plan, pybind11::arg("T"), pybind11::arg("K"), pybind11::arg("cin"),
        pybind11::arg("cin2"), pybind11::arg("cout"), pybind11::arg("has_map"),
        pybind11::arg("tuning") = pybind11::none());
  m.def("prepare_row_order", &prepare_row_order, pybind11::arg("map"), pybind11::arg("T"),
        pybind11::arg("request") = -1);
  m.def("prepare_row_orders", &prepare_row_orders, pybind11::arg("maps"), pybind11::arg("T"),
        pybind11::arg("requests"));
}

}  // namespace spira_host
