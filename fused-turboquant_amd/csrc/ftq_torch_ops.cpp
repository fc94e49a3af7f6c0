// PyTorch operator library over the C ABI (include/fused_tq.h): the
// torch.ops.fused_tq.* operators the Python package calls.  Each operator
// checks its tensors with TORCH_CHECK (RuntimeError), takes the current HIP
// stream of the tensors' device, and calls the C entry point; the kernels
// are the ones libfused_tq.so holds.  Schemas mark the tensors an operator
// writes in place (Tensor(a!)); shape-only fake implementations for tracing
// are registered from Python (fused_turboquant/_ops.py).
#include <torch/library.h>
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include "fused_tq.h"

namespace {

// a rejected argument raises ValueError (as the Python API does), a HIP
// error RuntimeError
void check_rc(int rc) {
  TORCH_CHECK_VALUE(rc != FTQ_ERR_ARG, "fused_tq: ", ftq_last_error());
  TORCH_CHECK(rc == FTQ_OK, "fused_tq: ", ftq_last_error());
}

int dt(const at::Tensor& t) {
  switch (t.scalar_type()) {
    case at::kFloat: return FTQ_F32;
    case at::kHalf: return FTQ_F16;
    case at::kBFloat16: return FTQ_BF16;
    default: TORCH_CHECK(false, "fused_tq: expected float32, float16 or bfloat16, got ", t.scalar_type());
  }
  return FTQ_F32;
}

int dt_of(c10::ScalarType s) {
  switch (s) {
    case at::kFloat: return FTQ_F32;
    case at::kHalf: return FTQ_F16;
    case at::kBFloat16: return FTQ_BF16;
    default: TORCH_CHECK(false, "fused_tq: output dtype must be float32, float16 or bfloat16");
  }
  return FTQ_F32;
}

void on_device(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda(), "fused_tq: ", name, " must be on a ROCm device");
}

void contig(const at::Tensor& t, const char* name) {
  on_device(t, name);
  TORCH_CHECK(t.is_contiguous(), "fused_tq: ", name, " must be contiguous");
}

void* stream_of(const at::Tensor& t) {
  return (void*)c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

// ---- library-format codec ----------------------------------------------

std::tuple<at::Tensor, at::Tensor> encode(const at::Tensor& x, const at::Tensor& signs, const at::Tensor& boundaries,
                                          int64_t bits, int64_t codebook_class) {
  contig(x, "x");
  contig(signs, "signs");
  contig(boundaries, "boundaries");
  const c10::DeviceGuard g(x.device());
  const int64_t d = x.size(-1);
  const int64_t n = d > 0 ? x.numel() / d : 0;
  auto sizes = x.sizes().vec();
  sizes.back() = d * bits / 8;
  at::Tensor packed = at::empty(sizes, x.options().dtype(at::kByte));
  sizes.pop_back();
  at::Tensor norms = at::empty(sizes, x.options().dtype(at::kHalf));
  check_rc(ftq_encode_cb(x.data_ptr(), dt(x), n, (int)d, signs.data_ptr<float>(), boundaries.data_ptr<float>(),
                         (int)bits, (int)codebook_class, packed.data_ptr<uint8_t>(),
                         reinterpret_cast<uint16_t*>(norms.data_ptr()), stream_of(x)));
  return {packed, norms};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> encode_kv(const at::Tensor& k, const at::Tensor& v,
                                                                     const at::Tensor& signs,
                                                                     const at::Tensor& boundaries, int64_t bits,
                                                                     int64_t codebook_class) {
  contig(k, "k");
  contig(v, "v");
  contig(signs, "signs");
  contig(boundaries, "boundaries");
  TORCH_CHECK(k.sizes() == v.sizes() && k.scalar_type() == v.scalar_type() && k.device() == v.device(),
              "fused_tq: k and v must agree in shape, dtype and device");
  const c10::DeviceGuard g(k.device());
  const int64_t d = k.size(-1);
  const int64_t n = d > 0 ? k.numel() / d : 0;
  auto sizes = k.sizes().vec();
  sizes.back() = d * bits / 8;
  at::Tensor kp = at::empty(sizes, k.options().dtype(at::kByte));
  at::Tensor vp = at::empty(sizes, k.options().dtype(at::kByte));
  sizes.pop_back();
  at::Tensor kn = at::empty(sizes, k.options().dtype(at::kHalf));
  at::Tensor vn = at::empty(sizes, k.options().dtype(at::kHalf));
  check_rc(ftq_encode_kv(k.data_ptr(), v.data_ptr(), dt(k), n, (int)d, signs.data_ptr<float>(),
                         boundaries.data_ptr<float>(), (int)bits, (int)codebook_class, kp.data_ptr<uint8_t>(),
                         reinterpret_cast<uint16_t*>(kn.data_ptr()), vp.data_ptr<uint8_t>(),
                         reinterpret_cast<uint16_t*>(vn.data_ptr()), stream_of(k)));
  return {kp, kn, vp, vn};
}

at::Tensor decode(const at::Tensor& packed, const at::Tensor& norms, const at::Tensor& levels, const at::Tensor& signs,
                  int64_t bits, int64_t d, c10::ScalarType out_dtype) {
  contig(packed, "packed");
  contig(norms, "norms");
  contig(levels, "levels");
  contig(signs, "signs");
  TORCH_CHECK(packed.scalar_type() == at::kByte && norms.scalar_type() == at::kHalf,
              "fused_tq: packed must be uint8 and norms float16");
  const c10::DeviceGuard g(packed.device());
  const int64_t n = norms.numel();
  auto sizes = norms.sizes().vec();
  sizes.push_back(d);
  at::Tensor out = at::empty(sizes, packed.options().dtype(out_dtype));
  check_rc(ftq_decode(packed.data_ptr<uint8_t>(), reinterpret_cast<const uint16_t*>(norms.data_ptr()), n, (int)d,
                      levels.data_ptr<float>(), signs.data_ptr<float>(), (int)bits, out.data_ptr(), dt_of(out_dtype),
                      stream_of(packed)));
  return out;
}

at::Tensor rht(const at::Tensor& x, const at::Tensor& signs, bool inverse, c10::ScalarType out_dtype) {
  contig(x, "x");
  contig(signs, "signs");
  const c10::DeviceGuard g(x.device());
  const int64_t d = x.size(-1);
  at::Tensor out = at::empty(x.sizes(), x.options().dtype(out_dtype));
  check_rc(ftq_rht(x.data_ptr(), dt(x), d > 0 ? x.numel() / d : 0, (int)d, signs.data_ptr<float>(), inverse ? 1 : 0,
                   out.data_ptr(), dt_of(out_dtype), stream_of(x)));
  return out;
}

// ---- paged library-format cache -----------------------------------------

void paged_store(const at::Tensor& key, const at::Tensor& value, at::Tensor& kv_cache, const at::Tensor& slot_mapping,
                 const at::Tensor& k_signs, const at::Tensor& v_signs, const at::Tensor& k_boundaries,
                 const at::Tensor& v_boundaries, int64_t bits_k, int64_t bits_v, int64_t page_size) {
  contig(key, "key");
  contig(value, "value");
  contig(kv_cache, "kv_cache");
  contig(slot_mapping, "slot_mapping");
  TORCH_CHECK(key.dim() == 3 && value.sizes() == key.sizes(), "fused_tq: key/value must be [n, Hkv, d]");
  TORCH_CHECK(key.scalar_type() == value.scalar_type(), "fused_tq: key and value dtypes differ");
  TORCH_CHECK(slot_mapping.scalar_type() == at::kLong, "fused_tq: slot_mapping must be int64");
  const c10::DeviceGuard g(key.device());
  check_rc(ftq_paged_store(key.data_ptr(), value.data_ptr(), dt(key), key.size(0), (int)key.size(1), (int)key.size(2),
                           k_signs.data_ptr<float>(), v_signs.data_ptr<float>(), k_boundaries.data_ptr<float>(),
                           v_boundaries.data_ptr<float>(), (int)bits_k, (int)bits_v, slot_mapping.data_ptr<int64_t>(),
                           kv_cache.data_ptr<uint8_t>(), (int)page_size, kv_cache.size(0), stream_of(key)));
}

void paged_decode_attention(const at::Tensor& query, const at::Tensor& kv_cache, const at::Tensor& block_table,
                            const at::Tensor& seq_lens, const at::Tensor& k_signs, const at::Tensor& v_signs,
                            const at::Tensor& k_levels, const at::Tensor& v_levels, int64_t bits_k, int64_t bits_v,
                            int64_t page_size, double scale, int64_t num_splits, at::Tensor& workspace,
                            at::Tensor& out, bool fp32_operands) {
  contig(query, "query");
  contig(kv_cache, "kv_cache");
  contig(block_table, "block_table");
  contig(seq_lens, "seq_lens");
  contig(workspace, "workspace");
  contig(out, "out");
  TORCH_CHECK(query.dim() == 3 && out.sizes() == query.sizes(), "fused_tq: query and out must be [B, Hq, d]");
  TORCH_CHECK(block_table.scalar_type() == at::kInt && seq_lens.scalar_type() == at::kInt,
              "fused_tq: block_table and seq_lens must be int32");
  const c10::DeviceGuard g(query.device());
  auto fn = fp32_operands ? ftq_paged_decode_attention_valu : ftq_paged_decode_attention;
  check_rc(fn(query.data_ptr(), dt(query), kv_cache.data_ptr<uint8_t>(), block_table.data_ptr<int32_t>(),
              seq_lens.data_ptr<int32_t>(), (int)query.size(0), (int)query.size(1), (int)kv_cache.size(1),
              (int)query.size(2), (int)page_size, (int)block_table.size(1), kv_cache.size(0),
              k_signs.data_ptr<float>(), v_signs.data_ptr<float>(), k_levels.data_ptr<float>(),
              v_levels.data_ptr<float>(), (int)bits_k, (int)bits_v, (float)scale, (int)num_splits,
              workspace.data_ptr(), workspace.numel() * workspace.element_size(), out.data_ptr(), dt(out),
              stream_of(query)));
}

// ---- vLLM v1 slot cache -------------------------------------------------

void v1_store(const at::Tensor& key, const at::Tensor& value, at::Tensor& kv_cache, const at::Tensor& slot_mapping,
              const at::Tensor& midpoints, int64_t key_bits, int64_t value_bits, int64_t v_flags,
              const std::optional<at::Tensor>& rotation, const std::optional<at::Tensor>& coeffs) {
  contig(key, "key");
  contig(value, "value");
  on_device(kv_cache, "kv_cache");
  contig(slot_mapping, "slot_mapping");
  contig(midpoints, "midpoints");
  TORCH_CHECK(key.dim() == 3 && value.sizes() == key.sizes(), "fused_tq: key/value must be [n, Hkv, d]");
  TORCH_CHECK(kv_cache.dim() == 4 && kv_cache.scalar_type() == at::kByte && kv_cache.stride(3) == 1,
              "fused_tq: kv_cache must be uint8 [num_blocks, block_size, Hkv, slot] with contiguous slots");
  TORCH_CHECK(slot_mapping.scalar_type() == at::kLong, "fused_tq: slot_mapping must be int64");
  const c10::DeviceGuard g(key.device());
  const int d = (int)key.size(2);
  if (coeffs.has_value()) {
    contig(*coeffs, "coeffs");
    check_rc(ftq_v1_store_blockdiag(key.data_ptr(), value.data_ptr(), dt(key), key.size(0), (int)key.size(1), d,
                                    midpoints.data_ptr<float>(), (int)key_bits, (int)value_bits, (int)v_flags,
                                    slot_mapping.data_ptr<int64_t>(), kv_cache.data_ptr<uint8_t>(), kv_cache.size(0),
                                    (int)kv_cache.size(1), kv_cache.stride(0), kv_cache.stride(1), kv_cache.stride(2),
                                    coeffs->data_ptr<float>(), (int)coeffs->size(0), stream_of(key)));
  } else {
    if (rotation.has_value()) contig(*rotation, "rotation");
    check_rc(ftq_v1_store_rot(key.data_ptr(), value.data_ptr(), dt(key), key.size(0), (int)key.size(1), d,
                              midpoints.data_ptr<float>(), (int)key_bits, (int)value_bits, (int)v_flags,
                              slot_mapping.data_ptr<int64_t>(), kv_cache.data_ptr<uint8_t>(), kv_cache.size(0),
                              (int)kv_cache.size(1), kv_cache.stride(0), kv_cache.stride(1), kv_cache.stride(2),
                              rotation.has_value() ? rotation->data_ptr<float>() : nullptr, stream_of(key)));
  }
}

void v1_decode_attention(const at::Tensor& query, const at::Tensor& kv_cache, const at::Tensor& block_table,
                         const at::Tensor& seq_lens, const std::optional<at::Tensor>& kv_start,
                         const at::Tensor& centroids, int64_t key_bits, int64_t value_bits, double scale,
                         int64_t v_flags, int64_t num_splits, at::Tensor& workspace, at::Tensor& out,
                         std::optional<at::Tensor> lse, const std::optional<at::Tensor>& rotation) {
  contig(query, "query");
  on_device(kv_cache, "kv_cache");
  contig(block_table, "block_table");
  contig(seq_lens, "seq_lens");
  contig(centroids, "centroids");
  contig(workspace, "workspace");
  contig(out, "out");
  TORCH_CHECK(query.dim() == 3 && out.sizes() == query.sizes(), "fused_tq: query and out must be [B, Hq, d]");
  TORCH_CHECK(kv_cache.dim() == 4 && kv_cache.scalar_type() == at::kByte && kv_cache.stride(3) == 1,
              "fused_tq: kv_cache must be uint8 [num_blocks, block_size, Hkv, slot] with contiguous slots");
  TORCH_CHECK(block_table.scalar_type() == at::kInt && seq_lens.scalar_type() == at::kInt,
              "fused_tq: block_table and seq_lens must be int32");
  if (kv_start.has_value()) contig(*kv_start, "kv_start");
  if (lse.has_value()) contig(*lse, "lse");
  if (rotation.has_value()) contig(*rotation, "rotation");
  const c10::DeviceGuard g(query.device());
  check_rc(ftq_v1_decode_attention_rot(
      query.data_ptr(), dt(query), kv_cache.data_ptr<uint8_t>(), kv_cache.size(0), (int)kv_cache.size(1),
      kv_cache.stride(0), kv_cache.stride(1), kv_cache.stride(2), block_table.data_ptr<int32_t>(),
      (int)block_table.size(1), seq_lens.data_ptr<int32_t>(),
      kv_start.has_value() ? kv_start->data_ptr<int32_t>() : nullptr, (int)query.size(0), (int)query.size(1),
      (int)kv_cache.size(2), (int)query.size(2), centroids.data_ptr<float>(), (int)key_bits, (int)value_bits,
      (float)scale, (int)v_flags, (int)num_splits, workspace.data_ptr(), workspace.numel() * workspace.element_size(),
      out.data_ptr(), dt(out), lse.has_value() ? lse->data_ptr<float>() : nullptr,
      rotation.has_value() ? rotation->data_ptr<float>() : nullptr, stream_of(query)));
}

// ---- raw fp16 slots (boundary layers) -------------------------------------

void raw_store(const at::Tensor& key, const at::Tensor& value, at::Tensor& kv_cache, const at::Tensor& slot_mapping) {
  contig(key, "key");
  contig(value, "value");
  on_device(kv_cache, "kv_cache");
  contig(slot_mapping, "slot_mapping");
  TORCH_CHECK(key.dim() == 3 && value.sizes() == key.sizes(), "fused_tq: key/value must be [n, Hkv, d]");
  TORCH_CHECK(kv_cache.dim() == 4 && kv_cache.scalar_type() == at::kByte && kv_cache.stride(3) == 1,
              "fused_tq: kv_cache must be uint8 [num_blocks, block_size, Hkv, slot] with contiguous slots");
  const c10::DeviceGuard g(key.device());
  check_rc(ftq_raw_store(key.data_ptr(), value.data_ptr(), dt(key), key.size(0), (int)key.size(1), (int)key.size(2),
                         slot_mapping.data_ptr<int64_t>(), kv_cache.data_ptr<uint8_t>(), kv_cache.size(0),
                         (int)kv_cache.size(1), kv_cache.stride(0), kv_cache.stride(1), kv_cache.stride(2),
                         stream_of(key)));
}

void raw_decode_attention(const at::Tensor& query, const at::Tensor& kv_cache, const at::Tensor& block_table,
                          const at::Tensor& seq_lens, const std::optional<at::Tensor>& kv_start, double scale,
                          int64_t num_splits, at::Tensor& workspace, at::Tensor& out, std::optional<at::Tensor> lse) {
  contig(query, "query");
  on_device(kv_cache, "kv_cache");
  contig(block_table, "block_table");
  contig(seq_lens, "seq_lens");
  contig(workspace, "workspace");
  contig(out, "out");
  TORCH_CHECK(query.dim() == 3 && out.sizes() == query.sizes(), "fused_tq: query and out must be [B, Hq, d]");
  TORCH_CHECK(kv_cache.dim() == 4 && kv_cache.scalar_type() == at::kByte && kv_cache.stride(3) == 1,
              "fused_tq: kv_cache must be uint8 [num_blocks, block_size, Hkv, slot] with contiguous slots");
  if (kv_start.has_value()) contig(*kv_start, "kv_start");
  if (lse.has_value()) contig(*lse, "lse");
  const c10::DeviceGuard g(query.device());
  check_rc(ftq_raw_decode_attention_lse(
      query.data_ptr(), dt(query), kv_cache.data_ptr<uint8_t>(), kv_cache.size(0), (int)kv_cache.size(1),
      kv_cache.stride(0), kv_cache.stride(1), kv_cache.stride(2), block_table.data_ptr<int32_t>(),
      (int)block_table.size(1), seq_lens.data_ptr<int32_t>(),
      kv_start.has_value() ? kv_start->data_ptr<int32_t>() : nullptr, (int)query.size(0), (int)query.size(1),
      (int)kv_cache.size(2), (int)query.size(2), (float)scale, (int)num_splits, workspace.data_ptr(),
      workspace.numel() * workspace.element_size(), out.data_ptr(), dt(out),
      lse.has_value() ? lse->data_ptr<float>() : nullptr, stream_of(query)));
}

}  // namespace

TORCH_LIBRARY(fused_tq, m) {
  m.def("encode(Tensor x, Tensor signs, Tensor boundaries, int bits, int codebook_class) -> (Tensor, Tensor)");
  m.def("encode_kv(Tensor k, Tensor v, Tensor signs, Tensor boundaries, int bits, int codebook_class) -> "
        "(Tensor, Tensor, Tensor, Tensor)");
  m.def("decode(Tensor packed, Tensor norms, Tensor levels, Tensor signs, int bits, int d, ScalarType out_dtype) -> Tensor");
  m.def("rht(Tensor x, Tensor signs, bool inverse, ScalarType out_dtype) -> Tensor");
  m.def("paged_store(Tensor key, Tensor value, Tensor(a!) kv_cache, Tensor slot_mapping, Tensor k_signs, "
        "Tensor v_signs, Tensor k_boundaries, Tensor v_boundaries, int bits_k, int bits_v, int page_size) -> ()");
  m.def("paged_decode_attention(Tensor query, Tensor kv_cache, Tensor block_table, Tensor seq_lens, "
        "Tensor k_signs, Tensor v_signs, Tensor k_levels, Tensor v_levels, int bits_k, int bits_v, int page_size, "
        "float scale, int num_splits, Tensor(a!) workspace, Tensor(b!) out, bool fp32_operands) -> ()");
  m.def("v1_store(Tensor key, Tensor value, Tensor(a!) kv_cache, Tensor slot_mapping, Tensor midpoints, "
        "int key_bits, int value_bits, int v_flags, Tensor? rotation, Tensor? coeffs) -> ()");
  m.def("v1_decode_attention(Tensor query, Tensor kv_cache, Tensor block_table, Tensor seq_lens, "
        "Tensor? kv_start, Tensor centroids, int key_bits, int value_bits, float scale, int v_flags, "
        "int num_splits, Tensor(a!) workspace, Tensor(b!) out, Tensor(c!)? lse, Tensor? rotation) -> ()");
  m.def("raw_store(Tensor key, Tensor value, Tensor(a!) kv_cache, Tensor slot_mapping) -> ()");
  m.def("raw_decode_attention(Tensor query, Tensor kv_cache, Tensor block_table, Tensor seq_lens, "
        "Tensor? kv_start, float scale, int num_splits, Tensor(a!) workspace, Tensor(b!) out, "
        "Tensor(c!)? lse) -> ()");
}

TORCH_LIBRARY_IMPL(fused_tq, CUDA, m) {
  m.impl("encode", &encode);
  m.impl("encode_kv", &encode_kv);
  m.impl("decode", &decode);
  m.impl("rht", &rht);
  m.impl("paged_store", &paged_store);
  m.impl("paged_decode_attention", &paged_decode_attention);
  m.impl("v1_store", &v1_store);
  m.impl("v1_decode_attention", &v1_decode_attention);
  m.impl("raw_store", &raw_store);
  m.impl("raw_decode_attention", &raw_decode_attention);
}
