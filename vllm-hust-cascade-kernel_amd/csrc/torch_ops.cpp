// torch_ops.cpp - PyTorch-ROCm custom-op layer over the C ABI (cascade_kernels.h).
//
// Registers the reference's op schemas verbatim under namespace `npu`
// (ascend-kernel/csrc/register.cpp:24-31) plus three additive ops, with the
// implementations on the CUDA dispatch key (HIP devices on PyTorch-ROCm) and a
// Meta implementation for shape inference. Validation mirrors the reference's
// op_host TORCH_CHECKs and their "<op>: ..." messages; every launch goes to the
// current HIP stream and never synchronises (except where the reference itself
// pulls seqlens to the host: fa_fp32_stage1 with q_seqlen_value == 0).
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <algorithm>
#include <cmath>
#include <tuple>
#include <vector>

#include "cascade_kernels.h"

namespace cascade_amd {
namespace {

void *stream_of(const at::Tensor &t) {
    return reinterpret_cast<void *>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

void check_launch(int rc, const char *op) {
    TORCH_CHECK(rc == CK_OK, op, ": kernel launch failed: ", ck_error_string(rc), " (code ", rc, ")");
}

bool on_device(const at::Tensor &t) { return t.device().is_cuda() || t.device().is_meta(); }

// ----------------------------------------------------------------------------
// lse_merge: ascend-kernel/csrc/ops/lse_merge/op_host/lse_merge.cpp:32-70
// ----------------------------------------------------------------------------
struct MergeShape {
    at::ScalarType out_type;
    int64_t dim, rows, s1, s2;
};

MergeShape merge_checks(const char *op, const at::Tensor &o1, const at::Tensor &o2, const at::Tensor &lse1,
                        const at::Tensor &lse2, int64_t out_code, bool o2_f32_ok) {
    TORCH_CHECK(o1.is_contiguous() && o2.is_contiguous() && lse1.is_contiguous() && lse2.is_contiguous(),
                op, ": all inputs must be contiguous");
    TORCH_CHECK(o1.scalar_type() == at::kBFloat16 || o1.scalar_type() == at::kFloat, op,
                ": o1 must be bf16 or fp32");
    if (o2_f32_ok) {
        TORCH_CHECK(o2.scalar_type() == at::kBFloat16 || o2.scalar_type() == at::kFloat, op,
                    ": o2 must be bf16 or fp32");
    } else {
        TORCH_CHECK(o2.scalar_type() == at::kBFloat16, op, ": o2 must be bf16");
    }
    TORCH_CHECK(lse1.scalar_type() == at::kFloat && lse2.scalar_type() == at::kFloat, op,
                ": lse1/lse2 must be fp32");
    TORCH_CHECK(out_code >= 0 && out_code <= 2, op, ": out_code must be 0 (follow o1), 1 (bf16) or 2 (fp32)");
    TORCH_CHECK(o1.dim() >= 1, op, ": o1 must have a head dim");
    TORCH_CHECK(o1.sizes() == o2.sizes(), op, ": o1 and o2 must have the same shape");
    TORCH_CHECK(on_device(o1) && o1.device() == o2.device() && o1.device() == lse1.device() &&
                    o1.device() == lse2.device(),
                op, ": all tensors must be on the same HIP device");
    MergeShape s;
    s.out_type = (out_code == 1) ? at::kBFloat16 : (out_code == 2) ? at::kFloat : o1.scalar_type();
    TORCH_CHECK(o1.size(-1) % 16 == 0, op, ": head dim must be a multiple of 16 (MTE 32B alignment)");
    s.dim = o1.size(-1);
    s.rows = s.dim > 0 ? o1.numel() / s.dim : 0;
    s.s1 = s.s2 = 1;
    if (s.rows > 0) {
        TORCH_CHECK(lse1.numel() % s.rows == 0 && lse2.numel() % s.rows == 0, op,
                    ": lse numel must be a multiple of the row count (row-stride packing)");
        s.s1 = lse1.numel() / s.rows;
        s.s2 = lse2.numel() / s.rows;
        TORCH_CHECK(s.s1 >= 1 && s.s1 <= 64 && s.s2 >= 1 && s.s2 <= 64, op, ": lse row stride must be in [1, 64]");
    }
    return s;
}

int dtype_tag(at::ScalarType t) { return t == at::kFloat ? CK_DTYPE_F32 : CK_DTYPE_BF16; }

at::Tensor lse_merge_impl(const at::Tensor &o1, const at::Tensor &o2, const at::Tensor &lse1,
                          const at::Tensor &lse2, int64_t out_code) {
    MergeShape s = merge_checks("lse_merge", o1, o2, lse1, lse2, out_code, false);
    auto out = at::empty(o1.sizes(), o1.options().dtype(s.out_type));
    if (s.rows == 0 || o1.device().is_meta()) return out;
    c10::OptionalDeviceGuard guard(o1.device());
    check_launch(ck_lse_merge(o1.data_ptr(), dtype_tag(o1.scalar_type()), o2.data_ptr(),
                              dtype_tag(o2.scalar_type()), lse1.data_ptr<float>(), s.s1, lse2.data_ptr<float>(),
                              s.s2, out.data_ptr(), dtype_tag(s.out_type), nullptr, s.rows, s.dim, stream_of(o1)),
                 "lse_merge");
    return out;
}

// Additive: fp32 or bf16 o2, and the merged LSE m + ln(w1 + w2) as a second output.
std::tuple<at::Tensor, at::Tensor> lse_merge_with_lse_impl(const at::Tensor &o1, const at::Tensor &o2,
                                                           const at::Tensor &lse1, const at::Tensor &lse2,
                                                           int64_t out_code) {
    MergeShape s = merge_checks("lse_merge_with_lse", o1, o2, lse1, lse2, out_code, true);
    auto out = at::empty(o1.sizes(), o1.options().dtype(s.out_type));
    auto lse_sizes = o1.sizes().vec();
    lse_sizes.pop_back();
    auto lse_out = at::empty(lse_sizes, o1.options().dtype(at::kFloat));
    if (s.rows == 0 || o1.device().is_meta()) return {out, lse_out};
    c10::OptionalDeviceGuard guard(o1.device());
    check_launch(ck_lse_merge(o1.data_ptr(), dtype_tag(o1.scalar_type()), o2.data_ptr(),
                              dtype_tag(o2.scalar_type()), lse1.data_ptr<float>(), s.s1, lse2.data_ptr<float>(),
                              s.s2, out.data_ptr(), dtype_tag(s.out_type), lse_out.data_ptr<float>(), s.rows,
                              s.dim, stream_of(o1)),
                 "lse_merge_with_lse");
    return {out, lse_out};
}

// ----------------------------------------------------------------------------
// fa_fp32_stage1: ascend-kernel/csrc/ops/fa_fp32_stage1/op_host/fa_fp32_stage1.cpp:178-329
// ----------------------------------------------------------------------------
std::tuple<at::Tensor, at::Tensor> fa_fp32_stage1_impl(const at::Tensor &query, const at::Tensor &key,
                                                       const at::Tensor &value, const at::Tensor &block_table,
                                                       const at::Tensor &actual_q_seqlens,
                                                       const at::Tensor &actual_kv_seqlens,
                                                       int64_t q_seqlen_value) {
    TORCH_CHECK(query.is_contiguous() && key.is_contiguous() && value.is_contiguous() &&
                    block_table.is_contiguous() && actual_q_seqlens.is_contiguous() &&
                    actual_kv_seqlens.is_contiguous(),
                "fa_fp32_stage1: all inputs must be contiguous");
    TORCH_CHECK(query.scalar_type() == at::kBFloat16, "fa_fp32_stage1: query must be bf16");
    TORCH_CHECK(key.scalar_type() == at::kBFloat16 && value.scalar_type() == at::kBFloat16,
                "fa_fp32_stage1: key/value must be bf16");
    TORCH_CHECK(block_table.scalar_type() == at::kInt, "fa_fp32_stage1: block_table must be int32");
    TORCH_CHECK(actual_q_seqlens.scalar_type() == at::kLong && actual_kv_seqlens.scalar_type() == at::kLong,
                "fa_fp32_stage1: seqlens must be int64");
    TORCH_CHECK(query.dim() == 3, "fa_fp32_stage1: query must be (T, H, D)");
    TORCH_CHECK(key.dim() == 4 && value.dim() == 4,
                "fa_fp32_stage1: key/value must be (numBlocks, blockSize, KVH, D)");
    TORCH_CHECK(key.sizes() == value.sizes(), "fa_fp32_stage1: key/value shapes must match");
    TORCH_CHECK(q_seqlen_value >= 0, "fa_fp32_stage1: q_seqlen_value must be >= 0 (0 = read seqlens from device)");
    TORCH_CHECK(block_table.dim() == 2, "fa_fp32_stage1: block_table must be (B, cols)");
    TORCH_CHECK(on_device(query) && key.device() == query.device() && value.device() == query.device() &&
                    block_table.device() == query.device() && actual_q_seqlens.device() == query.device() &&
                    actual_kv_seqlens.device() == query.device(),
                "fa_fp32_stage1: all tensors must be on the same HIP device");

    const int64_t num_tokens = query.size(0);
    const int64_t num_heads = query.size(1);
    const int64_t embed = query.size(2);
    const int64_t kv_heads = key.size(2);
    const int64_t block_size = key.size(1);
    const int64_t batch = actual_q_seqlens.numel();
    TORCH_CHECK(actual_kv_seqlens.numel() == batch, "fa_fp32_stage1: seqlen tensors must have batch entries");
    TORCH_CHECK(embed == 128, "fa_fp32_stage1: only head dim 128 is supported (the kernels' MFMA tiles span 128 dims)");
    TORCH_CHECK(block_size == 128, "fa_fp32_stage1: only paged blockSize 128 is supported");
    TORCH_CHECK(kv_heads > 0 && num_heads % kv_heads == 0, "fa_fp32_stage1: numHeads must be a multiple of kvHeads");
    TORCH_CHECK(key.size(3) == embed, "fa_fp32_stage1: key/value head dim must equal the query head dim");
    if (batch == 0 || num_tokens == 0) {
        auto empty_out = at::empty({num_tokens, num_heads, embed}, query.options().dtype(at::kFloat));
        auto empty_lse = at::empty({0}, query.options().dtype(at::kFloat));
        return {empty_out, empty_lse};
    }
    TORCH_CHECK(block_table.size(0) >= batch, "fa_fp32_stage1: block_table must have a row per request");
    const int64_t cols = block_table.size(1);

    int64_t max_q_len = 0, kv_cap = 0, q_len_uniform = 0;
    at::Tensor q_start_dev;
    if (q_seqlen_value > 0) {
        TORCH_CHECK(num_tokens == batch * q_seqlen_value, "fa_fp32_stage1: with q_seqlen_value=", q_seqlen_value,
                    ", query.size(0) must equal batch * q_seqlen_value");
        // Graph-capture-safe path: no device->host traffic. kv seqlens stay on the
        // device; block_table cols bound them (a caller contract, as in the reference).
        q_len_uniform = q_seqlen_value;
        max_q_len = q_seqlen_value;
        kv_cap = cols * block_size;
    } else {
        if (query.device().is_meta()) {
            // Meta: no values; shapes only.
            auto out = at::empty({num_tokens, num_heads, embed}, query.options().dtype(at::kFloat));
            auto lse = at::empty({num_tokens * num_heads * 8}, query.options().dtype(at::kFloat));
            return {out, lse};
        }
        auto q_cpu = actual_q_seqlens.to(at::kCPU);
        auto kv_cpu = actual_kv_seqlens.to(at::kCPU);
        const int64_t *q_seq = q_cpu.data_ptr<int64_t>();
        const int64_t *kv_seq = kv_cpu.data_ptr<int64_t>();
        int64_t sum_q = 0, max_kv = 0;
        std::vector<int32_t> starts(batch);
        bool uniform = true;
        for (int64_t b = 0; b < batch; ++b) {
            TORCH_CHECK(q_seq[b] >= 1 && kv_seq[b] >= 1, "fa_fp32_stage1: seqlens must be >= 1");
            starts[b] = static_cast<int32_t>(sum_q);
            sum_q += q_seq[b];
            max_q_len = std::max(max_q_len, q_seq[b]);
            max_kv = std::max(max_kv, kv_seq[b]);
            uniform = uniform && q_seq[b] == q_seq[0];
        }
        TORCH_CHECK(sum_q == num_tokens, "fa_fp32_stage1: query.size(0) must equal sum(actual_q_seqlens)");
        TORCH_CHECK((max_kv + block_size - 1) / block_size <= cols,
                    "fa_fp32_stage1: block_table cols too small for max kv seqlen");
        // Same kv bound as the shape-only path, so both call modes produce
        // identical splits and therefore bit-identical results.
        kv_cap = cols * block_size;
        if (uniform) {
            q_len_uniform = q_seq[0];
        } else {
            q_start_dev = at::from_blob(starts.data(), {batch}, at::TensorOptions().dtype(at::kInt))
                              .to(query.device());
        }
    }

    auto out = at::empty({num_tokens, num_heads, embed}, query.options().dtype(at::kFloat));
    auto lse = at::empty({num_tokens * num_heads * 8}, query.options().dtype(at::kFloat));
    if (query.device().is_meta()) return {out, lse};

    c10::OptionalDeviceGuard guard(query.device());
    int64_t num_splits = 0, ws_bytes = 0;
    check_launch(ck_fa_fp32_stage1_plan(batch, max_q_len, num_heads, kv_heads, embed, kv_cap, &num_splits,
                                        &ws_bytes),
                 "fa_fp32_stage1");
    at::Tensor ws;
    if (ws_bytes > 0) ws = at::empty({ws_bytes}, query.options().dtype(at::kByte));
    const float scale = static_cast<float>(1.0 / std::sqrt(1.0 * embed));
    check_launch(ck_fa_fp32_stage1(query.data_ptr(), key.data_ptr(), value.data_ptr(),
                                   block_table.data_ptr<int32_t>(), cols, actual_q_seqlens.data_ptr<int64_t>(),
                                   actual_kv_seqlens.data_ptr<int64_t>(),
                                   q_start_dev.defined() ? q_start_dev.data_ptr<int32_t>() : nullptr, batch,
                                   q_len_uniform, max_q_len, num_tokens, num_heads, kv_heads, embed, key.size(0),
                                   block_size, scale, kv_cap, num_splits, out.data_ptr<float>(),
                                   lse.data_ptr<float>(), ws.defined() ? ws.data_ptr() : nullptr, ws_bytes,
                                   stream_of(query)),
                 "fa_fp32_stage1");
    return {out, lse};
}

// ----------------------------------------------------------------------------
// suffix_decode (additive): the stage-2 role of CANN FIA v2 (ascend-kernel/README.md:181-197)
// ----------------------------------------------------------------------------
std::tuple<at::Tensor, at::Tensor> suffix_decode_impl(const at::Tensor &query, const at::Tensor &key,
                                                      const at::Tensor &value, const at::Tensor &block_table,
                                                      const at::Tensor &actual_kv_seqlens, int64_t kv_layout) {
    TORCH_CHECK(query.is_contiguous() && key.is_contiguous() && value.is_contiguous() &&
                    block_table.is_contiguous() && actual_kv_seqlens.is_contiguous(),
                "suffix_decode: all inputs must be contiguous");
    TORCH_CHECK(query.scalar_type() == at::kBFloat16, "suffix_decode: query must be bf16");
    TORCH_CHECK(key.scalar_type() == at::kBFloat16 && value.scalar_type() == at::kBFloat16,
                "suffix_decode: key/value must be bf16");
    TORCH_CHECK(block_table.scalar_type() == at::kInt, "suffix_decode: block_table must be int32");
    TORCH_CHECK(actual_kv_seqlens.scalar_type() == at::kLong, "suffix_decode: seqlens must be int64");
    TORCH_CHECK(query.dim() == 3, "suffix_decode: query must be (B, H, D)");
    TORCH_CHECK(kv_layout == CK_KV_NHD || kv_layout == CK_KV_BNSD,
                "suffix_decode: kv_layout must be 0 (NHD) or 1 (BNSD)");
    TORCH_CHECK(key.dim() == 4 && value.dim() == 4,
                "suffix_decode: key/value must be (numBlocks, blockSize, KVH, D) or (numBlocks, KVH, blockSize, D)");
    TORCH_CHECK(key.sizes() == value.sizes(), "suffix_decode: key/value shapes must match");
    TORCH_CHECK(block_table.dim() == 2, "suffix_decode: block_table must be (B, cols)");
    TORCH_CHECK(on_device(query) && key.device() == query.device() && value.device() == query.device() &&
                    block_table.device() == query.device() && actual_kv_seqlens.device() == query.device(),
                "suffix_decode: all tensors must be on the same HIP device");
    const int64_t batch = query.size(0), num_heads = query.size(1), embed = query.size(2);
    const bool bnsd = kv_layout == CK_KV_BNSD;
    const int64_t kv_heads = key.size(bnsd ? 1 : 2), block_size = key.size(bnsd ? 2 : 1);
    TORCH_CHECK(actual_kv_seqlens.numel() == batch && block_table.size(0) == batch,
                "suffix_decode: block_table rows and kv seqlens must have batch entries");
    TORCH_CHECK(embed == 128 && key.size(3) == 128, "suffix_decode: only head dim 128 is supported");
    TORCH_CHECK(block_size == 128, "suffix_decode: only paged blockSize 128 is supported");
    TORCH_CHECK(kv_heads > 0 && num_heads % kv_heads == 0, "suffix_decode: numHeads must be a multiple of kvHeads");
    auto out = at::empty({batch, num_heads, embed}, query.options());
    auto lse = at::empty({batch * num_heads}, query.options().dtype(at::kFloat));
    if (batch == 0 || query.device().is_meta()) return {out, lse};
    const int64_t cols = block_table.size(1);
    const int64_t kv_cap = cols * block_size;
    c10::OptionalDeviceGuard guard(query.device());
    int64_t num_splits = 0, ws_bytes = 0;
    check_launch(ck_suffix_decode_plan(batch, num_heads, kv_heads, embed, kv_cap, &num_splits, &ws_bytes),
                 "suffix_decode");
    at::Tensor ws;
    if (ws_bytes > 0) ws = at::empty({ws_bytes}, query.options().dtype(at::kByte));
    const float scale = static_cast<float>(1.0 / std::sqrt(1.0 * embed));
    check_launch(ck_suffix_decode(query.data_ptr(), key.data_ptr(), value.data_ptr(),
                                  block_table.data_ptr<int32_t>(), cols, actual_kv_seqlens.data_ptr<int64_t>(),
                                  batch, num_heads, kv_heads, embed, key.size(0), block_size, kv_layout, scale, kv_cap,
                                  num_splits, out.data_ptr(), lse.data_ptr<float>(),
                                  ws.defined() ? ws.data_ptr() : nullptr, ws_bytes, stream_of(query)),
                 "suffix_decode");
    return {out, lse};
}

// ----------------------------------------------------------------------------
// cascade_decode (additive): the documented caller-side cascade
// (ascend-kernel/README.md:160-201) as one op. Shape-only host logic, no
// device->host traffic: the kv bounds come from the block-table widths.
// ----------------------------------------------------------------------------
std::tuple<at::Tensor, at::Tensor> cascade_decode_impl(const at::Tensor &query, const at::Tensor &prefix_key,
                                                       const at::Tensor &prefix_value,
                                                       const at::Tensor &prefix_block_table,
                                                       const at::Tensor &prefix_kv_seqlens,
                                                       const at::Tensor &suffix_key, const at::Tensor &suffix_value,
                                                       const at::Tensor &suffix_block_table,
                                                       const at::Tensor &suffix_kv_seqlens, int64_t suffix_kv_layout) {
    for (const at::Tensor *t : {&query, &prefix_key, &prefix_value, &prefix_block_table, &prefix_kv_seqlens,
                                &suffix_key, &suffix_value, &suffix_block_table, &suffix_kv_seqlens})
        TORCH_CHECK(t->is_contiguous(), "cascade_decode: all inputs must be contiguous");
    TORCH_CHECK(query.scalar_type() == at::kBFloat16, "cascade_decode: query must be bf16");
    TORCH_CHECK(prefix_key.scalar_type() == at::kBFloat16 && prefix_value.scalar_type() == at::kBFloat16 &&
                    suffix_key.scalar_type() == at::kBFloat16 && suffix_value.scalar_type() == at::kBFloat16,
                "cascade_decode: key/value must be bf16");
    TORCH_CHECK(prefix_block_table.scalar_type() == at::kInt && suffix_block_table.scalar_type() == at::kInt,
                "cascade_decode: block tables must be int32");
    TORCH_CHECK(prefix_kv_seqlens.scalar_type() == at::kLong && suffix_kv_seqlens.scalar_type() == at::kLong,
                "cascade_decode: seqlens must be int64");
    TORCH_CHECK(query.dim() == 3, "cascade_decode: query must be (B, H, D)");
    TORCH_CHECK(prefix_key.dim() == 4 && prefix_key.sizes() == prefix_value.sizes() && suffix_key.dim() == 4 &&
                    suffix_key.sizes() == suffix_value.sizes(),
                "cascade_decode: key/value must be matching (numBlocks, blockSize, KVH, D) pools "
                "(the suffix pool (numBlocks, KVH, blockSize, D) with suffix_kv_layout 1)");
    TORCH_CHECK(suffix_kv_layout == CK_KV_NHD || suffix_kv_layout == CK_KV_BNSD,
                "cascade_decode: suffix_kv_layout must be 0 (NHD) or 1 (BNSD)");
    const bool sfx_bnsd = suffix_kv_layout == CK_KV_BNSD;
    TORCH_CHECK(prefix_block_table.dim() == 2 && prefix_block_table.size(0) >= 1 && prefix_kv_seqlens.numel() == 1,
                "cascade_decode: the prefix is one request: block_table (1, cols), kv seqlens (1,)");
    const int64_t batch = query.size(0), num_heads = query.size(1), embed = query.size(2);
    const int64_t kv_heads = prefix_key.size(2);
    TORCH_CHECK(suffix_key.size(sfx_bnsd ? 1 : 2) == kv_heads,
                "cascade_decode: prefix and suffix pools must have the same kv heads");
    TORCH_CHECK(suffix_block_table.dim() == 2 && suffix_block_table.size(0) == batch &&
                    suffix_kv_seqlens.numel() == batch,
                "cascade_decode: suffix block_table rows and kv seqlens must have batch entries");
    TORCH_CHECK(embed == 128 && prefix_key.size(3) == 128 && suffix_key.size(3) == 128,
                "cascade_decode: only head dim 128 is supported");
    TORCH_CHECK(prefix_key.size(1) == 128 && suffix_key.size(sfx_bnsd ? 2 : 1) == 128,
                "cascade_decode: only paged blockSize 128 is supported");
    TORCH_CHECK(kv_heads > 0 && num_heads % kv_heads == 0, "cascade_decode: numHeads must be a multiple of kvHeads");
    for (const at::Tensor *t : {&prefix_key, &prefix_value, &prefix_block_table, &prefix_kv_seqlens, &suffix_key,
                                &suffix_value, &suffix_block_table, &suffix_kv_seqlens})
        TORCH_CHECK(t->device() == query.device(), "cascade_decode: all tensors must be on the same HIP device");
    TORCH_CHECK(on_device(query), "cascade_decode: tensors must be on a HIP device");
    auto out = at::empty({batch, num_heads, embed}, query.options());
    auto lse = at::empty({batch * num_heads}, query.options().dtype(at::kFloat));
    if (batch == 0 || query.device().is_meta()) return {out, lse};
    const int64_t pcols = prefix_block_table.size(1), scols = suffix_block_table.size(1);
    const int64_t prefix_cap = pcols * 128, suffix_cap = scols * 128;
    c10::OptionalDeviceGuard guard(query.device());
    int64_t ws_bytes = 0;
    check_launch(ck_cascade_decode_plan(batch, num_heads, kv_heads, embed, prefix_cap, suffix_cap, &ws_bytes),
                 "cascade_decode");
    at::Tensor ws = at::empty({ws_bytes > 0 ? ws_bytes : 1}, query.options().dtype(at::kByte));
    const float scale = static_cast<float>(1.0 / std::sqrt(1.0 * embed));
    check_launch(ck_cascade_decode(query.data_ptr(), prefix_key.data_ptr(), prefix_value.data_ptr(),
                                   prefix_block_table.data_ptr<int32_t>(), pcols,
                                   prefix_kv_seqlens.data_ptr<int64_t>(), prefix_key.size(0), suffix_key.data_ptr(),
                                   suffix_value.data_ptr(), suffix_block_table.data_ptr<int32_t>(), scols,
                                   suffix_kv_seqlens.data_ptr<int64_t>(), suffix_key.size(0), suffix_kv_layout,
                                   batch, num_heads,
                                   kv_heads, embed, 128, scale, prefix_cap, suffix_cap, out.data_ptr(),
                                   lse.data_ptr<float>(), ws.data_ptr(), ws.numel(), stream_of(query)),
                 "cascade_decode");
    return {out, lse};
}

// ----------------------------------------------------------------------------
// f3_gateup_epilogue: ascend-kernel/csrc/ops/f3_floor/op_host/f3_floor.cpp:59-124
// ----------------------------------------------------------------------------
std::tuple<at::Tensor, at::Tensor> f3_gateup_epilogue_impl(const at::Tensor &a, const at::Tensor &b,
                                                           const c10::optional<at::Tensor> &workspace,
                                                           const c10::optional<at::Tensor> &out_d, int64_t mode) {
    TORCH_CHECK(a.dim() == 2 && a.is_contiguous() && a.scalar_type() == at::kBFloat16,
                "f3_gateup_epilogue: a must be a contiguous bf16 [M, K]");
    TORCH_CHECK(b.dim() == 2 && b.is_contiguous() && b.scalar_type() == at::kBFloat16,
                "f3_gateup_epilogue: b must be a contiguous bf16 [2I, K]");
    TORCH_CHECK((mode >= 0 && mode <= 5) || mode == 7 || mode == 8,
                "f3_gateup_epilogue: mode must be 0..5, 7 or 8");
    const int64_t m_rows = a.size(0), k_dim = a.size(1);
    TORCH_CHECK(b.size(0) % 2 == 0, "f3_gateup_epilogue: b.size(0) must be even (gate | up)");
    const int64_t i_half = b.size(0) / 2;
    TORCH_CHECK(b.size(1) == k_dim, "f3_gateup_epilogue: a.size(1) must equal b.size(1)");
    TORCH_CHECK(m_rows > 0 && k_dim > 0, "f3_gateup_epilogue: empty input");
    TORCH_CHECK(k_dim % 16 == 0, "f3_gateup_epilogue: K must be a multiple of 16");
    TORCH_CHECK(i_half % 128 == 0 && i_half > 0, "f3_gateup_epilogue: I must be a multiple of the N tile");
    TORCH_CHECK(k_dim >= 64, "f3_gateup_epilogue: K must be >= 64 (L0 K tile)");
    TORCH_CHECK(on_device(a) && b.device() == a.device(), "f3_gateup_epilogue: a and b must be on the same HIP device");

    at::Tensor ws;
    if (workspace.has_value() && workspace->defined()) {
        const at::Tensor &w = *workspace;
        TORCH_CHECK(w.is_contiguous() && w.scalar_type() == at::kBFloat16 && w.dim() == 2 && w.size(0) == m_rows &&
                        w.size(1) == 2 * i_half,
                    "f3_gateup_epilogue: workspace must be contiguous bf16 [M, 2I]");
        TORCH_CHECK(w.device() == a.device(), "f3_gateup_epilogue: workspace must be on the device of a");
        ws = w;
    } else {
        ws = at::empty({m_rows, 2 * i_half}, a.options());
    }
    at::Tensor d;
    int64_t d_stride = i_half;
    if (out_d.has_value() && out_d->defined()) {
        const at::Tensor &dg = *out_d;
        TORCH_CHECK(dg.scalar_type() == at::kBFloat16 && dg.dim() == 2 && dg.size(0) == m_rows && dg.size(1) == i_half,
                    "f3_gateup_epilogue: d must be bf16 [M, I]");
        TORCH_CHECK(dg.stride(1) == 1 && dg.stride(0) >= i_half && dg.stride(0) % 4 == 0,
                    "f3_gateup_epilogue: d must have unit column stride and a row stride >= I that is a multiple of 4");
        TORCH_CHECK(dg.device() == a.device(), "f3_gateup_epilogue: d must be on the device of a");
        d = dg;
        d_stride = dg.stride(0);
    } else {
        d = at::empty({m_rows, i_half}, a.options());
    }
    if (a.device().is_meta()) return {d, ws};
    c10::OptionalDeviceGuard guard(a.device());
    check_launch(ck_f3_gateup_epilogue(a.data_ptr(), b.data_ptr(), ws.data_ptr(), d.data_ptr(), m_rows, i_half,
                                       k_dim, mode, d_stride, stream_of(a)),
                 "f3_gateup_epilogue");
    return {d, ws};
}

// ----------------------------------------------------------------------------
// add_rms_norm_stats: ascend-kernel/csrc/ops/add_rms_norm_stats/op_host/add_rms_norm_stats.cpp:65-141
// ----------------------------------------------------------------------------
std::tuple<at::Tensor, at::Tensor, at::Tensor> add_rms_norm_stats_impl(const at::Tensor &x1, const at::Tensor &x2,
                                                                        const c10::optional<at::Tensor> &gamma,
                                                                        const c10::optional<at::Tensor> &beta,
                                                                        double eps, int64_t mode) {
    constexpr int64_t kMaxK = 5120, kRstdGroup = 8;
    TORCH_CHECK(x1.dim() == 2, "add_rms_norm_stats: x1 must be 2D (M, K)");
    TORCH_CHECK(x1.is_contiguous(), "add_rms_norm_stats: x1 must be contiguous");
    TORCH_CHECK(mode >= 0 && mode <= 2, "add_rms_norm_stats: mode must be 0, 1 or 2");
    TORCH_CHECK(eps > 0.0, "add_rms_norm_stats: eps must be > 0");
    const bool is_bf16 = x1.scalar_type() == at::kBFloat16;
    TORCH_CHECK(is_bf16 || x1.scalar_type() == at::kHalf, "add_rms_norm_stats: x1 must be bf16 or fp16");
    if (mode != 1) {
        TORCH_CHECK(x2.defined() && x2.is_contiguous() && x2.sizes() == x1.sizes() &&
                        x2.scalar_type() == x1.scalar_type(),
                    "add_rms_norm_stats: x2 must be contiguous, same shape and dtype as x1");
        TORCH_CHECK(x2.device() == x1.device(), "add_rms_norm_stats: x2 must be on the device of x1");
    }
    const int64_t m_rows = x1.size(0), k_dim = x1.size(1);
    TORCH_CHECK(m_rows > 0, "add_rms_norm_stats: empty row count");
    TORCH_CHECK(k_dim > 0 && k_dim <= kMaxK, "add_rms_norm_stats: K must be in (0, ", kMaxK, "] (one row per wave)");
    TORCH_CHECK(k_dim % 16 == 0, "add_rms_norm_stats: K must be a multiple of 16 (32B row copies)");
    const bool has_beta = mode == 1 && beta.has_value() && beta->defined() && beta->numel() > 0;
    if (mode == 1) {
        TORCH_CHECK(gamma.has_value() && gamma->defined() && gamma->is_contiguous() && gamma->numel() == k_dim &&
                        gamma->scalar_type() == x1.scalar_type(),
                    "add_rms_norm_stats: mode 1 needs a contiguous gamma of K elements, same dtype");
        TORCH_CHECK(gamma->device() == x1.device(), "add_rms_norm_stats: gamma must be on the device of x1");
        if (has_beta) {
            TORCH_CHECK(beta->is_contiguous() && beta->numel() == k_dim && beta->scalar_type() == x1.scalar_type(),
                        "add_rms_norm_stats: beta must be contiguous, K elements, same dtype");
            TORCH_CHECK(beta->device() == x1.device(), "add_rms_norm_stats: beta must be on the device of x1");
        }
    }
    TORCH_CHECK(on_device(x1), "add_rms_norm_stats: x1 must be on a HIP device");
    const int64_t m_pad = (m_rows + kRstdGroup - 1) / kRstdGroup * kRstdGroup;
    at::Tensor x_out = mode == 0 ? at::empty_like(x1) : at::empty({0}, x1.options());
    at::Tensor rstd = at::empty({m_pad, 1}, x1.options().dtype(at::kFloat));
    at::Tensor y = mode == 1 ? at::empty_like(x1) : at::empty({0}, x1.options());
    if (x1.device().is_meta()) return {x_out, rstd, y};
    c10::OptionalDeviceGuard guard(x1.device());
    check_launch(ck_add_rms_norm_stats(x1.data_ptr(), mode != 1 ? x2.data_ptr() : nullptr,
                                       mode == 1 ? gamma->data_ptr() : nullptr, has_beta ? beta->data_ptr() : nullptr,
                                       mode == 0 ? x_out.data_ptr() : nullptr, rstd.data_ptr<float>(),
                                       mode == 1 ? y.data_ptr() : nullptr, m_rows, k_dim,
                                       is_bf16 ? CK_DTYPE_BF16 : CK_DTYPE_F16, mode, eps, stream_of(x1)),
                 "add_rms_norm_stats");
    return {x_out, rstd, y};
}

}  // namespace
}  // namespace cascade_amd

TORCH_LIBRARY_FRAGMENT(npu, m) {
    // Reference schemas, verbatim (ascend-kernel/csrc/register.cpp:24-31).
    m.def("lse_merge(Tensor o1, Tensor o2, Tensor lse1, Tensor lse2, int out_code=0) -> Tensor");
    m.def("fa_fp32_stage1(Tensor query, Tensor key, Tensor value, Tensor block_table, "
          "Tensor actual_q_seqlens, Tensor actual_kv_seqlens, int q_seqlen_value=0) -> (Tensor, Tensor)");
    m.def("f3_gateup_epilogue(Tensor a, Tensor b, Tensor? workspace, Tensor? out_d, int mode) "
          "-> (Tensor, Tensor)");
    m.def("add_rms_norm_stats(Tensor x1, Tensor x2, Tensor? gamma, Tensor? beta, float eps, "
          "int mode) -> (Tensor, Tensor, Tensor)");
    // Additive ops (no reference counterpart in the wheel).
    m.def("lse_merge_with_lse(Tensor o1, Tensor o2, Tensor lse1, Tensor lse2, int out_code=0) -> (Tensor, Tensor)");
    m.def("suffix_decode(Tensor query, Tensor key, Tensor value, Tensor block_table, "
          "Tensor actual_kv_seqlens, int kv_layout=0) -> (Tensor, Tensor)");
    m.def("cascade_decode(Tensor query, Tensor prefix_key, Tensor prefix_value, Tensor prefix_block_table, "
          "Tensor prefix_kv_seqlens, Tensor suffix_key, Tensor suffix_value, Tensor suffix_block_table, "
          "Tensor suffix_kv_seqlens, int suffix_kv_layout=0) -> (Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(npu, CUDA, m) {
    m.impl("lse_merge", TORCH_FN(cascade_amd::lse_merge_impl));
    m.impl("lse_merge_with_lse", TORCH_FN(cascade_amd::lse_merge_with_lse_impl));
    m.impl("fa_fp32_stage1", TORCH_FN(cascade_amd::fa_fp32_stage1_impl));
    m.impl("suffix_decode", TORCH_FN(cascade_amd::suffix_decode_impl));
    m.impl("cascade_decode", TORCH_FN(cascade_amd::cascade_decode_impl));
    m.impl("f3_gateup_epilogue", TORCH_FN(cascade_amd::f3_gateup_epilogue_impl));
    m.impl("add_rms_norm_stats", TORCH_FN(cascade_amd::add_rms_norm_stats_impl));
}

TORCH_LIBRARY_IMPL(npu, Meta, m) {
    m.impl("lse_merge", TORCH_FN(cascade_amd::lse_merge_impl));
    m.impl("lse_merge_with_lse", TORCH_FN(cascade_amd::lse_merge_with_lse_impl));
    m.impl("fa_fp32_stage1", TORCH_FN(cascade_amd::fa_fp32_stage1_impl));
    m.impl("suffix_decode", TORCH_FN(cascade_amd::suffix_decode_impl));
    m.impl("cascade_decode", TORCH_FN(cascade_amd::cascade_decode_impl));
    m.impl("f3_gateup_epilogue", TORCH_FN(cascade_amd::f3_gateup_epilogue_impl));
    m.impl("add_rms_norm_stats", TORCH_FN(cascade_amd::add_rms_norm_stats_impl));
}
