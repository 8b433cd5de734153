// PyTorch-ROCm extension `mla_custom_cuda`: the reference's operator surface
// (mla_kernels.cu:1688-1693) on top of the C ABI of libmla_amd.so.
//
//   q_absorbed(x, W_q_a, q_norm_w, W_q_b, W_uk, positions, nope_dim, rope_dim, eps)
//       -> [q_absorbed [B,Sq,H,R], q_rope [B,Sq,H,rope]]        (mla_kernels.cu:599-767)
//   mla_attention(q_absorbed, q_rope, c_kv, pe_cache, W_uv, scale, causal=False)
//       -> out [B,Sq,H,v]                                         (mla_kernels.cu:1479-1682)
//
// plus one op per step (gemm, rmsnorm, rope, absorb, scores, combine, ctx, out) that runs
// the very kernels the fused calls run, and the path's neighbours: split_wkv_b (weight
// prep), kv_append (the cache write) and o_proj (wo); mla_attention_paged and
// kv_append_paged for a ragged, paged cache (q_absorbed takes [B, Sq] positions for it);
// mla_attention_fp8kv and mla_attention_paged_fp8kv for an e4m3 cache.  This file only
// validates tensors, allocates outputs and workspace from torch's caching allocator and
// passes raw pointers and the current HIP stream to the C ABI; all device work lives in
// libmla_amd.so.
//
// Validation order: shapes and dtypes first, then device, so every shape error is
// reported (and testable) without a GPU.

#include <torch/extension.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "mla/mla.h"

namespace {

void check_status(int st, const char* what) {
    TORCH_CHECK(st == MLA_OK, "MLA ", what, " failed (status ", st, "): ", mla_last_error());
}

mla_dtype_t to_mla_dtype(const torch::Tensor& t, const char* name) {
    if (t.scalar_type() == torch::kFloat32) return MLA_DTYPE_F32;
    if (t.scalar_type() == torch::kBFloat16) return MLA_DTYPE_BF16;
    if (t.scalar_type() == torch::kFloat16) return MLA_DTYPE_F16;
    if (t.scalar_type() == torch::kFloat64) return MLA_DTYPE_F64;
    TORCH_CHECK(false, "MLA: ", name, " has dtype ", t.scalar_type(),
                "; supported dtypes are float32, bfloat16, float16 and float64 (float64 in "
                "q_absorbed and mla_attention)");
    return MLA_DTYPE_F32;
}

void check_same_dtype(const torch::Tensor& ref, const torch::Tensor& t, const char* name) {
    TORCH_CHECK(t.scalar_type() == ref.scalar_type(), "MLA: ", name, " has dtype ",
                t.scalar_type(), " but the inputs are ", ref.scalar_type());
}

void check_dim(const torch::Tensor& t, int64_t dim, const char* name, const char* shape) {
    TORCH_CHECK(t.dim() == dim, "MLA: ", name, " must be ", shape, " (got ", t.sizes(), ")");
}

void check_device(const std::vector<const torch::Tensor*>& ts) {
    const auto dev = ts[0]->device();
    for (const auto* t : ts) {
        TORCH_CHECK(t->is_cuda(), "MLA: tensors must be on a ROCm GPU device (got ", t->device(),
                    ")");
        TORCH_CHECK(t->device() == dev, "MLA: all tensors must be on one device (", dev, " vs ",
                    t->device(), ")");
    }
}

hipStream_t current_stream() { return c10::hip::getCurrentHIPStream().stream(); }

torch::Tensor workspace(size_t bytes, const torch::Tensor& like) {
    return torch::empty({static_cast<int64_t>(bytes > 0 ? bytes : 1)},
                        like.options().dtype(torch::kUInt8));
}

// RoPE inverse frequencies with the reference oracle's own expression,
// 1 / 10000 ** (arange(0, rope, 2) / rope)  (exhaustive_benchmark_suite.py:216-219), in the
// accumulate dtype (float32, float64 for float64 inputs), evaluated by the same ATen CPU ops
// so kernel and oracle angles are bit-identical.
torch::Tensor rope_inv_freq(int64_t rope, torch::ScalarType acc = torch::kFloat32) {
    TORCH_CHECK(rope > 0 && rope % 2 == 0, "MLA: rope_dim must be positive and even");
    auto e = torch::arange(0, rope, 2, torch::TensorOptions().dtype(acc)) / rope;
    return torch::pow(10000, e).reciprocal();
}

// The table lives on the device once per (device, rope width): a per-call host->device
// copy would be a synchronous pageable copy that stalls the caller's stream every layer.
// The cache is intentionally leaked so no tensor is freed after the HIP runtime shuts down.
torch::Tensor device_inv_freq(int64_t rope, const torch::Device& dev,
                              torch::ScalarType acc = torch::kFloat32) {
    static std::mutex mu;
    static auto* cache = new std::map<std::pair<int, int64_t>, torch::Tensor>();
    std::lock_guard<std::mutex> lock(mu);
    // one table per (device, rope width, accumulate dtype)
    const auto key = std::make_pair(static_cast<int>(dev.index()),
                                    rope * 2 + (acc == torch::kFloat64 ? 1 : 0));
    auto it = cache->find(key);
    if (it != cache->end()) return it->second;
    auto t = rope_inv_freq(rope, acc).to(dev);
    cache->emplace(key, t);
    return t;
}

// ------------------------------------------------------------------ fused: Q path

std::vector<torch::Tensor> op_q_absorbed(torch::Tensor x, torch::Tensor W_q_a, torch::Tensor q_norm_w,
                                      torch::Tensor W_q_b, torch::Tensor W_uk,
                                      torch::Tensor positions, int64_t nope_dim, int64_t rope_dim,
                                      double eps) {
    check_dim(x, 3, "x", "[B, Sq, hidden]");
    check_dim(W_q_a, 2, "W_q_a", "[hidden, q_lora]");
    check_dim(W_q_b, 2, "W_q_b", "[q_lora, H*(nope+rope)]");
    check_dim(W_uk, 3, "W_uk", "[H, nope, kv_rank]");
    const int64_t B = x.size(0), Sq = x.size(1), hidden = x.size(2);
    const int64_t q_lora = W_q_a.size(1), H = W_uk.size(0), R = W_uk.size(2);
    TORCH_CHECK(nope_dim > 0 && rope_dim > 0, "MLA: nope_dim and rope_dim must be positive");
    TORCH_CHECK(W_q_a.size(0) == hidden, "W_q_a must be [hidden, q_lora]");
    TORCH_CHECK(W_q_b.size(0) == q_lora && W_q_b.size(1) == H * (nope_dim + rope_dim),
                "W_q_b must be [q_lora, H*(nope+rope)]");
    TORCH_CHECK(W_uk.size(1) == nope_dim, "W_uk must be [H, nope, kv_rank]");
    TORCH_CHECK(q_norm_w.dim() == 1 && q_norm_w.size(0) == q_lora,
                "q_norm_w must be a 1-D tensor of length q_lora (got ", q_norm_w.sizes(), ")");
    const bool per_seq = positions.dim() == 2;
    TORCH_CHECK((positions.dim() == 1 && positions.size(0) == Sq) ||
                    (per_seq && positions.size(0) == B && positions.size(1) == Sq),
                "positions must be [Sq] (shared by the batch) or [B, Sq] (per sequence) (got ",
                positions.sizes(), ")");
    TORCH_CHECK(!positions.is_floating_point() && !positions.is_complex(),
                "positions must be an integer tensor");
    const mla_dtype_t dt = to_mla_dtype(x, "x");
    check_same_dtype(x, W_q_a, "W_q_a");
    check_same_dtype(x, q_norm_w, "q_norm_w");
    check_same_dtype(x, W_q_b, "W_q_b");
    check_same_dtype(x, W_uk, "W_uk");
    check_device({&x, &W_q_a, &q_norm_w, &W_q_b, &W_uk, &positions});

    c10::DeviceGuard guard(x.device());
    auto xc = x.contiguous();
    auto wa = W_q_a.contiguous();
    auto g = q_norm_w.contiguous();
    auto wb = W_q_b.contiguous();
    auto wuk = W_uk.contiguous();
    auto pos = positions.to(torch::kLong).contiguous();
    auto inv_freq = device_inv_freq(rope_dim, x.device(),
                                    dt == MLA_DTYPE_F64 ? torch::kFloat64 : torch::kFloat32);

    mla_dims_t d{};
    d.batch = (int32_t)B; d.sq = (int32_t)Sq; d.hidden = (int32_t)hidden;
    d.q_lora = (int32_t)q_lora; d.heads = (int32_t)H; d.nope = (int32_t)nope_dim;
    d.rope = (int32_t)rope_dim; d.kv_rank = (int32_t)R;

    auto qa = torch::empty({B, Sq, H, R}, x.options());
    auto qr = torch::empty({B, Sq, H, rope_dim}, x.options());
    const size_t wsb = mla_q_absorbed_workspace_bytes(dt, &d);
    auto ws = workspace(wsb, x);
    auto q_fn = per_seq ? mla_q_absorbed_ragged : mla_q_absorbed;
    check_status(q_fn(dt, &d, xc.data_ptr(), wa.data_ptr(), g.data_ptr(), wb.data_ptr(),
                      wuk.data_ptr(), pos.data_ptr<int64_t>(), inv_freq.data_ptr(), eps,
                      qa.data_ptr(), qr.data_ptr(), ws.data_ptr(), wsb, current_stream()),
                 "q_absorbed");
    return {qa, qr};
}

// ------------------------------------------------------------------ fused: attention

mla_dims_t attn_dims(const torch::Tensor& qa, const torch::Tensor& qr, const torch::Tensor& ckv,
                     const torch::Tensor& pe, const torch::Tensor* W_uv) {
    check_dim(qa, 4, "q_absorbed", "[B, Sq, H, kv_rank]");
    check_dim(qr, 4, "q_rope", "[B, Sq, H, rope]");
    check_dim(ckv, 3, "c_kv", "[B, Sk, kv_rank]");
    check_dim(pe, 3, "pe_cache", "[B, Sk, rope]");
    const int64_t B = qa.size(0), Sq = qa.size(1), H = qa.size(2), R = qa.size(3);
    const int64_t Sk = ckv.size(1), D = qr.size(3);
    TORCH_CHECK(qr.size(0) == B && qr.size(1) == Sq && qr.size(2) == H,
                "q_rope must be [B, Sq, H, rope] matching q_absorbed (got ", qr.sizes(), ")");
    TORCH_CHECK(ckv.size(0) == B && ckv.size(2) == R,
                "c_kv must be [B, Sk, kv_rank] (got ", ckv.sizes(), ")");
    TORCH_CHECK(pe.size(0) == B && pe.size(1) == Sk && pe.size(2) == D,
                "pe_cache must be [B, Sk, rope] (got ", pe.sizes(), ")");
    mla_dims_t d{};
    d.batch = (int32_t)B; d.sq = (int32_t)Sq; d.sk = (int32_t)Sk; d.heads = (int32_t)H;
    d.kv_rank = (int32_t)R; d.rope = (int32_t)D;
    if (W_uv) {
        check_dim(*W_uv, 3, "W_uv", "[H, v, kv_rank]");
        TORCH_CHECK(W_uv->size(0) == H && W_uv->size(2) == R,
                    "W_uv must be [H, v, kv_rank] (got ", W_uv->sizes(), ")");
        d.v = (int32_t)W_uv->size(1);
    }
    return d;
}

torch::Tensor op_mla_attention(torch::Tensor q_absorbed, torch::Tensor q_rope, torch::Tensor c_kv,
                            torch::Tensor pe_cache, torch::Tensor W_uv, double scale,
                            bool causal) {
    mla_dims_t d = attn_dims(q_absorbed, q_rope, c_kv, pe_cache, &W_uv);
    const mla_dtype_t dt = to_mla_dtype(q_absorbed, "q_absorbed");
    check_same_dtype(q_absorbed, q_rope, "q_rope");
    check_same_dtype(q_absorbed, c_kv, "c_kv");
    check_same_dtype(q_absorbed, pe_cache, "pe_cache");
    check_same_dtype(q_absorbed, W_uv, "W_uv");
    TORCH_CHECK(d.sk > 0, "MLA: c_kv must hold at least one key");
    TORCH_CHECK(!causal || d.sk >= d.sq, "MLA: causal attention needs Sk >= Sq");
    check_device({&q_absorbed, &q_rope, &c_kv, &pe_cache, &W_uv});

    c10::DeviceGuard guard(q_absorbed.device());
    auto qa = q_absorbed.contiguous();
    auto qr = q_rope.contiguous();
    auto ck = c_kv.contiguous();
    auto pe = pe_cache.contiguous();
    auto wuv = W_uv.contiguous();
    auto out = torch::empty({d.batch, d.sq, d.heads, d.v}, qa.options());
    const size_t wsb = mla_attention_workspace_bytes(dt, &d, causal ? 1 : 0);
    auto ws = workspace(wsb, qa);
    check_status(mla_attention(dt, &d, qa.data_ptr(), qr.data_ptr(), ck.data_ptr(), pe.data_ptr(),
                               wuv.data_ptr(), scale, causal ? 1 : 0, out.data_ptr(),
                               ws.data_ptr(), wsb, current_stream()),
                 "mla_attention");
    return out;
}

// Attention over an fp8 cache: c_kv / pe_cache hold e4m3 codes (torch.float8_e4m3fn or
// their bytes as uint8) of value / kv_scale; the queries, W_uv and the output are bf16.
torch::Tensor op_mla_attention_fp8kv(torch::Tensor q_absorbed, torch::Tensor q_rope,
                                     torch::Tensor c_kv, torch::Tensor pe_cache, double kv_scale,
                                     torch::Tensor W_uv, double scale, bool causal) {
    mla_dims_t d = attn_dims(q_absorbed, q_rope, c_kv, pe_cache, &W_uv);
    TORCH_CHECK(q_absorbed.scalar_type() == torch::kBFloat16,
                "MLA: an fp8 cache is read with bfloat16 queries (q_absorbed has dtype ",
                q_absorbed.scalar_type(), ")");
    check_same_dtype(q_absorbed, q_rope, "q_rope");
    check_same_dtype(q_absorbed, W_uv, "W_uv");
    for (const torch::Tensor* t : {&c_kv, &pe_cache})
        TORCH_CHECK(t->scalar_type() == torch::kFloat8_e4m3fn || t->scalar_type() == torch::kByte,
                    "MLA: the fp8 cache must be float8_e4m3fn or uint8 codes (got ",
                    t->scalar_type(), ")");
    TORCH_CHECK(d.sk > 0, "MLA: c_kv must hold at least one key");
    TORCH_CHECK(!causal || d.sk >= d.sq, "MLA: causal attention needs Sk >= Sq");
    check_device({&q_absorbed, &q_rope, &c_kv, &pe_cache, &W_uv});

    c10::DeviceGuard guard(q_absorbed.device());
    auto qa = q_absorbed.contiguous();
    auto qr = q_rope.contiguous();
    auto ck = c_kv.contiguous();
    auto pe = pe_cache.contiguous();
    auto wuv = W_uv.contiguous();
    auto out = torch::empty({d.batch, d.sq, d.heads, d.v}, qa.options());
    const size_t wsb = mla_attention_fp8kv_workspace_bytes(MLA_DTYPE_BF16, &d, causal ? 1 : 0);
    auto ws = workspace(wsb, qa);
    check_status(mla_attention_fp8kv(MLA_DTYPE_BF16, &d, qa.data_ptr(), qr.data_ptr(),
                                     ck.data_ptr(), pe.data_ptr(), (float)kv_scale,
                                     wuv.data_ptr(), scale, causal ? 1 : 0, out.data_ptr(),
                                     ws.data_ptr(), wsb, current_stream()),
                 "mla_attention_fp8kv");
    return out;
}

// e4m3 codes -> float32 values code * scale, with the attention's own conversion
torch::Tensor op_fp8_dequantize(torch::Tensor codes, double scale) {
    TORCH_CHECK(codes.scalar_type() == torch::kFloat8_e4m3fn || codes.scalar_type() == torch::kByte,
                "MLA: codes must be float8_e4m3fn or uint8 (got ", codes.scalar_type(), ")");
    check_device({&codes});
    c10::DeviceGuard guard(codes.device());
    auto c = codes.contiguous();
    auto out = torch::empty(c.sizes(), c.options().dtype(torch::kFloat32));
    check_status(mla_fp8_dequantize(c.data_ptr(), c.numel(), (float)scale, out.data_ptr<float>(),
                                    current_stream()),
                 "mla_fp8_dequantize");
    return out;
}

// Same contract as mla_attention, with keys processed in bounded chunks (the score matrix
// is never materialised whole); key_chunk = 0 picks the chunk so one chunk's fp32 score
// buffer stays within 1 GiB.
torch::Tensor op_mla_attention_streaming(torch::Tensor q_absorbed, torch::Tensor q_rope,
                                         torch::Tensor c_kv, torch::Tensor pe_cache,
                                         torch::Tensor W_uv, double scale, bool causal,
                                         int64_t key_chunk) {
    mla_dims_t d = attn_dims(q_absorbed, q_rope, c_kv, pe_cache, &W_uv);
    const mla_dtype_t dt = to_mla_dtype(q_absorbed, "q_absorbed");
    check_same_dtype(q_absorbed, q_rope, "q_rope");
    check_same_dtype(q_absorbed, c_kv, "c_kv");
    check_same_dtype(q_absorbed, pe_cache, "pe_cache");
    check_same_dtype(q_absorbed, W_uv, "W_uv");
    TORCH_CHECK(d.sk > 0, "MLA: c_kv must hold at least one key");
    TORCH_CHECK(!causal || d.sk >= d.sq, "MLA: causal attention needs Sk >= Sq");
    TORCH_CHECK(key_chunk >= 0 && key_chunk % mla_score_tile() == 0,
                "MLA: key_chunk must be 0 or a positive multiple of ", mla_score_tile());
    check_device({&q_absorbed, &q_rope, &c_kv, &pe_cache, &W_uv});

    c10::DeviceGuard guard(q_absorbed.device());
    auto qa = q_absorbed.contiguous();
    auto qr = q_rope.contiguous();
    auto ck = c_kv.contiguous();
    auto pe = pe_cache.contiguous();
    auto wuv = W_uv.contiguous();
    auto out = torch::empty({d.batch, d.sq, d.heads, d.v}, qa.options());
    const size_t wsb = mla_attention_streaming_workspace_bytes(dt, &d, causal ? 1 : 0,
                                                               (int32_t)key_chunk);
    auto ws = workspace(wsb, qa);
    check_status(mla_attention_streaming(dt, &d, qa.data_ptr(), qr.data_ptr(), ck.data_ptr(),
                                         pe.data_ptr(), wuv.data_ptr(), scale, causal ? 1 : 0,
                                         (int32_t)key_chunk, out.data_ptr(), ws.data_ptr(), wsb,
                                         current_stream()),
                 "mla_attention_streaming");
    return out;
}

// ------------------------------------------------------------------ per-step ops

void check_contig(const torch::Tensor& t, const char* name) {
    TORCH_CHECK(t.is_contiguous(), "MLA: ", name, " must be contiguous");
}

torch::Tensor step_gemm(torch::Tensor A, torch::Tensor W) {
    check_dim(A, 2, "A", "[M, K]");
    check_dim(W, 2, "W", "[K, N]");
    TORCH_CHECK(A.size(1) == W.size(0), "MLA gemm: A is [M, K] and W must be [K, N]");
    const mla_dtype_t dt = to_mla_dtype(A, "A");
    check_same_dtype(A, W, "W");
    check_contig(A, "A");
    check_contig(W, "W");
    check_device({&A, &W});
    c10::DeviceGuard guard(A.device());
    const int32_t M = (int32_t)A.size(0), K = (int32_t)A.size(1), N = (int32_t)W.size(1);
    auto C = torch::empty({M, N}, A.options().dtype(torch::kFloat32));
    const size_t wsb = mla_gemm_workspace_bytes(dt, M, N, K);
    auto ws = workspace(wsb, A);
    check_status(mla_gemm(dt, A.data_ptr(), W.data_ptr(), C.data_ptr<float>(), M, N, K,
                          ws.data_ptr(), wsb, current_stream()),
                 "gemm");
    return C;
}

torch::Tensor step_rmsnorm(torch::Tensor in, torch::Tensor gain, double eps) {
    check_dim(in, 2, "in", "[M, N]");
    TORCH_CHECK(in.scalar_type() == torch::kFloat32, "MLA rmsnorm: input must be float32");
    TORCH_CHECK(gain.dim() == 1 && gain.size(0) == in.size(1), "MLA rmsnorm: gain must be [N]");
    const mla_dtype_t dt = to_mla_dtype(gain, "gain");
    check_contig(in, "in");
    check_contig(gain, "gain");
    check_device({&in, &gain});
    c10::DeviceGuard guard(in.device());
    auto out = torch::empty(in.sizes(), gain.options());
    check_status(mla_rmsnorm(dt, in.data_ptr<float>(), gain.data_ptr(), out.data_ptr(),
                             (int32_t)in.size(0), (int32_t)in.size(1), eps, current_stream()),
                 "rmsnorm");
    return out;
}

mla_dims_t q_dims(const torch::Tensor& q_raw, int64_t B, int64_t Sq, int64_t H, int64_t nope,
                  int64_t rope) {
    check_dim(q_raw, 2, "q_raw", "[B*Sq, H*(nope+rope)]");
    TORCH_CHECK(q_raw.scalar_type() == torch::kFloat32, "MLA: q_raw must be float32");
    TORCH_CHECK(q_raw.size(0) == B * Sq && q_raw.size(1) == H * (nope + rope),
                "MLA: q_raw must be [B*Sq, H*(nope+rope)] (got ", q_raw.sizes(), ")");
    check_contig(q_raw, "q_raw");
    mla_dims_t d{};
    d.batch = (int32_t)B; d.sq = (int32_t)Sq; d.heads = (int32_t)H; d.nope = (int32_t)nope;
    d.rope = (int32_t)rope;
    d.hidden = 4; d.q_lora = 4;  // unused by the step
    return d;
}

torch::Tensor step_rope(torch::Tensor q_raw, torch::Tensor positions, int64_t B, int64_t Sq,
                        int64_t H, int64_t nope, int64_t rope, torch::ScalarType out_dtype) {
    mla_dims_t d = q_dims(q_raw, B, Sq, H, nope, rope);
    d.kv_rank = 4;
    TORCH_CHECK(positions.dim() == 1 && positions.size(0) == Sq, "MLA rope: positions must be [Sq]");
    const mla_dtype_t dt = to_mla_dtype(torch::empty({0}, torch::TensorOptions().dtype(out_dtype)),
                                        "out_dtype");
    check_device({&q_raw, &positions});
    c10::DeviceGuard guard(q_raw.device());
    auto pos = positions.to(torch::kLong).contiguous();
    auto inv_freq = device_inv_freq(rope, q_raw.device());
    auto out = torch::empty({B, Sq, H, rope}, q_raw.options().dtype(out_dtype));
    check_status(mla_rope(dt, &d, q_raw.data_ptr<float>(), pos.data_ptr<int64_t>(),
                          inv_freq.data_ptr<float>(), out.data_ptr(), current_stream()),
                 "rope");
    return out;
}

torch::Tensor step_absorb(torch::Tensor q_raw, torch::Tensor W_uk, int64_t B, int64_t Sq,
                          int64_t rope) {
    check_dim(W_uk, 3, "W_uk", "[H, nope, kv_rank]");
    const int64_t H = W_uk.size(0), nope = W_uk.size(1), R = W_uk.size(2);
    mla_dims_t d = q_dims(q_raw, B, Sq, H, nope, rope);
    d.kv_rank = (int32_t)R;
    const mla_dtype_t dt = to_mla_dtype(W_uk, "W_uk");
    check_contig(W_uk, "W_uk");
    check_device({&q_raw, &W_uk});
    c10::DeviceGuard guard(q_raw.device());
    auto out = torch::empty({B, Sq, H, R}, W_uk.options());
    check_status(mla_absorb(dt, &d, q_raw.data_ptr<float>(), W_uk.data_ptr(), out.data_ptr(),
                            current_stream()),
                 "absorb");
    return out;
}

std::vector<torch::Tensor> step_scores(torch::Tensor qa, torch::Tensor qr, torch::Tensor ckv,
                                       torch::Tensor pe, double scale, bool causal) {
    mla_dims_t d = attn_dims(qa, qr, ckv, pe, nullptr);
    d.v = 4;
    const mla_dtype_t dt = to_mla_dtype(qa, "q_absorbed");
    check_same_dtype(qa, qr, "q_rope");
    check_same_dtype(qa, ckv, "c_kv");
    check_same_dtype(qa, pe, "pe_cache");
    for (auto* t : {&qa, &qr, &ckv, &pe}) check_contig(*t, "scores input");
    check_device({&qa, &qr, &ckv, &pe});
    c10::DeviceGuard guard(qa.device());
    const int64_t rows = (int64_t)d.batch * d.sq * d.heads;
    const int32_t ld = mla_score_ld(d.sk);
    const int64_t P = (d.sk + mla_score_tile() - 1) / mla_score_tile();
    auto f32 = qa.options().dtype(torch::kFloat32);
    auto p = torch::empty({rows, ld}, f32);
    auto m = torch::empty({rows, P}, f32);
    auto l = torch::empty({rows, P}, f32);
    check_status(mla_scores(dt, &d, qa.data_ptr(), qr.data_ptr(), ckv.data_ptr(), pe.data_ptr(),
                            scale, causal ? 1 : 0, p.data_ptr<float>(), ld, m.data_ptr<float>(),
                            l.data_ptr<float>(), current_stream()),
                 "scores");
    return {p, m, l};
}

std::vector<torch::Tensor> step_combine(torch::Tensor m, torch::Tensor l) {
    check_dim(m, 2, "m_part", "[rows, P]");
    TORCH_CHECK(l.sizes() == m.sizes(), "MLA combine: l_part must match m_part");
    TORCH_CHECK(m.scalar_type() == torch::kFloat32 && l.scalar_type() == torch::kFloat32,
                "MLA combine: partials must be float32");
    check_contig(m, "m_part");
    check_contig(l, "l_part");
    check_device({&m, &l});
    c10::DeviceGuard guard(m.device());
    auto alpha = torch::empty_like(m);
    auto rs = torch::empty({m.size(0)}, m.options());
    check_status(mla_combine(m.data_ptr<float>(), l.data_ptr<float>(), alpha.data_ptr<float>(),
                             rs.data_ptr<float>(), (int32_t)m.size(0), (int32_t)m.size(1),
                             current_stream()),
                 "combine");
    return {alpha, rs};
}

torch::Tensor step_ctx(torch::Tensor p, torch::Tensor alpha, torch::Tensor c_kv, int64_t Sq,
                       int64_t H) {
    check_dim(p, 2, "scores", "[B*Sq*H, ld]");
    check_dim(c_kv, 3, "c_kv", "[B, Sk, kv_rank]");
    const int64_t B = c_kv.size(0), Sk = c_kv.size(1), R = c_kv.size(2);
    TORCH_CHECK(p.size(0) == B * Sq * H, "MLA ctx: scores must have B*Sq*H rows");
    const int64_t P = (Sk + mla_score_tile() - 1) / mla_score_tile();
    TORCH_CHECK(alpha.dim() == 2 && alpha.size(0) == p.size(0) && alpha.size(1) == P,
                "MLA ctx: alpha must be [B*Sq*H, ceil(Sk/tile)]");
    TORCH_CHECK(p.scalar_type() == torch::kFloat32 && alpha.scalar_type() == torch::kFloat32,
                "MLA ctx: scores and alpha must be float32");
    const mla_dtype_t dt = to_mla_dtype(c_kv, "c_kv");
    for (auto* t : {&p, &alpha, &c_kv}) check_contig(*t, "ctx input");
    check_device({&p, &alpha, &c_kv});
    c10::DeviceGuard guard(p.device());
    mla_dims_t d{};
    d.batch = (int32_t)B; d.sq = (int32_t)Sq; d.sk = (int32_t)Sk; d.heads = (int32_t)H;
    d.kv_rank = (int32_t)R; d.rope = 4; d.v = 4;
    auto ctx = torch::empty({B, Sq, H, R}, p.options());
    const size_t wsb = mla_ctx_workspace_bytes(dt, &d);
    auto ws = workspace(wsb, p);
    check_status(mla_ctx(dt, &d, p.data_ptr<float>(), (int32_t)p.size(1), alpha.data_ptr<float>(),
                         c_kv.data_ptr(), ctx.data_ptr<float>(), ws.data_ptr(), wsb,
                         current_stream()),
                 "ctx");
    return ctx;
}

// 3a+3b+3c fused (bf16): [ctx [B, Sq, H, kv_rank], row_sum [B*Sq*H]], float32, with
// ctx / row_sum the softmax-weighted sum of the c_kv rows (the pair shares one per-row
// factor that differs from the per-step path's)
std::vector<torch::Tensor> step_attn_ctx(torch::Tensor qa, torch::Tensor qr, torch::Tensor ckv,
                                         torch::Tensor pe, double scale, bool causal) {
    mla_dims_t d = attn_dims(qa, qr, ckv, pe, nullptr);
    d.v = 4;
    const mla_dtype_t dt = to_mla_dtype(qa, "q_absorbed");
    check_same_dtype(qa, qr, "q_rope");
    check_same_dtype(qa, ckv, "c_kv");
    check_same_dtype(qa, pe, "pe_cache");
    TORCH_CHECK(!causal || d.sk >= d.sq, "MLA: causal attention needs Sk >= Sq");
    for (auto* t : {&qa, &qr, &ckv, &pe}) check_contig(*t, "attn_ctx input");
    check_device({&qa, &qr, &ckv, &pe});
    c10::DeviceGuard guard(qa.device());
    auto f32 = qa.options().dtype(torch::kFloat32);
    auto ctx = torch::empty({d.batch, d.sq, d.heads, d.kv_rank}, f32);
    auto rs = torch::empty({(int64_t)d.batch * d.sq * d.heads}, f32);
    const size_t wsb = mla_attn_ctx_workspace_bytes(dt, &d, causal ? 1 : 0);
    auto ws = workspace(wsb, qa);
    check_status(mla_attn_ctx(dt, &d, qa.data_ptr(), qr.data_ptr(), ckv.data_ptr(), pe.data_ptr(),
                              scale, causal ? 1 : 0, ctx.data_ptr<float>(), rs.data_ptr<float>(),
                              ws.data_ptr(), wsb, current_stream()),
                 "attn_ctx");
    return {ctx, rs};
}

torch::Tensor step_out(torch::Tensor ctx, torch::Tensor row_sum, torch::Tensor W_uv) {
    check_dim(ctx, 4, "ctx", "[B, Sq, H, kv_rank]");
    check_dim(W_uv, 3, "W_uv", "[H, v, kv_rank]");
    const int64_t B = ctx.size(0), Sq = ctx.size(1), H = ctx.size(2), R = ctx.size(3);
    TORCH_CHECK(W_uv.size(0) == H && W_uv.size(2) == R, "MLA out: W_uv must be [H, v, kv_rank]");
    TORCH_CHECK(row_sum.numel() == B * Sq * H, "MLA out: row_sum must have B*Sq*H entries");
    TORCH_CHECK(ctx.scalar_type() == torch::kFloat32 && row_sum.scalar_type() == torch::kFloat32,
                "MLA out: ctx and row_sum must be float32");
    const mla_dtype_t dt = to_mla_dtype(W_uv, "W_uv");
    for (auto* t : {&ctx, &row_sum, &W_uv}) check_contig(*t, "out input");
    check_device({&ctx, &row_sum, &W_uv});
    c10::DeviceGuard guard(ctx.device());
    mla_dims_t d{};
    d.batch = (int32_t)B; d.sq = (int32_t)Sq; d.sk = 1; d.heads = (int32_t)H;
    d.kv_rank = (int32_t)R; d.rope = 4; d.v = (int32_t)W_uv.size(1);
    auto out = torch::empty({B, Sq, H, d.v}, W_uv.options());
    const size_t wsb = mla_out_workspace_bytes(dt, &d);
    auto ws = workspace(wsb, ctx);
    check_status(mla_out(dt, &d, ctx.data_ptr<float>(), row_sum.data_ptr<float>(), W_uv.data_ptr(),
                         out.data_ptr(), ws.data_ptr(), wsb, current_stream()),
                 "out");
    return out;
}

// ------------------------------------------------------------------ ragged, paged cache

// Shapes of a paged call: q [B, Sq, H, ·], pools [pages, page_size, ·], block_table
// [B, max_pages] int32, seq_lens [B] int32.
mla_dims_t paged_dims(const torch::Tensor& qa, const torch::Tensor& qr, const torch::Tensor& ckv,
                      const torch::Tensor& pe, const torch::Tensor& table,
                      const torch::Tensor* seq_lens, const torch::Tensor* W_uv, int64_t* page) {
    check_dim(qa, 4, "q_absorbed", "[B, Sq, H, kv_rank]");
    check_dim(qr, 4, "q_rope", "[B, Sq, H, rope]");
    check_dim(ckv, 3, "c_kv_pages", "[num_pages, page_size, kv_rank]");
    check_dim(pe, 3, "pe_pages", "[num_pages, page_size, rope]");
    check_dim(table, 2, "block_table", "[B, max_pages]");
    const int64_t B = qa.size(0), Sq = qa.size(1), H = qa.size(2), R = qa.size(3);
    const int64_t D = qr.size(3);
    TORCH_CHECK(qr.size(0) == B && qr.size(1) == Sq && qr.size(2) == H,
                "q_rope must be [B, Sq, H, rope] matching q_absorbed (got ", qr.sizes(), ")");
    TORCH_CHECK(ckv.size(2) == R, "c_kv_pages must be [num_pages, page_size, kv_rank] (got ",
                ckv.sizes(), ")");
    TORCH_CHECK(pe.size(0) == ckv.size(0) && pe.size(1) == ckv.size(1) && pe.size(2) == D,
                "pe_pages must be [num_pages, page_size, rope] matching c_kv_pages (got ",
                pe.sizes(), ")");
    TORCH_CHECK(table.size(0) == B, "block_table must be [B, max_pages] (got ", table.sizes(), ")");
    TORCH_CHECK(table.scalar_type() == torch::kInt32, "block_table must be int32");
    if (seq_lens) {
        TORCH_CHECK(seq_lens->dim() == 1 && seq_lens->size(0) == B,
                    "seq_lens must be a 1-D tensor of length B (got ", seq_lens->sizes(), ")");
        TORCH_CHECK(seq_lens->scalar_type() == torch::kInt32, "seq_lens must be int32");
    }
    *page = ckv.size(1);
    mla_dims_t d{};
    d.batch = (int32_t)B; d.sq = (int32_t)Sq; d.heads = (int32_t)H;
    d.kv_rank = (int32_t)R; d.rope = (int32_t)D;
    TORCH_CHECK(table.size(1) * *page < INT32_MAX, "MLA: block_table spans too many keys");
    d.sk = (int32_t)(table.size(1) * *page);
    if (W_uv) {
        check_dim(*W_uv, 3, "W_uv", "[H, v, kv_rank]");
        TORCH_CHECK(W_uv->size(0) == H && W_uv->size(2) == R,
                    "W_uv must be [H, v, kv_rank] (got ", W_uv->sizes(), ")");
        d.v = (int32_t)W_uv->size(1);
    }
    return d;
}

// Attention over a paged, ragged cache: sequence b attends to its first seq_lens[b] keys,
// found through its row of block_table.
torch::Tensor op_mla_attention_paged(torch::Tensor q_absorbed, torch::Tensor q_rope,
                                     torch::Tensor c_kv_pages, torch::Tensor pe_pages,
                                     torch::Tensor block_table, torch::Tensor seq_lens,
                                     torch::Tensor W_uv, double scale, bool causal) {
    int64_t page = 0;
    mla_dims_t d = paged_dims(q_absorbed, q_rope, c_kv_pages, pe_pages, block_table, &seq_lens,
                              &W_uv, &page);
    const mla_dtype_t dt = to_mla_dtype(q_absorbed, "q_absorbed");
    check_same_dtype(q_absorbed, q_rope, "q_rope");
    check_same_dtype(q_absorbed, c_kv_pages, "c_kv_pages");
    check_same_dtype(q_absorbed, pe_pages, "pe_pages");
    check_same_dtype(q_absorbed, W_uv, "W_uv");
    check_device({&q_absorbed, &q_rope, &c_kv_pages, &pe_pages, &block_table, &seq_lens, &W_uv});

    c10::DeviceGuard guard(q_absorbed.device());
    auto qa = q_absorbed.contiguous();
    auto qr = q_rope.contiguous();
    auto ck = c_kv_pages.contiguous();
    auto pe = pe_pages.contiguous();
    auto tab = block_table.contiguous();
    auto lens = seq_lens.contiguous();
    auto wuv = W_uv.contiguous();
    auto out = torch::empty({d.batch, d.sq, d.heads, d.v}, qa.options());
    const size_t wsb = mla_attention_paged_workspace_bytes(dt, &d, causal ? 1 : 0, (int32_t)page);
    auto ws = workspace(wsb, qa);
    check_status(mla_attention_paged(dt, &d, qa.data_ptr(), qr.data_ptr(), ck.data_ptr(),
                                     pe.data_ptr(), tab.data_ptr<int32_t>(),
                                     lens.data_ptr<int32_t>(), (int32_t)page, wuv.data_ptr(),
                                     scale, causal ? 1 : 0, out.data_ptr(), ws.data_ptr(), wsb,
                                     current_stream()),
                 "mla_attention_paged");
    return out;
}

// Attention over a paged fp8 cache: the pools hold e4m3 codes (torch.float8_e4m3fn or
// their bytes as uint8) of value / kv_scale; sequence b attends to its first seq_lens[b]
// keys through its row of block_table; the queries, W_uv and the output are bf16.
torch::Tensor op_mla_attention_paged_fp8kv(torch::Tensor q_absorbed, torch::Tensor q_rope,
                                           torch::Tensor c_kv_pages, torch::Tensor pe_pages,
                                           torch::Tensor block_table, torch::Tensor seq_lens,
                                           double kv_scale, torch::Tensor W_uv, double scale,
                                           bool causal) {
    int64_t page = 0;
    mla_dims_t d = paged_dims(q_absorbed, q_rope, c_kv_pages, pe_pages, block_table, &seq_lens,
                              &W_uv, &page);
    TORCH_CHECK(q_absorbed.scalar_type() == torch::kBFloat16,
                "MLA: an fp8 cache is read with bfloat16 queries (q_absorbed has dtype ",
                q_absorbed.scalar_type(), ")");
    check_same_dtype(q_absorbed, q_rope, "q_rope");
    check_same_dtype(q_absorbed, W_uv, "W_uv");
    for (const torch::Tensor* t : {&c_kv_pages, &pe_pages})
        TORCH_CHECK(t->scalar_type() == torch::kFloat8_e4m3fn || t->scalar_type() == torch::kByte,
                    "MLA: the fp8 cache must be float8_e4m3fn or uint8 codes (got ",
                    t->scalar_type(), ")");
    check_device({&q_absorbed, &q_rope, &c_kv_pages, &pe_pages, &block_table, &seq_lens, &W_uv});

    c10::DeviceGuard guard(q_absorbed.device());
    auto qa = q_absorbed.contiguous();
    auto qr = q_rope.contiguous();
    auto ck = c_kv_pages.contiguous();
    auto pe = pe_pages.contiguous();
    auto tab = block_table.contiguous();
    auto lens = seq_lens.contiguous();
    auto wuv = W_uv.contiguous();
    auto out = torch::empty({d.batch, d.sq, d.heads, d.v}, qa.options());
    const size_t wsb = mla_attention_paged_fp8kv_workspace_bytes(MLA_DTYPE_BF16, &d, causal ? 1 : 0,
                                                                 (int32_t)page);
    auto ws = workspace(wsb, qa);
    check_status(mla_attention_paged_fp8kv(MLA_DTYPE_BF16, &d, qa.data_ptr(), qr.data_ptr(),
                                           ck.data_ptr(), pe.data_ptr(), tab.data_ptr<int32_t>(),
                                           lens.data_ptr<int32_t>(), (int32_t)page, (float)kv_scale,
                                           wuv.data_ptr(), scale, causal ? 1 : 0, out.data_ptr(),
                                           ws.data_ptr(), wsb, current_stream()),
                 "mla_attention_paged_fp8kv");
    return out;
}

// The work list the fused paged pass builds from seq_lens (int32, layout in mla.h).
torch::Tensor op_attention_work_list(torch::Tensor seq_lens, int64_t Sq, int64_t H, int64_t Sk,
                                     torch::ScalarType dtype) {
    TORCH_CHECK(seq_lens.dim() == 1 && seq_lens.scalar_type() == torch::kInt32,
                "seq_lens must be a 1-D int32 tensor (got ", seq_lens.sizes(), ")");
    TORCH_CHECK(Sq > 0 && H > 0 && Sk > 0 && Sk < INT32_MAX, "MLA: Sq, H and Sk must be positive");
    const mla_dtype_t dt = to_mla_dtype(torch::empty({0}, torch::TensorOptions().dtype(dtype)),
                                        "dtype");
    check_device({&seq_lens});
    c10::DeviceGuard guard(seq_lens.device());
    auto lens = seq_lens.contiguous();
    mla_dims_t d{};
    d.batch = (int32_t)lens.size(0); d.sq = (int32_t)Sq; d.heads = (int32_t)H; d.sk = (int32_t)Sk;
    const int32_t n = mla_attention_work_list_ints(dt, &d);
    TORCH_CHECK(n > 0, "MLA: invalid work-list dims");
    auto wl = torch::empty({n}, lens.options());
    check_status(mla_attention_work_list(dt, &d, lens.data_ptr<int32_t>(), wl.data_ptr<int32_t>(),
                                         n, current_stream()),
                 "attention_work_list");
    return wl;
}

// KV-cache append into the paged cache: token (b, s) goes to slot positions[b, s] of
// sequence b (pool row through block_table).
void op_kv_append_paged(torch::Tensor x, torch::Tensor W_kv_a, torch::Tensor kv_norm_w,
                        torch::Tensor positions, torch::Tensor block_table,
                        torch::Tensor c_kv_pages, torch::Tensor pe_pages, double eps) {
    check_dim(x, 3, "x", "[B, Sq, hidden]");
    check_dim(W_kv_a, 2, "W_kv_a", "[hidden, kv_rank + rope]");
    check_dim(c_kv_pages, 3, "c_kv_pages", "[num_pages, page_size, kv_rank]");
    check_dim(pe_pages, 3, "pe_pages", "[num_pages, page_size, rope]");
    check_dim(block_table, 2, "block_table", "[B, max_pages]");
    const int64_t B = x.size(0), Sq = x.size(1), hidden = x.size(2);
    const int64_t page = c_kv_pages.size(1), R = c_kv_pages.size(2), D = pe_pages.size(2);
    TORCH_CHECK(W_kv_a.size(0) == hidden && W_kv_a.size(1) == R + D,
                "W_kv_a must be [hidden, kv_rank + rope] (got ", W_kv_a.sizes(), ")");
    TORCH_CHECK(pe_pages.size(0) == c_kv_pages.size(0) && pe_pages.size(1) == page,
                "pe_pages must be [num_pages, page_size, rope] matching c_kv_pages");
    TORCH_CHECK(block_table.size(0) == B && block_table.scalar_type() == torch::kInt32,
                "block_table must be an int32 [B, max_pages] tensor");
    TORCH_CHECK(kv_norm_w.dim() == 1 && kv_norm_w.size(0) == R,
                "kv_norm_w must be a 1-D tensor of length kv_rank (got ", kv_norm_w.sizes(), ")");
    TORCH_CHECK(positions.dim() == 2 && positions.size(0) == B && positions.size(1) == Sq,
                "positions must be [B, Sq] (got ", positions.sizes(), ")");
    TORCH_CHECK(!positions.is_floating_point() && !positions.is_complex(),
                "positions must be an integer tensor");
    TORCH_CHECK(D > 0 && D % 2 == 0, "MLA: the rope width must be positive and even");
    TORCH_CHECK(c_kv_pages.is_contiguous() && pe_pages.is_contiguous(),
                "MLA: c_kv_pages and pe_pages are updated in place and must be contiguous");
    const mla_dtype_t dt = to_mla_dtype(x, "x");
    check_same_dtype(x, W_kv_a, "W_kv_a");
    check_same_dtype(x, kv_norm_w, "kv_norm_w");
    check_same_dtype(x, c_kv_pages, "c_kv_pages");
    check_same_dtype(x, pe_pages, "pe_pages");
    check_device({&x, &W_kv_a, &kv_norm_w, &positions, &block_table, &c_kv_pages, &pe_pages});

    c10::DeviceGuard guard(x.device());
    auto xc = x.contiguous();
    auto wa = W_kv_a.contiguous();
    auto g = kv_norm_w.contiguous();
    auto pos = positions.to(torch::kLong).contiguous();
    auto tab = block_table.contiguous();
    auto inv_freq = device_inv_freq(D, x.device());
    mla_dims_t d{};
    d.batch = (int32_t)B; d.sq = (int32_t)Sq; d.hidden = (int32_t)hidden;
    d.kv_rank = (int32_t)R; d.rope = (int32_t)D;
    TORCH_CHECK(block_table.size(1) * page < INT32_MAX, "MLA: block_table spans too many keys");
    d.sk = (int32_t)(block_table.size(1) * page);
    const size_t wsb = mla_kv_append_workspace_bytes(dt, &d);
    auto ws = workspace(wsb, x);
    check_status(mla_kv_append_paged(dt, &d, xc.data_ptr(), wa.data_ptr(), g.data_ptr(),
                                     pos.data_ptr<int64_t>(), inv_freq.data_ptr<float>(), eps,
                                     tab.data_ptr<int32_t>(), (int32_t)page, c_kv_pages.data_ptr(),
                                     pe_pages.data_ptr(), ws.data_ptr(), wsb, current_stream()),
                 "kv_append_paged");
}

// ------------------------------------------------------------------ neighbours of the path

// Weight prep once at load: the W_uk / W_uv halves of wkv_b as contiguous tensors.
std::vector<torch::Tensor> op_split_wkv_b(torch::Tensor wkv_b, int64_t nope_dim) {
    check_dim(wkv_b, 3, "wkv_b", "[H, nope + v, kv_rank]");
    const int64_t H = wkv_b.size(0), rows = wkv_b.size(1), R = wkv_b.size(2);
    TORCH_CHECK(nope_dim > 0 && nope_dim < rows, "MLA: nope_dim must lie in (0, ", rows, ")");
    const mla_dtype_t dt = to_mla_dtype(wkv_b, "wkv_b");
    check_device({&wkv_b});
    c10::DeviceGuard guard(wkv_b.device());
    auto w = wkv_b.contiguous();
    mla_dims_t d{};
    d.heads = (int32_t)H; d.nope = (int32_t)nope_dim; d.v = (int32_t)(rows - nope_dim);
    d.kv_rank = (int32_t)R;
    auto uk = torch::empty({H, nope_dim, R}, w.options());
    auto uv = torch::empty({H, rows - nope_dim, R}, w.options());
    check_status(mla_split_wkv_b(dt, &d, w.data_ptr(), uk.data_ptr(), uv.data_ptr(),
                                 current_stream()),
                 "split_wkv_b");
    return {uk, uv};
}

// KV-cache append: writes rows [start_row, start_row + Sq) of c_kv and pe_cache in place.
void op_kv_append(torch::Tensor x, torch::Tensor W_kv_a, torch::Tensor kv_norm_w,
                  torch::Tensor positions, torch::Tensor c_kv, torch::Tensor pe_cache,
                  int64_t start_row, double eps) {
    check_dim(x, 3, "x", "[B, Sq, hidden]");
    check_dim(W_kv_a, 2, "W_kv_a", "[hidden, kv_rank + rope]");
    check_dim(c_kv, 3, "c_kv", "[B, cache_rows, kv_rank]");
    check_dim(pe_cache, 3, "pe_cache", "[B, cache_rows, rope]");
    const int64_t B = x.size(0), Sq = x.size(1), hidden = x.size(2);
    const int64_t rows = c_kv.size(1), R = c_kv.size(2), D = pe_cache.size(2);
    TORCH_CHECK(W_kv_a.size(0) == hidden && W_kv_a.size(1) == R + D,
                "W_kv_a must be [hidden, kv_rank + rope] (got ", W_kv_a.sizes(), ")");
    TORCH_CHECK(c_kv.size(0) == B && pe_cache.size(0) == B && pe_cache.size(1) == rows,
                "c_kv [B, cache_rows, kv_rank] and pe_cache [B, cache_rows, rope] must agree "
                "with x (got ", c_kv.sizes(), " and ", pe_cache.sizes(), ")");
    TORCH_CHECK(kv_norm_w.dim() == 1 && kv_norm_w.size(0) == R,
                "kv_norm_w must be a 1-D tensor of length kv_rank (got ", kv_norm_w.sizes(), ")");
    TORCH_CHECK(positions.dim() == 1 && positions.size(0) == Sq,
                "positions must be a 1-D tensor of length Sq (got ", positions.sizes(), ")");
    TORCH_CHECK(!positions.is_floating_point() && !positions.is_complex(),
                "positions must be an integer tensor");
    TORCH_CHECK(D > 0 && D % 2 == 0, "MLA: the rope width must be positive and even");
    TORCH_CHECK(c_kv.is_contiguous() && pe_cache.is_contiguous(),
                "MLA: c_kv and pe_cache are updated in place and must be contiguous");
    const mla_dtype_t dt = to_mla_dtype(x, "x");
    check_same_dtype(x, W_kv_a, "W_kv_a");
    check_same_dtype(x, kv_norm_w, "kv_norm_w");
    check_same_dtype(x, c_kv, "c_kv");
    check_same_dtype(x, pe_cache, "pe_cache");
    check_device({&x, &W_kv_a, &kv_norm_w, &positions, &c_kv, &pe_cache});

    c10::DeviceGuard guard(x.device());
    auto xc = x.contiguous();
    auto wa = W_kv_a.contiguous();
    auto g = kv_norm_w.contiguous();
    auto pos = positions.to(torch::kLong).contiguous();
    auto inv_freq = device_inv_freq(D, x.device());
    mla_dims_t d{};
    d.batch = (int32_t)B; d.sq = (int32_t)Sq; d.hidden = (int32_t)hidden;
    d.kv_rank = (int32_t)R; d.rope = (int32_t)D;
    TORCH_CHECK(start_row >= 0 && rows < INT32_MAX && start_row + Sq <= rows,
                "MLA: start_row + Sq must not exceed the cache rows");
    const size_t wsb = mla_kv_append_workspace_bytes(dt, &d);
    auto ws = workspace(wsb, x);
    check_status(mla_kv_append(dt, &d, xc.data_ptr(), wa.data_ptr(), g.data_ptr(),
                               pos.data_ptr<int64_t>(), inv_freq.data_ptr<float>(), eps,
                               (int32_t)start_row, (int32_t)rows, c_kv.data_ptr(),
                               pe_cache.data_ptr(), ws.data_ptr(), wsb, current_stream()),
                 "kv_append");
}

// Output projection wo: [B, Sq, H, v] @ [H*v, hidden] -> [B, Sq, hidden].
torch::Tensor op_o_proj(torch::Tensor attn, torch::Tensor W_o) {
    check_dim(attn, 4, "attn", "[B, Sq, H, v]");
    check_dim(W_o, 2, "W_o", "[H*v, hidden]");
    const int64_t B = attn.size(0), Sq = attn.size(1), H = attn.size(2), v = attn.size(3);
    const int64_t hidden = W_o.size(1);
    TORCH_CHECK(W_o.size(0) == H * v, "W_o must be [H*v, hidden] (got ", W_o.sizes(), ")");
    const mla_dtype_t dt = to_mla_dtype(attn, "attn");
    check_same_dtype(attn, W_o, "W_o");
    check_device({&attn, &W_o});
    c10::DeviceGuard guard(attn.device());
    auto a = attn.contiguous();
    auto w = W_o.contiguous();
    mla_dims_t d{};
    d.batch = (int32_t)B; d.sq = (int32_t)Sq; d.heads = (int32_t)H; d.v = (int32_t)v;
    d.hidden = (int32_t)hidden;
    auto out = torch::empty({B, Sq, hidden}, a.options());
    const size_t wsb = mla_o_proj_workspace_bytes(dt, &d);
    auto ws = workspace(wsb, a);
    check_status(mla_o_proj(dt, &d, a.data_ptr(), w.data_ptr(), out.data_ptr(), ws.data_ptr(),
                            wsb, current_stream()),
                 "o_proj");
    return out;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "MI355X (gfx950) absorbed MLA layer: drop-in for the reference's mla_custom_cuda";
    m.def("q_absorbed", &op_q_absorbed,
          "Q path 2a1 -> 2a-n -> 2a2 -> 2b -> 2c: returns [q_absorbed, q_rope]",
          py::arg("x"), py::arg("W_q_a"), py::arg("q_norm_w"), py::arg("W_q_b"), py::arg("W_uk"),
          py::arg("positions"), py::arg("nope_dim"), py::arg("rope_dim"), py::arg("eps"));
    m.def("mla_attention_fp8kv", &op_mla_attention_fp8kv,
          "Attention over an fp8 e4m3 cache (codes of value / kv_scale; bf16 queries and "
          "output): returns out [B, Sq, H, v]",
          py::arg("q_absorbed"), py::arg("q_rope"), py::arg("c_kv"), py::arg("pe_cache"),
          py::arg("kv_scale"), py::arg("W_uv"), py::arg("scale"), py::arg("causal") = false);
    m.def("fp8_dequantize", &op_fp8_dequantize,
          "e4m3 codes -> float32 code * scale, with the fused attention's conversion",
          py::arg("codes"), py::arg("scale") = 1.0);
    m.def("mla_attention", &op_mla_attention,
          "Absorbed attention 3a -> 3b -> 3c -> 3d: returns out [B, Sq, H, v]",
          py::arg("q_absorbed"), py::arg("q_rope"), py::arg("c_kv"), py::arg("pe_cache"),
          py::arg("W_uv"), py::arg("scale"), py::arg("causal") = false);
    m.def("mla_attention_streaming", &op_mla_attention_streaming,
          "Attention with keys in bounded chunks (online-softmax merge): returns out [B, Sq, H, v]",
          py::arg("q_absorbed"), py::arg("q_rope"), py::arg("c_kv"), py::arg("pe_cache"),
          py::arg("W_uv"), py::arg("scale"), py::arg("causal") = false, py::arg("key_chunk") = 0);
    m.def("rope_inv_freq",
          [](int64_t rope, bool float64) {
              return rope_inv_freq(rope, float64 ? torch::kFloat64 : torch::kFloat32);
          },
          "RoPE inverse-frequency table q_absorbed passes to the library (float32, or float64 "
          "for float64 inputs)", py::arg("rope"), py::arg("float64") = false);
    m.def("gemm", &step_gemm, "2a1/2a2: float32 C = A @ W", py::arg("A"), py::arg("W"));
    m.def("rmsnorm", &step_rmsnorm, "2a-n", py::arg("input"), py::arg("gain"), py::arg("eps"));
    m.def("rope", &step_rope, "2b", py::arg("q_raw"), py::arg("positions"), py::arg("B"),
          py::arg("Sq"), py::arg("H"), py::arg("nope"), py::arg("rope"), py::arg("out_dtype"));
    m.def("absorb", &step_absorb, "2c", py::arg("q_raw"), py::arg("W_uk"), py::arg("B"),
          py::arg("Sq"), py::arg("rope"));
    m.def("scores", &step_scores, "3a: returns [scores, m_part, l_part]", py::arg("q_absorbed"),
          py::arg("q_rope"), py::arg("c_kv"), py::arg("pe_cache"), py::arg("scale"),
          py::arg("causal") = false);
    m.def("combine", &step_combine, "3b: returns [alpha, row_sum]", py::arg("m_part"),
          py::arg("l_part"));
    m.def("ctx", &step_ctx, "3c: unnormalised ctx", py::arg("scores"), py::arg("alpha"),
          py::arg("c_kv"), py::arg("Sq"), py::arg("H"));
    m.def("out", &step_out, "3d", py::arg("ctx"), py::arg("row_sum"), py::arg("W_uv"));
    m.def("attn_ctx", &step_attn_ctx, "3a+3b+3c fused (bf16 or fp32): returns [ctx, row_sum]",
          py::arg("q_absorbed"), py::arg("q_rope"), py::arg("c_kv"), py::arg("pe_cache"),
          py::arg("scale"), py::arg("causal") = false);
    m.def("score_tile", []() { return mla_score_tile(); });
    m.def("score_ld", [](int32_t sk) { return mla_score_ld(sk); });
    m.def("version", []() { return std::string(mla_version()); });
    m.def("split_wkv_b", &op_split_wkv_b,
          "Weight prep: contiguous [W_uk, W_uv] halves of wkv_b [H, nope + v, kv_rank]",
          py::arg("wkv_b"), py::arg("nope_dim"));
    m.def("kv_append", &op_kv_append,
          "KV-cache append in place: c_kv rows = RMSNorm((x @ W_kv_a)[..., :kv_rank]), "
          "pe_cache rows = RoPE((x @ W_kv_a)[..., kv_rank:])",
          py::arg("x"), py::arg("W_kv_a"), py::arg("kv_norm_w"), py::arg("positions"),
          py::arg("c_kv"), py::arg("pe_cache"), py::arg("start_row"), py::arg("eps"));
    m.def("o_proj", &op_o_proj, "Output projection: [B, Sq, H, v] @ W_o [H*v, hidden]",
          py::arg("attn"), py::arg("W_o"));
    m.def("mla_attention_paged", &op_mla_attention_paged,
          "Attention over a paged, ragged KV cache: returns out [B, Sq, H, v]",
          py::arg("q_absorbed"), py::arg("q_rope"), py::arg("c_kv_pages"), py::arg("pe_pages"),
          py::arg("block_table"), py::arg("seq_lens"), py::arg("W_uv"), py::arg("scale"),
          py::arg("causal") = false);
    m.def("mla_attention_paged_fp8kv", &op_mla_attention_paged_fp8kv,
          "Attention over a paged fp8 e4m3 cache (codes of value / kv_scale; bf16 queries and "
          "output): returns out [B, Sq, H, v]",
          py::arg("q_absorbed"), py::arg("q_rope"), py::arg("c_kv_pages"), py::arg("pe_pages"),
          py::arg("block_table"), py::arg("seq_lens"), py::arg("kv_scale"), py::arg("W_uv"),
          py::arg("scale"), py::arg("causal") = false);
    m.def("attention_work_list", &op_attention_work_list,
          "The fused paged pass's device-built work list for seq_lens (int32)",
          py::arg("seq_lens"), py::arg("Sq"), py::arg("H"), py::arg("Sk"), py::arg("dtype"));
    m.def("kv_append_paged", &op_kv_append_paged,
          "KV-cache append into a paged cache: token (b, s) to slot positions[b, s]",
          py::arg("x"), py::arg("W_kv_a"), py::arg("kv_norm_w"), py::arg("positions"),
          py::arg("block_table"), py::arg("c_kv_pages"), py::arg("pe_pages"), py::arg("eps"));
}
