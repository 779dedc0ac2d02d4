// PyTorch-ROCm operator library of the engine: the `bcjr` torch operators,
// registered from C++ (TORCH_LIBRARY) with a HIP-device kernel (PyTorch-ROCm
// dispatches HIP tensors under the CUDA key) and a Meta kernel each, over the
// C ABI of libbcjr_hip.so (include/bcjr_hip.h).  Outputs and workspace come
// from torch's caching allocator; launches go on the current stream.  No host
// synchronisation, so every operator can be captured into a HIP graph and
// traced by torch.compile.
//
// The operators replace the compute behind the reference's node and helpers
// (file:line into the reference repository):
//   bcjr::forward / bcjr::backward   the BCJR node, src/bcjr/forward_backward.py:190-232
//                                    and its analytic backward, src/bcjr/bcjr_monolithic.py:192-243
//   bcjr::forward_internals           return_internals=True, forward_backward.py:230-231
//   bcjr::forward_entropy             the P-materialising body of entropy_diagnostic,
//                                    src/bcjr/anneal.py:143-184
//   bcjr::viterbi                     viterbi_encode_v_batched_cuda, src/viterbi/cuda_kernel.py:166-220
//                                    (constrained form: src/viterbi/encode.py:328-389)
//   bcjr::decode                      viterbi_decode_v, src/viterbi/encode.py:310-325
//   bcjr::viterbi_trace               viterbi_encode_v(return_trace=True), src/viterbi/encode.py:250-307
//   bcjr::dequant                     dequant_target before the inverse RHT,
//                                    src/quantize/serialize.py:56-107
//   bcjr::codebook                    src/codes/ref.py:33-41,76-91, src/qat/ste.py:376-392
//   bcjr::hadamard                    fast_hadamard_transform.hadamard_transform
//   bcjr::rht / bcjr::rht_batched     apply_rht_gpu / apply_inverse_rht_gpu, src/qat/ste.py:113-135
//
// Codebook resolution (recognising a plain table as 1MAD / 3INST / HYB) and the
// autograd formulas stay in the Python package; these operators take the
// resolved code, its LUT or table, and L, k, V, Q.
#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <c10/core/DeviceGuard.h>
#include <torch/library.h>

#include <optional>
#include <tuple>

#include "../../include/bcjr_hip.h"

namespace {

using at::Tensor;

// A failed C ABI call: a RuntimeError whose message starts with "bcjr status
// <n>:" (the Python package re-raises it as BcjrError with that status).
void check(int status, const char* what) {
  if (status != BCJR_OK)
    TORCH_CHECK(false, "bcjr status ", status, ": ", what, " failed: ", bcjr_strerror(status), ": ",
                bcjr_last_error());
}

hipStream_t stream_of(const Tensor& t) {
  return at::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream();
}

bcjr_problem problem(int64_t L, int64_t k, int64_t V, int64_t B, int64_t N, int64_t code, int64_t Q,
                     bool t_per_seq) {
  bcjr_problem p;
  p.L = (int)L;
  p.k = (int)k;
  p.V = (int)V;
  p.B = B;
  p.N = N;
  p.code = (int)code;
  p.Q = (int)Q;
  p.t_per_seq = t_per_seq ? 1 : 0;
  return p;
}

const float* fptr(const std::optional<Tensor>& t) { return t ? t->data_ptr<float>() : nullptr; }

void same_device(const Tensor& ref, const std::optional<Tensor>& t, const char* name) {
  if (t) TORCH_CHECK(t->device() == ref.device(), name, " is on ", t->device(), " but the launch runs on ", ref.device());
}

Tensor as_f32(const Tensor& t) { return t.to(at::kFloat).contiguous(); }

std::optional<Tensor> as_f32(const std::optional<Tensor>& t) {
  if (!t) return std::nullopt;
  return as_f32(*t);
}

// (B, N, V) float32 sequences, contiguous.
Tensor sequences(const Tensor& seq, int64_t V) {
  TORCH_CHECK(seq.dim() == 3 && seq.size(2) == V, "sequences must be (B, N, V=", V, "); got ", seq.sizes());
  return as_f32(seq);
}

// T as float32 with 1 or B values; returns (T, one value per sequence).
std::pair<Tensor, bool> temperature(const Tensor& seq, const Tensor& T, int64_t B) {
  TORCH_CHECK(T.device() == seq.device(), "T is on ", T.device(), " but the launch runs on ", seq.device());
  Tensor t = as_f32(T.reshape({-1}));
  TORCH_CHECK(t.numel() == 1 || t.numel() == B, "T has ", t.numel(), " values; expected 1 or B=", B);
  return {t, t.numel() != 1};
}

Tensor workspace(const bcjr_problem& p, int op, const Tensor& like) {
  size_t bytes = 0;
  check(bcjr_workspace_bytes(&p, op, &bytes), "bcjr_workspace_bytes");
  return at::empty({(int64_t)std::max<size_t>(bytes, 1)}, like.options().dtype(at::kByte));
}

// ------------------------------------------------------------------ soft path

std::tuple<Tensor, Tensor> forward_hip(const Tensor& seq_in, const Tensor& T, const std::optional<Tensor>& table_in,
                                       int64_t L, int64_t k, int64_t V, int64_t code, int64_t Q) {
  const c10::OptionalDeviceGuard guard(at::device_of(seq_in));
  const Tensor seq = sequences(seq_in, V);
  same_device(seq, table_in, "codebook_or_lut");
  const auto table = as_f32(table_in);
  const int64_t B = seq.size(0), N = seq.size(1);
  auto [Tt, per] = temperature(seq, T, B);
  Tensor soft = at::empty_like(seq), logZ = at::empty({B}, seq.options());
  if (B == 0) return {soft, logZ};
  const bcjr_problem p = problem(L, k, V, B, N, code, Q, per);
  Tensor ws = workspace(p, BCJR_OP_FORWARD, seq);
  check(bcjr_forward(&p, seq.data_ptr<float>(), Tt.data_ptr<float>(), fptr(table), soft.data_ptr<float>(),
                     logZ.data_ptr<float>(), ws.data_ptr(), (size_t)ws.numel(), stream_of(seq)),
        "bcjr_forward");
  return {soft, logZ};
}

std::tuple<Tensor, Tensor> forward_meta(const Tensor& seq, const Tensor& T, const std::optional<Tensor>& table,
                                        int64_t L, int64_t k, int64_t V, int64_t code, int64_t Q) {
  TORCH_CHECK(seq.dim() == 3 && seq.size(2) == V, "sequences must be (B, N, V=", V, "); got ", seq.sizes());
  return {at::empty(seq.sizes(), seq.options().dtype(at::kFloat)), at::empty({seq.size(0)}, seq.options().dtype(at::kFloat))};
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> forward_internals_hip(
    const Tensor& seq_in, const Tensor& T, const std::optional<Tensor>& table_in, int64_t L, int64_t k, int64_t V,
    int64_t code, int64_t Q) {
  const c10::OptionalDeviceGuard guard(at::device_of(seq_in));
  const Tensor seq = sequences(seq_in, V);
  same_device(seq, table_in, "codebook_or_lut");
  const auto table = as_f32(table_in);
  const int64_t B = seq.size(0), N = seq.size(1), S = int64_t(1) << L;
  auto [Tt, per] = temperature(seq, T, B);
  Tensor soft = at::empty_like(seq), logZ = at::empty({B}, seq.options());
  Tensor P = at::empty({B, N, S}, seq.options()), la = at::empty_like(P), lb = at::empty_like(P);
  if (B == 0) return {soft, logZ, P, la, lb};
  const bcjr_problem p = problem(L, k, V, B, N, code, Q, per);
  Tensor ws = workspace(p, BCJR_OP_FORWARD, seq);
  check(bcjr_forward_internals(&p, seq.data_ptr<float>(), Tt.data_ptr<float>(), fptr(table), soft.data_ptr<float>(),
                               logZ.data_ptr<float>(), P.data_ptr<float>(), la.data_ptr<float>(),
                               lb.data_ptr<float>(), ws.data_ptr(), (size_t)ws.numel(), stream_of(seq)),
        "bcjr_forward_internals");
  return {soft, logZ, P, la, lb};
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> forward_internals_meta(
    const Tensor& seq, const Tensor& T, const std::optional<Tensor>& table, int64_t L, int64_t k, int64_t V,
    int64_t code, int64_t Q) {
  const auto o = seq.options().dtype(at::kFloat);
  const int64_t B = seq.size(0), N = seq.size(1), S = int64_t(1) << L;
  Tensor P = at::empty({B, N, S}, o);
  return {at::empty(seq.sizes(), o), at::empty({B}, o), P, at::empty({B, N, S}, o), at::empty({B, N, S}, o)};
}

std::tuple<Tensor, Tensor, Tensor> forward_entropy_hip(const Tensor& seq_in, const Tensor& T,
                                                       const std::optional<Tensor>& table_in, int64_t L, int64_t k,
                                                       int64_t V, int64_t code, int64_t Q) {
  const c10::OptionalDeviceGuard guard(at::device_of(seq_in));
  const Tensor seq = sequences(seq_in, V);
  same_device(seq, table_in, "codebook_or_lut");
  const auto table = as_f32(table_in);
  const int64_t B = seq.size(0), N = seq.size(1);
  auto [Tt, per] = temperature(seq, T, B);
  Tensor soft = at::empty_like(seq), logZ = at::empty({B}, seq.options()), H = at::empty({B, N}, seq.options());
  if (B == 0) return {soft, logZ, H};
  const bcjr_problem p = problem(L, k, V, B, N, code, Q, per);
  Tensor ws = workspace(p, BCJR_OP_FORWARD, seq);
  check(bcjr_forward_entropy(&p, seq.data_ptr<float>(), Tt.data_ptr<float>(), fptr(table), soft.data_ptr<float>(),
                             logZ.data_ptr<float>(), H.data_ptr<float>(), ws.data_ptr(), (size_t)ws.numel(),
                             stream_of(seq)),
        "bcjr_forward_entropy");
  return {soft, logZ, H};
}

std::tuple<Tensor, Tensor, Tensor> forward_entropy_meta(const Tensor& seq, const Tensor& T,
                                                        const std::optional<Tensor>& table, int64_t L, int64_t k,
                                                        int64_t V, int64_t code, int64_t Q) {
  const auto o = seq.options().dtype(at::kFloat);
  return {at::empty(seq.sizes(), o), at::empty({seq.size(0)}, o), at::empty({seq.size(0), seq.size(1)}, o)};
}

Tensor backward_hip(const Tensor& seq_in, const Tensor& T, const std::optional<Tensor>& table_in,
                    const Tensor& g_soft_in, const std::optional<Tensor>& g_logZ_in, int64_t L, int64_t k, int64_t V,
                    int64_t code, int64_t Q) {
  const c10::OptionalDeviceGuard guard(at::device_of(seq_in));
  const Tensor seq = sequences(seq_in, V);
  same_device(seq, table_in, "codebook_or_lut");
  same_device(seq, g_soft_in, "g_soft");
  same_device(seq, g_logZ_in, "g_logZ");
  const int64_t B = seq.size(0), N = seq.size(1);
  TORCH_CHECK(g_soft_in.sizes() == seq.sizes(), "g_soft must be ", seq.sizes(), "; got ", g_soft_in.sizes());
  const auto table = as_f32(table_in);
  auto [Tt, per] = temperature(seq, T, B);
  const Tensor g = as_f32(g_soft_in);
  std::optional<Tensor> gz;
  if (g_logZ_in) gz = as_f32(g_logZ_in->reshape({-1}).expand({B}));
  Tensor d = at::empty_like(seq);
  if (B == 0) return d;
  const bcjr_problem p = problem(L, k, V, B, N, code, Q, per);
  Tensor ws = workspace(p, BCJR_OP_BACKWARD, seq);
  check(bcjr_backward(&p, seq.data_ptr<float>(), Tt.data_ptr<float>(), fptr(table), nullptr, g.data_ptr<float>(),
                      fptr(gz), d.data_ptr<float>(), ws.data_ptr(), (size_t)ws.numel(), stream_of(seq)),
        "bcjr_backward");
  return d;
}

Tensor backward_meta(const Tensor& seq, const Tensor& T, const std::optional<Tensor>& table, const Tensor& g_soft,
                     const std::optional<Tensor>& g_logZ, int64_t L, int64_t k, int64_t V, int64_t code, int64_t Q) {
  return at::empty(seq.sizes(), seq.options().dtype(at::kFloat));
}

// ---------------------------------------------------------------- T -> 0 path

using VitOut = std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor>;

VitOut vit_outputs(const Tensor& seq, int64_t k, int64_t V, bool want_packed) {
  const int64_t B = seq.size(0), N = seq.size(1), kV = k * V;
  const auto i32 = seq.options().dtype(at::kInt);
  const int64_t nbytes = (want_packed && 8 % kV == 0) ? (N * kV + 7) / 8 : 0;
  return {at::empty({B, N}, i32), at::empty({B, N}, i32), at::empty({B}, i32),
          at::empty(seq.sizes(), seq.options().dtype(at::kFloat)), at::empty({B}, seq.options().dtype(at::kFloat)),
          at::empty({B, nbytes}, seq.options().dtype(at::kByte))};
}

// walk, bitstream, start, recon, mse, packed; packed is (B, 0) when not asked
// for (or kV does not divide 8).  With overlap ((B,) int32) the tail-biting
// constraint of bcjr_viterbi_constrained applies.
VitOut viterbi_hip(const Tensor& seq_in, const std::optional<Tensor>& table_in, int64_t L, int64_t k, int64_t V,
                   int64_t code, int64_t Q, bool want_packed, const std::optional<Tensor>& overlap_in,
                   int64_t overlap_bits) {
  const c10::OptionalDeviceGuard guard(at::device_of(seq_in));
  const Tensor seq = sequences(seq_in, V);
  same_device(seq, table_in, "codebook_or_lut");
  same_device(seq, overlap_in, "overlap");
  const auto table = as_f32(table_in);
  VitOut out = vit_outputs(seq, k, V, want_packed);
  auto& [walk, bits, start, recon, mse, packed] = out;
  const int64_t B = seq.size(0), N = seq.size(1);
  if (B == 0) return out;
  const bcjr_problem p = problem(L, k, V, B, N, code, Q, false);
  Tensor ws = workspace(p, BCJR_OP_VITERBI, seq);
  uint8_t* pk = packed.size(1) ? packed.data_ptr<uint8_t>() : nullptr;
  if (!overlap_in) {
    check(bcjr_viterbi(&p, seq.data_ptr<float>(), fptr(table), walk.data_ptr<int32_t>(), bits.data_ptr<int32_t>(),
                       start.data_ptr<int32_t>(), recon.data_ptr<float>(), mse.data_ptr<float>(), pk, ws.data_ptr(),
                       (size_t)ws.numel(), stream_of(seq)),
          "bcjr_viterbi");
  } else {
    const Tensor ov = overlap_in->to(at::kInt).reshape({-1}).contiguous();
    TORCH_CHECK(ov.numel() == B, "overlap has ", ov.numel(), " values for B=", B, " sequences");
    check(bcjr_viterbi_constrained(&p, seq.data_ptr<float>(), fptr(table), (int)overlap_bits, ov.data_ptr<int32_t>(),
                                   walk.data_ptr<int32_t>(), bits.data_ptr<int32_t>(), start.data_ptr<int32_t>(),
                                   recon.data_ptr<float>(), mse.data_ptr<float>(), pk, ws.data_ptr(),
                                   (size_t)ws.numel(), stream_of(seq)),
          "bcjr_viterbi_constrained");
  }
  return out;
}

VitOut viterbi_meta(const Tensor& seq, const std::optional<Tensor>& table, int64_t L, int64_t k, int64_t V,
                    int64_t code, int64_t Q, bool want_packed, const std::optional<Tensor>& overlap,
                    int64_t overlap_bits) {
  return vit_outputs(seq, k, V, want_packed);
}

// Walks (B, N) int32 and recon (B, N, V) float32 (recon (B, N, 0) when
// want_recon is false) from start states and a bitstream: (B, N) int32, or
// packed (B, ceil(N*kV/8)) uint8 with N given.
std::tuple<Tensor, Tensor> decode_hip(const Tensor& start_in, const std::optional<Tensor>& table_in,
                                      const std::optional<Tensor>& bits_in, const std::optional<Tensor>& packed_in,
                                      int64_t N, int64_t L, int64_t k, int64_t V, int64_t code, int64_t Q,
                                      bool want_recon) {
  const c10::OptionalDeviceGuard guard(at::device_of(start_in));
  same_device(start_in, table_in, "codebook_or_lut");
  same_device(start_in, bits_in, "bitstream");
  same_device(start_in, packed_in, "packed");
  TORCH_CHECK(bits_in || packed_in, "need bitstream or packed");
  const Tensor start = start_in.to(at::kInt).reshape({-1}).contiguous();
  const int64_t B = start.numel();
  std::optional<Tensor> bits, packed;
  if (bits_in) {
    bits = bits_in->to(at::kInt).contiguous();
    TORCH_CHECK(bits->dim() == 2 && bits->size(0) == B, "bitstream must be (B=", B, ", N); got ", bits->sizes());
    N = bits->size(1);
  } else {
    packed = packed_in->to(at::kByte).contiguous();
  }
  const auto table = as_f32(table_in);
  Tensor walk = at::empty({B, N}, start.options());
  Tensor recon = at::empty({B, N, want_recon ? V : 0}, start.options().dtype(at::kFloat));
  if (B == 0 || N == 0) return {walk, recon};
  const bcjr_problem p = problem(L, k, V, B, N, code, Q, false);
  check(bcjr_decode(&p, bits ? bits->data_ptr<int32_t>() : nullptr, packed ? packed->data_ptr<uint8_t>() : nullptr,
                    start.data_ptr<int32_t>(), fptr(table), walk.data_ptr<int32_t>(),
                    want_recon ? recon.data_ptr<float>() : nullptr, stream_of(start)),
        "bcjr_decode");
  return {walk, recon};
}

std::tuple<Tensor, Tensor> decode_meta(const Tensor& start, const std::optional<Tensor>& table,
                                       const std::optional<Tensor>& bits, const std::optional<Tensor>& packed,
                                       int64_t N, int64_t L, int64_t k, int64_t V, int64_t code, int64_t Q,
                                       bool want_recon) {
  const int64_t B = start.numel(), n = bits ? bits->size(1) : N;
  return {at::empty({B, n}, start.options().dtype(at::kInt)),
          at::empty({B, n, want_recon ? V : 0}, start.options().dtype(at::kFloat))};
}

std::tuple<Tensor, Tensor> viterbi_trace_hip(const Tensor& seq_in, const std::optional<Tensor>& table_in, int64_t L,
                                             int64_t k, int64_t V, int64_t code, int64_t Q) {
  const c10::OptionalDeviceGuard guard(at::device_of(seq_in));
  const Tensor seq = sequences(seq_in, V);
  same_device(seq, table_in, "codebook_or_lut");
  const auto table = as_f32(table_in);
  const int64_t B = seq.size(0), N = seq.size(1), S = int64_t(1) << L;
  Tensor trace = at::empty({B, N, S}, seq.options()), backptr = at::empty({B, N, S}, seq.options().dtype(at::kInt));
  if (B == 0 || N == 0) return {trace, backptr};
  const bcjr_problem p = problem(L, k, V, B, N, code, Q, false);
  check(bcjr_viterbi_trace(&p, seq.data_ptr<float>(), fptr(table), trace.data_ptr<float>(),
                           backptr.data_ptr<int32_t>(), stream_of(seq)),
        "bcjr_viterbi_trace");
  return {trace, backptr};
}

std::tuple<Tensor, Tensor> viterbi_trace_meta(const Tensor& seq, const std::optional<Tensor>& table, int64_t L,
                                              int64_t k, int64_t V, int64_t code, int64_t Q) {
  const int64_t B = seq.size(0), N = seq.size(1), S = int64_t(1) << L;
  return {at::empty({B, N, S}, seq.options().dtype(at::kFloat)), at::empty({B, N, S}, seq.options().dtype(at::kInt))};
}

// (m, n) float32 = scale * c(walk) from one step per byte (uint8 bitstream),
// one per int32, or packed kV bits per step (packed given).
Tensor dequant_hip(const Tensor& start_in, const std::optional<Tensor>& table_in, const std::optional<Tensor>& bits_in,
                   const std::optional<Tensor>& packed_in, int64_t m, int64_t n, int64_t Tx, int64_t Ty, double scale,
                   int64_t L, int64_t k, int64_t V, int64_t code, int64_t Q) {
  const c10::OptionalDeviceGuard guard(at::device_of(start_in));
  same_device(start_in, table_in, "codebook_or_lut");
  same_device(start_in, bits_in, "bitstream");
  same_device(start_in, packed_in, "packed");
  TORCH_CHECK(bits_in || packed_in, "need bitstream or packed");
  TORCH_CHECK(Tx >= 1 && Ty >= 1 && (Tx * Ty) % V == 0, "tile ", Tx, "x", Ty, " for V=", V);
  const Tensor start = start_in.reshape({-1}).to(at::kInt).contiguous();
  const int64_t B = start.numel(), N = (Tx * Ty) / V;
  Tensor bits;
  int fmt;
  if (bits_in) {
    TORCH_CHECK(bits_in->numel() == B * N, "bitstream has ", bits_in->numel(), " steps, expected ", B, " tiles x ", N);
    fmt = bits_in->scalar_type() == at::kByte ? BCJR_BITS_U8 : BCJR_BITS_I32;
    bits = fmt == BCJR_BITS_U8 ? bits_in->reshape({B, N}).contiguous() : bits_in->reshape({B, N}).to(at::kInt).contiguous();
  } else {
    const int64_t nbytes = (N * k * V + 7) / 8;
    TORCH_CHECK(packed_in->numel() == B * nbytes, "packed bitstream has ", packed_in->numel(), " bytes, expected ", B,
                " tiles x ", nbytes);
    fmt = BCJR_BITS_PACKED;
    bits = packed_in->reshape({B, nbytes}).to(at::kByte).contiguous();
  }
  const auto table = as_f32(table_in);
  Tensor out = at::empty({m, n}, start.options().dtype(at::kFloat));
  const bcjr_problem p = problem(L, k, V, B, N, code, Q, false);
  check(bcjr_dequant(&p, bits.data_ptr(), fmt, start.data_ptr<int32_t>(), fptr(table), m, n, (int)Tx, (int)Ty, scale,
                     out.data_ptr<float>(), stream_of(start)),
        "bcjr_dequant");
  return out;
}

Tensor dequant_meta(const Tensor& start, const std::optional<Tensor>& table, const std::optional<Tensor>& bits,
                    const std::optional<Tensor>& packed, int64_t m, int64_t n, int64_t Tx, int64_t Ty, double scale,
                    int64_t L, int64_t k, int64_t V, int64_t code, int64_t Q) {
  return at::empty({m, n}, start.options().dtype(at::kFloat));
}

// The (2^L, V) codebook of a generator, on the device of `like` (any tensor).
Tensor codebook_hip(const Tensor& like, const std::optional<Tensor>& lut_in, int64_t L, int64_t code, int64_t Q) {
  const c10::OptionalDeviceGuard guard(at::device_of(like));
  same_device(like, lut_in, "lut");
  const int64_t V = code == BCJR_CODE_HYB ? 2 : 1;
  const auto lut = as_f32(lut_in);
  Tensor out = at::empty({int64_t(1) << L, V}, like.options().dtype(at::kFloat));
  const bcjr_problem p = problem(L, 2, V, 0, 1, code, Q, false);
  check(bcjr_codebook(&p, fptr(lut), out.data_ptr<float>(), stream_of(like)), "bcjr_codebook");
  return out;
}

Tensor codebook_meta(const Tensor& like, const std::optional<Tensor>& lut, int64_t L, int64_t code, int64_t Q) {
  return at::empty({int64_t(1) << L, code == BCJR_CODE_HYB ? 2 : 1}, like.options().dtype(at::kFloat));
}

// ------------------------------------------------------------------------ RHT

Tensor hadamard_hip(const Tensor& x, double scale) {
  TORCH_CHECK(x.scalar_type() == at::kFloat, "hadamard_transform expects a float32 GPU tensor");
  const c10::OptionalDeviceGuard guard(at::device_of(x));
  const Tensor xc = x.contiguous();
  Tensor out = at::empty_like(xc);
  const int64_t n = xc.dim() ? xc.size(-1) : 1;
  const int64_t rows = n ? xc.numel() / n : 0;
  check(bcjr_hadamard(xc.data_ptr<float>(), out.data_ptr<float>(), rows, n, (float)scale, stream_of(xc)),
        "bcjr_hadamard");
  return out;
}

Tensor hadamard_meta(const Tensor& x, double scale) { return at::empty(x.sizes(), x.options().dtype(at::kFloat)); }

Tensor rht_hip(const Tensor& W, const Tensor& sign_l, const Tensor& sign_r, bool inverse) {
  TORCH_CHECK(W.dim() == 2 && W.scalar_type() == at::kFloat, "W must be a 2-D float32 GPU tensor; got ", W.sizes(),
              " ", W.scalar_type());
  const int64_t m = W.size(0), n = W.size(1);
  TORCH_CHECK(sign_l.sizes() == at::IntArrayRef({m}) && sign_r.sizes() == at::IntArrayRef({n}),
              "sign vectors must be (", m, ",) and (", n, ",); got ", sign_l.sizes(), ", ", sign_r.sizes());
  const c10::OptionalDeviceGuard guard(at::device_of(W));
  const Tensor Wc = W.contiguous();
  const Tensor sl = sign_l.to(W.device(), at::kFloat).contiguous(), sr = sign_r.to(W.device(), at::kFloat).contiguous();
  Tensor out = at::empty_like(Wc);
  check(bcjr_rht(Wc.data_ptr<float>(), out.data_ptr<float>(), m, n, sl.data_ptr<float>(), sr.data_ptr<float>(),
                 inverse ? 1 : 0, stream_of(Wc)),
        "bcjr_rht");
  return out;
}

Tensor rht_meta(const Tensor& W, const Tensor& sign_l, const Tensor& sign_r, bool inverse) {
  TORCH_CHECK(W.dim() == 2 && sign_l.dim() == 1 && sign_r.dim() == 1 && sign_l.size(0) == W.size(0) &&
                  sign_r.size(0) == W.size(1),
              "RHT of ", W.sizes(), " with signs ", sign_l.sizes(), ", ", sign_r.sizes());
  return at::empty(W.sizes(), W.options().dtype(at::kFloat));
}

Tensor rht_batched_hip(const Tensor& W, const Tensor& sign_l, const Tensor& sign_r, bool inverse) {
  TORCH_CHECK(W.dim() == 3 && W.scalar_type() == at::kFloat, "W must be a 3-D float32 GPU tensor; got ", W.sizes(),
              " ", W.scalar_type());
  const int64_t E = W.size(0), m = W.size(1), n = W.size(2);
  TORCH_CHECK(sign_l.sizes() == at::IntArrayRef({E, m}) && sign_r.sizes() == at::IntArrayRef({E, n}),
              "sign vectors must be (", E, ", ", m, ") and (", E, ", ", n, "); got ", sign_l.sizes(), ", ",
              sign_r.sizes());
  const c10::OptionalDeviceGuard guard(at::device_of(W));
  const Tensor Wc = W.contiguous();
  const Tensor sl = sign_l.to(W.device(), at::kFloat).contiguous(), sr = sign_r.to(W.device(), at::kFloat).contiguous();
  Tensor out = at::empty_like(Wc);
  check(bcjr_rht_batched(Wc.data_ptr<float>(), out.data_ptr<float>(), E, m, n, sl.data_ptr<float>(),
                         sr.data_ptr<float>(), inverse ? 1 : 0, stream_of(Wc)),
        "bcjr_rht_batched");
  return out;
}

Tensor rht_batched_meta(const Tensor& W, const Tensor& sign_l, const Tensor& sign_r, bool inverse) {
  return at::empty(W.sizes(), W.options().dtype(at::kFloat));
}

}  // namespace

TORCH_LIBRARY(bcjr, m) {
  m.def("forward(Tensor sequences, Tensor T, Tensor? table, int L, int k, int V, int code, int Q) -> (Tensor, Tensor)");
  m.def("forward_internals(Tensor sequences, Tensor T, Tensor? table, int L, int k, int V, int code, int Q) "
        "-> (Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("forward_entropy(Tensor sequences, Tensor T, Tensor? table, int L, int k, int V, int code, int Q) "
        "-> (Tensor, Tensor, Tensor)");
  m.def("backward(Tensor sequences, Tensor T, Tensor? table, Tensor g_soft, Tensor? g_logZ, int L, int k, int V, "
        "int code, int Q) -> Tensor");
  m.def("viterbi(Tensor sequences, Tensor? table, int L, int k, int V, int code, int Q, bool packed, "
        "Tensor? overlap=None, int overlap_bits=0) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("decode(Tensor start, Tensor? table, Tensor? bitstream, Tensor? packed, int N, int L, int k, int V, int code, "
        "int Q, bool recon) -> (Tensor, Tensor)");
  m.def("viterbi_trace(Tensor sequences, Tensor? table, int L, int k, int V, int code, int Q) -> (Tensor, Tensor)");
  m.def("dequant(Tensor start, Tensor? table, Tensor? bitstream, Tensor? packed, int m, int n, int Tx, int Ty, "
        "float scale, int L, int k, int V, int code, int Q) -> Tensor");
  m.def("codebook(Tensor like, Tensor? lut, int L, int code, int Q) -> Tensor");
  m.def("hadamard(Tensor x, float scale) -> Tensor");
  m.def("rht(Tensor W, Tensor sign_l, Tensor sign_r, bool inverse) -> Tensor");
  m.def("rht_batched(Tensor W, Tensor sign_l, Tensor sign_r, bool inverse) -> Tensor");
}

TORCH_LIBRARY_IMPL(bcjr, CUDA, m) {
  m.impl("forward", &forward_hip);
  m.impl("forward_internals", &forward_internals_hip);
  m.impl("forward_entropy", &forward_entropy_hip);
  m.impl("backward", &backward_hip);
  m.impl("viterbi", &viterbi_hip);
  m.impl("decode", &decode_hip);
  m.impl("viterbi_trace", &viterbi_trace_hip);
  m.impl("dequant", &dequant_hip);
  m.impl("codebook", &codebook_hip);
  m.impl("hadamard", &hadamard_hip);
  m.impl("rht", &rht_hip);
  m.impl("rht_batched", &rht_batched_hip);
}

TORCH_LIBRARY_IMPL(bcjr, Meta, m) {
  m.impl("forward", &forward_meta);
  m.impl("forward_internals", &forward_internals_meta);
  m.impl("forward_entropy", &forward_entropy_meta);
  m.impl("backward", &backward_meta);
  m.impl("viterbi", &viterbi_meta);
  m.impl("decode", &decode_meta);
  m.impl("viterbi_trace", &viterbi_trace_meta);
  m.impl("dequant", &dequant_meta);
  m.impl("codebook", &codebook_meta);
  m.impl("hadamard", &hadamard_meta);
  m.impl("rht", &rht_meta);
  m.impl("rht_batched", &rht_batched_meta);
}
