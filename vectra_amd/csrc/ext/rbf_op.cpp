// torch.library registration of vectra::rbf_attention for PyTorch-ROCm.
//
// Mirrors the reference operator kernels/vectra_kernels/custom_ops.py:52-97 (op and schema :52-72, 'cuda' kernel :75-85):
//   schema  rbf_attention(Tensor q, Tensor k, Tensor v, Tensor scale,
//                         Tensor? key_bias=None) -> Tensor
//   CUDA key (HIP tensors on ROCm)  -> libvectra_rbf.so (include/vectra_rbf.h),
//                                      on the caller's current HIP stream
//   CPU key                         -> the native loop below
//   fake/meta                       -> registered from Python (SymInt-safe)
// The operator is functional (no aliasing, no mutation) and forward-only, as
// in the reference (compiler/vectra_compiler/rewrite_pass.py:71-74).
//
// There is no CPU fallback for device tensors: if the HIP library cannot be
// loaded this extension does not load either.

#include <ATen/ATen.h>
#include <ATen/Parallel.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <cmath>
#include <limits>
#include <vector>

#include "vectra_rbf.h"

namespace {

int32_t to_vectra_dtype(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return VECTRA_F32;
    case at::kHalf: return VECTRA_F16;
    case at::kBFloat16: return VECTRA_BF16;
    case at::kDouble: return VECTRA_F64;
    default: return -1;
  }
}

// Shapes, dtypes and broadcast views shared by both implementations.
struct Inputs {
  int64_t B, H, Nq, Nk, D, Dv;
  at::Tensor scale;  // expanded view [B, H, 1, 1] (any float dtype)
  at::Tensor bias;   // expanded view [B, H, 1, Nk] or undefined
};

// The coefficient and the bias are read in their own dtype when the kernels
// decode it (fp32, fp16, bf16, fp64).  Any other real dtype (integers, bool,
// 8-bit floats) is converted to fp32 first, as the reference converts both
// with `.to(torch.float32)` (spatial_rbf_attention.py:208-213, :221;
// reference.py:43, :98).
at::Tensor readable_coefficient(const at::Tensor& t, const char* name) {
  if (to_vectra_dtype(t.scalar_type()) >= 0) return t;
  TORCH_CHECK(!at::isComplexType(t.scalar_type()), "vectra::rbf_attention: ", name,
              " must be real; got ", t.scalar_type());
  return t.to(at::kFloat);
}

Inputs check_inputs(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                    const at::Tensor& scale_in, const std::optional<at::Tensor>& key_bias) {
  TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4,
              "vectra::rbf_attention: q, k and v must be 4-D [B, H, N, D]; got ", q.sizes(), ", ",
              k.sizes(), ", ", v.sizes());
  Inputs in{};
  in.B = q.size(0);
  in.H = q.size(1);
  in.Nq = q.size(2);
  in.D = q.size(3);
  in.Nk = k.size(2);
  in.Dv = v.size(3);
  TORCH_CHECK(k.size(0) == in.B && k.size(1) == in.H && k.size(3) == in.D,
              "vectra::rbf_attention: k must be [B, H, Nk, D] matching q ", q.sizes(), "; got ",
              k.sizes());
  TORCH_CHECK(v.size(0) == in.B && v.size(1) == in.H && v.size(2) == in.Nk,
              "vectra::rbf_attention: v must be [B, H, Nk, Dv] matching k ", k.sizes(), "; got ",
              v.sizes());
  const auto dt = q.scalar_type();
  TORCH_CHECK(dt == at::kFloat || dt == at::kHalf || dt == at::kBFloat16,
              "vectra::rbf_attention: q, k, v must be float32, float16 or bfloat16; got ", dt);
  TORCH_CHECK(k.scalar_type() == dt && v.scalar_type() == dt,
              "vectra::rbf_attention: q, k and v must share a dtype; got ", dt, ", ",
              k.scalar_type(), ", ", v.scalar_type());
  const at::Tensor scale = readable_coefficient(scale_in, "scale");
  TORCH_CHECK(scale.dim() <= 4, "vectra::rbf_attention: scale must broadcast to [B, H, 1, 1]");
  // Broadcasting rules and errors of Tensor.expand (spatial_rbf_attention.py:208-213).
  in.scale = scale.expand({in.B, in.H, 1, 1});
  if (key_bias.has_value() && key_bias->defined()) {
    at::Tensor bias = readable_coefficient(*key_bias, "key_bias");
    TORCH_CHECK(bias.dim() <= 4, "vectra::rbf_attention: key_bias must broadcast to [B, H, 1, Nk]");
    while (bias.dim() < 4) bias = bias.unsqueeze(0);
    // spatial_rbf_attention.py:224-225.
    TORCH_CHECK_VALUE(bias.size(2) == 1, "key_bias must be constant across queries");
    TORCH_CHECK(bias.size(1) == 1 || bias.size(1) == in.H,
                "vectra::rbf_attention: key_bias must be per key or per (head, key); got ",
                key_bias->sizes());
    in.bias = bias.expand({in.B, in.H, 1, in.Nk});
  }
  return in;
}

// ---------------------------------------------------------------- device

at::Tensor rbf_attention_hip(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                             const at::Tensor& scale, const std::optional<at::Tensor>& key_bias) {
  Inputs in = check_inputs(q, k, v, scale, key_bias);
  TORCH_CHECK(q.is_cuda() && k.device() == q.device() && v.device() == q.device(),
              "vectra::rbf_attention: q, k and v must be on one GPU; got ", q.device(), ", ",
              k.device(), ", ", v.device());
  at::Tensor scale_dev = in.scale;
  if (scale_dev.device() != q.device()) {
    // A CPU scalar coefficient is accepted, as elementwise ops accept it.
    TORCH_CHECK(scale_dev.device().is_cpu() && scale.numel() == 1,
                "vectra::rbf_attention: scale must be on ", q.device(), " (or a CPU scalar)");
    scale_dev = readable_coefficient(scale, "scale").reshape({1, 1, 1, 1}).to(q.device()).expand(
        {in.B, in.H, 1, 1});
  }
  if (in.bias.defined())
    TORCH_CHECK(in.bias.device() == q.device(), "vectra::rbf_attention: key_bias must be on ",
                q.device());

  c10::DeviceGuard guard(q.device());
  at::Tensor out = at::empty({in.B, in.H, in.Nq, in.Dv}, v.options());

  vectra_rbf_args a{};
  a.struct_size = sizeof(vectra_rbf_args);
  a.q = q.data_ptr();
  a.k = k.data_ptr();
  a.v = v.data_ptr();
  a.out = out.data_ptr();
  a.scale = scale_dev.data_ptr();
  a.key_bias = in.bias.defined() ? in.bias.data_ptr() : nullptr;
  a.in_dtype = to_vectra_dtype(q.scalar_type());
  a.out_dtype = to_vectra_dtype(out.scalar_type());
  a.scale_dtype = to_vectra_dtype(scale_dev.scalar_type());
  a.bias_dtype = in.bias.defined() ? to_vectra_dtype(in.bias.scalar_type()) : VECTRA_F32;
  a.batch = in.B;
  a.heads = in.H;
  a.n_q = in.Nq;
  a.n_k = in.Nk;
  a.head_dim = in.D;
  a.value_dim = in.Dv;
  for (int i = 0; i < 4; ++i) {
    a.q_stride[i] = q.stride(i);
    a.k_stride[i] = k.stride(i);
    a.v_stride[i] = v.stride(i);
    a.out_stride[i] = out.stride(i);
  }
  a.scale_stride_b = scale_dev.stride(0);
  a.scale_stride_h = scale_dev.stride(1);
  if (in.bias.defined()) {
    a.bias_stride_b = in.bias.stride(0);
    a.bias_stride_h = in.bias.stride(1);
    a.bias_stride_n = in.bias.stride(3);
  }
  a.variant = VECTRA_VARIANT_AUTO;
  auto stream = c10::hip::getCurrentHIPStream(q.device().index());
  const int status =
      vectra_rbf_attention_fwd(&a, reinterpret_cast<vectra_stream_t>(stream.stream()));
  TORCH_CHECK(status == VECTRA_OK, "vectra::rbf_attention: ", vectra_rbf_status_string(status));
  return out;
}

// ------------------------------------------------------------------- host
//
// The operator's implementation off the GPU (the reference's default
// implementation, custom_ops.py:52-72 calling reference.py:79-99): same expansion, clamp, masking and
// fp32 accumulation as the device kernels, one task per query row.

template <typename T>
void cpu_rows(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
              const at::Tensor& scale, const at::Tensor& bias, at::Tensor& out, const Inputs& in) {
  const T* qp = q.const_data_ptr<T>();
  const T* kp = k.const_data_ptr<T>();
  const T* vp = v.const_data_ptr<T>();
  const float* sp = scale.const_data_ptr<float>();
  const float* bp = bias.defined() ? bias.const_data_ptr<float>() : nullptr;
  float* op = out.mutable_data_ptr<float>();
  const auto sq = q.strides(), sk = k.strides(), sv = v.strides();
  const int64_t ssb = scale.stride(0), ssh = scale.stride(1);
  const int64_t sbb = bp ? bias.stride(0) : 0, sbh = bp ? bias.stride(1) : 0,
                sbn = bp ? bias.stride(3) : 0;
  const int64_t rows = in.B * in.H * in.Nq;
  at::parallel_for(0, rows, 16, [&](int64_t begin, int64_t end) {
    std::vector<float> logit(static_cast<size_t>(in.Nk));
    std::vector<float> qf(static_cast<size_t>(in.D));
    std::vector<float> acc(static_cast<size_t>(in.Dv));
    for (int64_t r = begin; r < end; ++r) {
      const int64_t i = r % in.Nq, bh = r / in.Nq, h = bh % in.H, b = bh / in.H;
      const T* qrow = qp + b * sq[0] + h * sq[1] + i * sq[2];
      float q_norm = 0.f;
      for (int64_t d = 0; d < in.D; ++d) {
        qf[d] = static_cast<float>(qrow[d * sq[3]]);
        q_norm += qf[d] * qf[d];
      }
      const float neg_scale = -sp[b * ssb + h * ssh];
      float row_max = -std::numeric_limits<float>::infinity();
      for (int64_t j = 0; j < in.Nk; ++j) {
        const T* krow = kp + b * sk[0] + h * sk[1] + j * sk[2];
        float dot = 0.f, k_norm = 0.f;
        for (int64_t d = 0; d < in.D; ++d) {
          const float x = static_cast<float>(krow[d * sk[3]]);
          dot += qf[d] * x;
          k_norm += x * x;
        }
        float x = neg_scale * std::max((q_norm + k_norm) - 2.f * dot, 0.f);
        if (bp) x += bp[b * sbb + h * sbh + j * sbn];
        logit[j] = x;
        row_max = std::max(row_max, x);
      }
      const float safe_max = std::isinf(row_max) && row_max < 0 ? 0.f : row_max;
      std::fill(acc.begin(), acc.end(), 0.f);
      float sum = 0.f;
      for (int64_t j = 0; j < in.Nk; ++j) {
        const float w = std::exp(logit[j] - safe_max);
        sum += w;
        const T* vrow = vp + b * sv[0] + h * sv[1] + j * sv[2];
        for (int64_t d = 0; d < in.Dv; ++d) acc[d] += w * static_cast<float>(vrow[d * sv[3]]);
      }
      float* orow = op + r * in.Dv;
      for (int64_t d = 0; d < in.Dv; ++d) orow[d] = in.Nk > 0 ? acc[d] / sum : 0.f;
    }
  });
}

at::Tensor rbf_attention_cpu(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                             const at::Tensor& scale, const std::optional<at::Tensor>& key_bias) {
  Inputs in = check_inputs(q, k, v, scale, key_bias);
  TORCH_CHECK(q.is_cpu() && k.is_cpu() && v.is_cpu() && scale.is_cpu() &&
                  (!in.bias.defined() || in.bias.is_cpu()),
              "vectra::rbf_attention: mixed CPU and GPU arguments");
  const at::Tensor scale_f = in.scale.to(at::kFloat);
  const at::Tensor bias_f = in.bias.defined() ? in.bias.to(at::kFloat) : at::Tensor();
  at::Tensor out = at::empty({in.B, in.H, in.Nq, in.Dv}, v.options().dtype(at::kFloat));
  switch (q.scalar_type()) {
    case at::kFloat: cpu_rows<float>(q, k, v, scale_f, bias_f, out, in); break;
    case at::kHalf: cpu_rows<at::Half>(q, k, v, scale_f, bias_f, out, in); break;
    default: cpu_rows<at::BFloat16>(q, k, v, scale_f, bias_f, out, in); break;
  }
  return out.to(v.scalar_type());
}

}  // namespace

TORCH_LIBRARY(vectra, m) {
  m.def(
      "rbf_attention(Tensor q, Tensor k, Tensor v, Tensor scale, Tensor? key_bias=None) -> "
      "Tensor");
}

TORCH_LIBRARY_IMPL(vectra, CUDA, m) { m.impl("rbf_attention", rbf_attention_hip); }

TORCH_LIBRARY_IMPL(vectra, CPU, m) { m.impl("rbf_attention", rbf_attention_cpu); }
