// TensorFlow op OneDNNFlashAttention on this library (TensorFlow-ROCm).
//
// Same op name, inputs, attributes, defaults, shape function and error texts
// as the reference's tensorflow_ops/onednn_flash_attention_op.cc:13-146, with
// one attribute added: T in {float, bfloat16, half}, default float, so that
// graphs written for the reference (float only, no T attribute) load
// unchanged. Kernels:
//   DEVICE_GPU, T = float / bfloat16 / half: ofh_attention_fwd on the device
//       tensors, ordered on TensorFlow's compute stream (no host copies);
//   DEVICE_CPU, T = float: ofh_attention_fwd_host (the reference's registration;
//       the arithmetic still runs on the GPU, with copies in and out).
// scale is 1/sqrt(D) and the mask is top-left causal when causal = true, as in
// the reference (:91-92). query_block_size, key_block_size, use_onednn,
// tile_kernel and qk_tile_layout are validated as in the reference (the
// onednn_brgemm + strided_k refusal in Compute, as its oneDNN BRGEMM builds
// do); the GPU kernels choose their own tiles, so the values are otherwise
// advisory.
//
// Build (needs TensorFlow's headers and library, see the package Makefile's
// tf_op target): the op library links libonednn_flash_hip.so.

#define EIGEN_USE_GPU

#include <cmath>
#include <string>

#include "onednn_flash_hip.h"
#include "tensorflow/core/framework/op.h"
#include "tensorflow/core/framework/op_kernel.h"
#include "tensorflow/core/framework/shape_inference.h"
#include "tensorflow/core/framework/types.h"
#include "unsupported/Eigen/CXX11/Tensor"

namespace onednn_flash_tf {

using tensorflow::DEVICE_CPU;
using tensorflow::DEVICE_GPU;
using tensorflow::OpKernel;
using tensorflow::OpKernelConstruction;
using tensorflow::OpKernelContext;
using tensorflow::Tensor;
using tensorflow::TensorShape;
namespace errors = tensorflow::errors;
namespace shape_inference = tensorflow::shape_inference;

REGISTER_OP("OneDNNFlashAttention")
    .Input("q: T")
    .Input("k: T")
    .Input("v: T")
    .Output("out: T")
    .Attr("T: {float, bfloat16, half} = DT_FLOAT")
    .Attr("causal: bool = true")
    .Attr("query_block_size: int = 16")
    .Attr("key_block_size: int = 32")
    .Attr("use_onednn: bool = true")
    .Attr("tile_kernel: string = 'onednn'")
    .Attr("qk_tile_layout: string = 'strided_k'")
    .SetShapeFn([](shape_inference::InferenceContext* c) {
        shape_inference::ShapeHandle q, k, v;
        TF_RETURN_IF_ERROR(c->WithRank(c->input(0), 4, &q));
        TF_RETURN_IF_ERROR(c->WithRank(c->input(1), 4, &k));
        TF_RETURN_IF_ERROR(c->WithRank(c->input(2), 4, &v));
        c->set_output(0, c->MakeShape({c->Dim(q, 0), c->Dim(q, 1), c->Dim(q, 2), c->Dim(v, 3)}));
        return tensorflow::OkStatus();
    });

template <typename T>
constexpr int32_t dtype_code();
template <>
constexpr int32_t dtype_code<float>() { return OFH_DTYPE_F32; }
template <>
constexpr int32_t dtype_code<Eigen::bfloat16>() { return OFH_DTYPE_BF16; }
template <>
constexpr int32_t dtype_code<Eigen::half>() { return OFH_DTYPE_F16; }

// OP_REQUIRES for a function that returns bool.
#define OP_REQUIRES_VALUE_OR_FALSE(CTX, EXP, STATUS) \
    do {                                             \
        if (!(EXP)) {                                \
            (CTX)->CtxFailure((STATUS));             \
            return false;                            \
        }                                            \
    } while (0)

// Attribute and shape checks shared by both kernels (reference :42-98).
class AttentionOpBase : public OpKernel {
public:
    explicit AttentionOpBase(OpKernelConstruction* ctx) : OpKernel(ctx) {
        OP_REQUIRES_OK(ctx, ctx->GetAttr("causal", &causal_));
        OP_REQUIRES_OK(ctx, ctx->GetAttr("query_block_size", &query_block_size_));
        OP_REQUIRES_OK(ctx, ctx->GetAttr("key_block_size", &key_block_size_));
        OP_REQUIRES_OK(ctx, ctx->GetAttr("use_onednn", &use_onednn_));
        OP_REQUIRES_OK(ctx, ctx->GetAttr("tile_kernel", &tile_kernel_));
        OP_REQUIRES_OK(ctx, ctx->GetAttr("qk_tile_layout", &qk_tile_layout_));
        OP_REQUIRES(ctx, tile_kernel_ == "onednn" || tile_kernel_ == "onednn_brgemm",
                    errors::InvalidArgument("tile_kernel must be 'onednn' or 'onednn_brgemm'"));
        OP_REQUIRES(ctx,
                    qk_tile_layout_ == "strided_k" || qk_tile_layout_ == "copied_transposed" ||
                        qk_tile_layout_ == "brgemm_transformed_k",
                    errors::InvalidArgument("qk_tile_layout must be 'strided_k', 'copied_transposed', or "
                                            "'brgemm_transformed_k'"));
    }

protected:
    // Validates the inputs, allocates the output and fills the parameters.
    // Returns false when the context already holds an error.
    bool prepare(OpKernelContext* ctx, int32_t dtype, Tensor** out, ofh_attention_params* p) {
        const Tensor& q = ctx->input(0);
        const Tensor& k = ctx->input(1);
        const Tensor& v = ctx->input(2);
        OP_REQUIRES_VALUE_OR_FALSE(ctx, q.dims() == 4, errors::InvalidArgument("q must be rank 4 [B,H,M,D]"));
        OP_REQUIRES_VALUE_OR_FALSE(ctx, k.dims() == 4, errors::InvalidArgument("k must be rank 4 [B,H,N,D]"));
        OP_REQUIRES_VALUE_OR_FALSE(ctx, v.dims() == 4, errors::InvalidArgument("v must be rank 4 [B,H,N,Dv]"));
        OP_REQUIRES_VALUE_OR_FALSE(ctx, q.dim_size(0) == k.dim_size(0) && q.dim_size(0) == v.dim_size(0),
                                   errors::InvalidArgument("batch dimensions must match"));
        OP_REQUIRES_VALUE_OR_FALSE(ctx, q.dim_size(1) == k.dim_size(1) && q.dim_size(1) == v.dim_size(1),
                                   errors::InvalidArgument("head dimensions must match"));
        OP_REQUIRES_VALUE_OR_FALSE(ctx, q.dim_size(3) == k.dim_size(3),
                                   errors::InvalidArgument("q/k head dimensions must match"));
        OP_REQUIRES_VALUE_OR_FALSE(ctx, k.dim_size(2) == v.dim_size(2),
                                   errors::InvalidArgument("k/v key-token dimensions must match"));
        OP_REQUIRES_VALUE_OR_FALSE(ctx, query_block_size_ > 0 && key_block_size_ > 0,
                                   errors::InvalidArgument("block sizes must be positive"));
        const TensorShape out_shape({q.dim_size(0), q.dim_size(1), q.dim_size(2), v.dim_size(3)});
        const tensorflow::Status s = ctx->allocate_output(0, out_shape, out);
        if (!s.ok()) {
            ctx->CtxFailure(s);
            return false;
        }
        // The reference rejects this combination in Compute, after the output
        // is allocated, with InvalidArgument, in its builds with oneDNN BRGEMM
        // (:102-119); the tile attributes are otherwise advisory here.
        OP_REQUIRES_VALUE_OR_FALSE(
            ctx, !(use_onednn_ && tile_kernel_ == "onednn_brgemm" && qk_tile_layout_ == "strided_k"),
            errors::InvalidArgument("tile_kernel='onednn_brgemm' does not support qk_tile_layout='strided_k'; "
                                    "use 'copied_transposed' or 'brgemm_transformed_k'"));
        ofh_attention_params_init(p);
        p->batch = (size_t)q.dim_size(0);
        p->heads = (size_t)q.dim_size(1);
        p->query_tokens = (size_t)q.dim_size(2);
        p->key_tokens = (size_t)k.dim_size(2);
        p->head_dim = (size_t)q.dim_size(3);
        p->value_dim = (size_t)v.dim_size(3);
        p->dtype = dtype;
        p->out_dtype = dtype;
        p->scale = 1.0f / std::sqrt(static_cast<float>(p->head_dim));
        p->causal = causal_ ? 1 : 0;
        return true;
    }

    // Library errors, zero-sized dimensions included, become Internal errors
    // with the library's text, as the reference wraps its exceptions (:132-134).
    void fail(OpKernelContext* ctx) {
        ctx->CtxFailure(errors::Internal("OneDNNFlashAttention failed: ", ofh_last_error()));
    }

private:
    bool causal_ = true;
    int query_block_size_ = 16;
    int key_block_size_ = 32;
    bool use_onednn_ = true;
    std::string tile_kernel_ = "onednn";
    std::string qk_tile_layout_ = "strided_k";
};

template <typename T>
class AttentionGpuOp final : public AttentionOpBase {
public:
    using AttentionOpBase::AttentionOpBase;

    void Compute(OpKernelContext* ctx) override {
        Tensor* out = nullptr;
        ofh_attention_params p;
        if (!prepare(ctx, dtype_code<T>(), &out, &p)) return;
        void* stream = (void*)ctx->eigen_device<Eigen::GpuDevice>().stream();
        // Scratch (block-mask tile lists, key-split partial rows) comes from
        // TensorFlow's allocator, so the library neither allocates nor blocks
        // the host inside Compute.
        size_t ws_bytes = 0;
        if (ofh_attention_workspace_bytes(&p, &ws_bytes) != OFH_SUCCESS) {
            fail(ctx);
            return;
        }
        Tensor ws;
        void* ws_ptr = nullptr;
        if (ws_bytes > 0) {
            OP_REQUIRES_OK(ctx, ctx->allocate_temp(tensorflow::DT_UINT8, TensorShape({(int64_t)ws_bytes}), &ws));
            ws_ptr = ws.flat<uint8_t>().data();
        }
        const int rc = ofh_attention_fwd(&p, ctx->input(0).flat<T>().data(), ctx->input(1).flat<T>().data(),
                                         ctx->input(2).flat<T>().data(), out->flat<T>().data(), ws_ptr,
                                         ws_bytes, stream);
        if (rc != OFH_SUCCESS) fail(ctx);
    }
};

class AttentionCpuOp final : public AttentionOpBase {
public:
    using AttentionOpBase::AttentionOpBase;

    void Compute(OpKernelContext* ctx) override {
        Tensor* out = nullptr;
        ofh_attention_params p;
        if (!prepare(ctx, OFH_DTYPE_F32, &out, &p)) return;
        const int rc = ofh_attention_fwd_host(&p, ctx->input(0).flat<float>().data(),
                                              ctx->input(1).flat<float>().data(),
                                              ctx->input(2).flat<float>().data(), out->flat<float>().data());
        if (rc != OFH_SUCCESS) fail(ctx);
    }
};

REGISTER_KERNEL_BUILDER(Name("OneDNNFlashAttention").Device(DEVICE_CPU).TypeConstraint<float>("T"),
                        AttentionCpuOp);
REGISTER_KERNEL_BUILDER(Name("OneDNNFlashAttention").Device(DEVICE_GPU).TypeConstraint<float>("T"),
                        AttentionGpuOp<float>);
REGISTER_KERNEL_BUILDER(Name("OneDNNFlashAttention").Device(DEVICE_GPU).TypeConstraint<Eigen::bfloat16>("T"),
                        AttentionGpuOp<Eigen::bfloat16>);
REGISTER_KERNEL_BUILDER(Name("OneDNNFlashAttention").Device(DEVICE_GPU).TypeConstraint<Eigen::half>("T"),
                        AttentionGpuOp<Eigen::half>);

}  // namespace onednn_flash_tf
