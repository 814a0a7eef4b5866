// helix_ops.cpp — HipTensor's tensor-trait operations (TensorOps, TensorActivation,
// TensorReduce::mean, TensorBroadcast, the Tensor shape operations) with CpuTensor's semantics
// and errors (crates/backend-cpu/src/lib.rs), the exported nn::S4Block, ssm::S4Block's
// convolutional forward, and the reference's nn bodies over these operations (helix::generic).
// Host code only: shapes and errors are decided here, every value comes from a device primitive
// of include/helix_hip.h.
#include <algorithm>
#include <cmath>

#include "helix/helix.hpp"
#include "helix_detail.h"
#include "helix_hip.h"
#include "ndlayout.hpp"

namespace helix {

using detail::invalid_dimension;
using detail::invalid_input;
using detail::shape_mismatch;
using detail::unsupported;

namespace {

void need_f32(const HipTensor& t) {
    if (t.storage() != Storage::F32)
        throw TensorError(ErrorKind::DTypeMismatch, "DType mismatch: expected \"F32 storage\", got \"BF16\"");
}

// cat, stack and broadcast_to read `data.as_slice().unwrap()`, which panics unless the array is
// in standard layout (e.g. after a transpose of two axes longer than 1)
void need_standard_layout(const HipTensor& t, const char* op) {
    if (!t.is_contiguous())
        unsupported(std::string(op) + " of a tensor that is not in standard layout (the reference's "
                    "as_slice().unwrap() panics)");
}

std::vector<int64_t> row_major_strides(const std::vector<size_t>& dims) {
    std::vector<int64_t> s(dims.size(), 1);
    for (size_t i = dims.size(); i-- > 1;) s[i - 1] = s[i] * (int64_t)dims[i];
    return s;
}

// dst (contiguous, `dims`) = src read through `src_strides` (elements) starting at `src`.
void strided_copy(const std::vector<size_t>& dims, const float* src,
                  const std::vector<int64_t>& src_strides, float* dst,
                  const std::vector<int64_t>& dst_strides) {
    if (dims.size() > HX_MAX_DIMS) unsupported("tensors of more than 8 dimensions");
    std::vector<int64_t> d(dims.begin(), dims.end());
    check(hx_copy_strided_f32((int)d.size(), d.data(), src, src_strides.data(), dst,
                              dst_strides.data(), nullptr),
          "hx_copy_strided_f32");
}

HipTensor binary(const HipTensor& a, const HipTensor& b, int op) {
    // equal shapes only: ShapeMismatch { expected: self, actual: other } (lib.rs:571-576)
    if (a.shape() != b.shape()) shape_mismatch(a.shape().as_slice(), b.shape().as_slice());
    need_f32(a);
    need_f32(b);
    HipTensor y(a.shape(), Storage::F32, 0);
    check(hx_binary_f32(op, (int64_t)a.numel(), (const float*)a.data(), (const float*)b.data(),
                        (float*)y.data(), nullptr),
          "hx_binary_f32");
    // &a + &b collects by the Zip's layout preference (C or F order)
    y.set_ref_strides(ndlayout::collect(a.shape().as_slice(), {a.ref_strides(), b.ref_strides()}));
    return y;
}

HipTensor unary(const HipTensor& x, int op, float s = 0.0f) {
    need_f32(x);
    HipTensor y(x.shape(), Storage::F32, 0);
    check(hx_unary_f32(op, (int64_t)x.numel(), (const float*)x.data(), s, (float*)y.data(), nullptr),
          "hx_unary_f32");
    y.set_ref_strides(x.ref_strides());  // mapv / map_inplace keep the strides
    return y;
}

}  // namespace

// ----------------------------------------------------------------------------- TensorOps
HipTensor HipTensor::matmul(const HipTensor& b) const {
    // CpuTensor::matmul (backend-cpu/src/lib.rs:634-757): every product is an f32 sum from 0.0
    // over k ascending, which hx_matmul_f32 reproduces; 1-D operands are [1, K] / [K, 1] there.
    const size_t ra = shape_.ndim(), rb = b.shape_.ndim();
    if (ra == 0 || rb == 0) unsupported("matrix multiplication requires at least 1D tensors");
    need_f32(*this);
    need_f32(b);
    size_t M, K, K2, N;
    Shape out;
    if (ra == 2 && rb == 2) {
        M = shape_.dim(0), K = shape_.dim(1), K2 = b.shape_.dim(0), N = b.shape_.dim(1);
        if (K != K2) shape_mismatch({K}, {K2});
        out = Shape({M, N});
    } else if (ra == 1 && rb == 2) {
        M = 1, K = shape_.dim(0), K2 = b.shape_.dim(0), N = b.shape_.dim(1);
        if (K != K2) shape_mismatch({K}, {K2});
        out = Shape({N});
    } else if (ra == 2 && rb == 1) {
        M = shape_.dim(0), K = shape_.dim(1), K2 = b.shape_.dim(0), N = 1;
        if (K != K2) shape_mismatch({K}, {K2});
        out = Shape({M});
    } else {
        unsupported("batch matrix multiplication for >2D tensors not implemented yet");
    }
    HipTensor y(out, Storage::F32, device_);
    check(hx_matmul_f32((int64_t)M, (int64_t)K, (int64_t)N, (const float*)data(),
                        (const float*)b.data(), (float*)y.data(), nullptr),
          "hx_matmul_f32");
    return y;
}

HipTensor HipTensor::add(const HipTensor& o) const { return binary(*this, o, HX_ADD); }
HipTensor HipTensor::sub(const HipTensor& o) const { return binary(*this, o, HX_SUB); }
HipTensor HipTensor::mul(const HipTensor& o) const { return binary(*this, o, HX_MUL); }
HipTensor HipTensor::div(const HipTensor& o) const { return binary(*this, o, HX_DIV); }
HipTensor HipTensor::add_scalar(float s) const { return unary(*this, HX_ADD_SCALAR, s); }
HipTensor HipTensor::mul_scalar(float s) const { return unary(*this, HX_MUL_SCALAR, s); }
HipTensor HipTensor::neg() const { return unary(*this, HX_NEG); }
HipTensor HipTensor::abs() const { return unary(*this, HX_ABS); }
HipTensor HipTensor::sqrt() const { return unary(*this, HX_SQRT); }
HipTensor HipTensor::exp() const { return unary(*this, HX_EXP); }
HipTensor HipTensor::log() const { return unary(*this, HX_LOG); }
HipTensor HipTensor::sin() const { return unary(*this, HX_SIN); }
HipTensor HipTensor::cos() const { return unary(*this, HX_COS); }
HipTensor HipTensor::silu() const { return unary(*this, HX_SILU); }
HipTensor HipTensor::sigmoid() const { return unary(*this, HX_SIGMOID); }

float HipTensor::to_scalar() const {
    if (numel() != 1)  // lib.rs:966-974
        invalid_input("Cannot convert tensor with " + std::to_string(numel()) + " elements to scalar");
    return to_host()[0];
}

HipTensor HipTensor::from_scalar(float value, Shape shape, int device) {
    HipTensor y(std::move(shape), Storage::F32, device);
    check(hx_fill_f32((int64_t)y.numel(), value, (float*)y.data(), nullptr), "hx_fill_f32");
    return y;
}

HipTensor HipTensor::eye(size_t n, int device) {
    HipTensor y(Shape({n, n}), Storage::F32, device);
    check(hx_eye_f32((int64_t)n, (float*)y.data(), nullptr), "hx_eye_f32");
    return y;
}

// ----------------------------------------------------------------------------- TensorReduce::mean
HipTensor HipTensor::mean(const std::vector<size_t>* dims, bool /*keepdim*/) const {
    need_f32(*this);
    std::vector<size_t> order;
    if (dims) order = *dims;
    else for (size_t i = 0; i < shape_.ndim(); ++i) order.push_back(i);
    HipTensor cur = *this;
    // dims.iter().rev(): each mean_axis removes its axis from the running result (lib.rs:998-1001)
    for (size_t k = order.size(); k-- > 0;) {
        const size_t ax = order[k];
        const std::vector<size_t>& d = cur.shape().as_slice();
        if (ax >= d.size()) invalid_dimension(ax, d);  // ndarray panics on an axis out of range
        if (d[ax] == 0) invalid_dimension(ax, d);       // mean_axis returns None -> unwrap panics
        size_t outer = 1, inner = 1;
        for (size_t i = 0; i < ax; ++i) outer *= d[i];
        for (size_t i = ax + 1; i < d.size(); ++i) inner *= d[i];
        std::vector<size_t> nd(d);
        nd.erase(nd.begin() + (long)ax);
        HipTensor y(Shape(nd), Storage::F32, device_);
        // ndarray sums a lane with its unrolled fold when the axis is the array's minimum-stride
        // axis with contiguous lanes (the last axis of a row-major array), else in axis order
        const std::vector<int64_t> cs = cur.ref_strides();
        const int lane = ndlayout::sums_with_lane_fold(d, cs, ax) ? 1 : 0;
        if (lane && inner > 1) {
            // the reference's lanes are contiguous along an axis that is not last on the device:
            // bring that axis last ([outer, inner, len]) and fold the rows
            const size_t len = d[ax];
            HipTensor tmp(Shape({outer, inner, len}), Storage::F32, device_);
            strided_copy({outer, inner, len}, (const float*)cur.data(),
                         {(int64_t)(len * inner), 1, (int64_t)inner}, (float*)tmp.data(),
                         row_major_strides({outer, inner, len}));
            check(hx_mean_axis_f32((int64_t)(outer * inner), (int64_t)len, 1, 1,
                                   (const float*)tmp.data(), (float*)y.data(), nullptr),
                  "hx_mean_axis_f32");
        } else {
            check(hx_mean_axis_f32((int64_t)outer, (int64_t)d[ax], (int64_t)inner, lane,
                                   (const float*)cur.data(), (float*)y.data(), nullptr),
                  "hx_mean_axis_f32");
        }
        y.set_ref_strides(ndlayout::mean_axis_result(d, cs, ax));
        cur = y;
    }
    return order.empty() ? clone() : cur;
}

// ----------------------------------------------------------------------------- TensorBroadcast
HipTensor HipTensor::broadcast_to(const Shape& target) const {
    need_f32(*this);
    const std::vector<size_t>& s = shape_.as_slice();
    const std::vector<size_t>& t = target.as_slice();
    const size_t sn = s.size(), tn = t.size();
    if (sn > tn) shape_mismatch({tn}, {sn});  // lib.rs:1356-1361
    if (shape_ == target) return clone();      // lib.rs:1364-1366
    need_standard_layout(*this, "broadcast_to");
    std::vector<size_t> padded(tn - sn, 1);
    padded.insert(padded.end(), s.begin(), s.end());
    for (size_t j = 0; j < tn; ++j)  // lib.rs:1373-1380
        if (padded[j] != 1 && padded[j] != t[j]) shape_mismatch({t[j]}, {padded[j]});
    std::vector<int64_t> src(tn, 0);
    if (sn == 1 && tn == 2) {  // lib.rs:1384-1428
        if (s[0] == t[1]) src = {0, 1};        // repeat rows
        else if (s[0] == t[0]) src = {1, 0};   // repeat columns
        else shape_mismatch({t[1]}, {s[0]});
    } else if (sn == 2 && tn == 3) {  // lib.rs:1429-1475
        if (s[0] == t[1] && s[1] == t[2]) src = {0, (int64_t)s[1], 1};
        else if (s[0] == 1 && s[1] == t[2]) src = {0, 0, 1};
        else shape_mismatch({t[1], t[2]}, {s[0], s[1]});
    } else if (sn == 1 && tn == 3) {  // lib.rs:1476-1505
        if (s[0] == t[2]) src = {0, 0, 1};
        else shape_mismatch({t[2]}, {s[0]});
    } else {
        // generic_broadcast_to (lib.rs:511-560) as written: target dim j reads the source with
        // stride self_strides[j] (the source's own row-major strides indexed by the TARGET dim,
        // 1 past the source's rank) where padded[j] != 1, else 0
        if (sn == 0) invalid_dimension(0, s);  // the reference's stride loop underflows (panic)
        const std::vector<int64_t> ss = row_major_strides(s);
        for (size_t j = 0; j < tn; ++j) src[j] = padded[j] != 1 ? (j < sn ? ss[j] : 1) : 0;
    }
    HipTensor y(target, Storage::F32, device_);
    if (y.numel()) strided_copy(t, (const float*)data(), src, (float*)y.data(), row_major_strides(t));
    return y;
}

// ----------------------------------------------------------------------------- shape operations
HipTensor HipTensor::transpose(size_t d0, size_t d1) const {
    const std::vector<size_t>& s = shape_.as_slice();
    if (d0 >= s.size() || d1 >= s.size()) invalid_dimension(std::max(d0, d1), s);  // lib.rs:116-122
    need_f32(*this);
    std::vector<size_t> nd(s);
    std::swap(nd[d0], nd[d1]);
    std::vector<int64_t> src = row_major_strides(s);
    std::swap(src[d0], src[d1]);
    HipTensor y(Shape(nd), Storage::F32, device_);
    if (y.numel()) strided_copy(nd, (const float*)data(), src, (float*)y.data(), row_major_strides(nd));
    y.set_ref_strides(ndlayout::transposed(ref_strides(), d0, d1));  // permuted_axes + to_owned
    return y;
}

HipTensor HipTensor::slice(const std::vector<size_t>& start, const std::vector<size_t>& end) const {
    const std::vector<size_t>& s = shape_.as_slice();
    if (start.size() != s.size() || end.size() != s.size())  // lib.rs:140-145
        shape_mismatch({s.size()}, {std::max(start.size(), end.size())});
    for (size_t i = 0; i < s.size(); ++i)  // lib.rs:148-156
        if (start[i] >= s[i] || end[i] > s[i] || start[i] >= end[i]) invalid_dimension(i, s);
    if (s.size() != 2)  // lib.rs:176-181
        unsupported("Slicing for " + std::to_string(s.size()) + "D tensors not implemented yet");
    need_f32(*this);
    const std::vector<size_t> nd = {end[0] - start[0], end[1] - start[1]};
    HipTensor y(Shape(nd), Storage::F32, device_);
    const float* base = (const float*)data() + start[0] * s[1] + start[1];
    strided_copy(nd, base, {(int64_t)s[1], 1}, (float*)y.data(), row_major_strides(nd));
    y.set_ref_strides(ndlayout::owned(nd, ref_strides()));  // to_owned of the sliced view
    return y;
}

HipTensor HipTensor::cat(const std::vector<HipTensor>& ts, size_t dim) {
    if (ts.empty()) unsupported("concatenation of empty tensor list");  // lib.rs:186-190
    if (ts.size() == 1) return ts[0].clone();
    const std::vector<size_t>& f = ts[0].shape().as_slice();
    if (dim >= f.size()) invalid_dimension(dim, f);
    for (size_t k = 1; k < ts.size(); ++k) {  // lib.rs:205-222
        const std::vector<size_t>& o = ts[k].shape().as_slice();
        if (o.size() != f.size()) shape_mismatch({f.size()}, {o.size()});
        for (size_t i = 0; i < f.size(); ++i)
            if (i != dim && f[i] != o[i]) shape_mismatch({f[i]}, {o[i]});
    }
    if (f.size() != 1)  // lib.rs:247-251
        unsupported("Concatenation for " + std::to_string(f.size()) + "D tensors not implemented yet");
    size_t total = 0;
    for (const HipTensor& t : ts) {
        need_f32(t);
        need_standard_layout(t, "cat");  // lib.rs:233
        total += t.numel();
    }
    HipTensor y(Shape({total}), Storage::F32, ts[0].device_);
    size_t off = 0;
    for (const HipTensor& t : ts) {
        if (t.numel())
            check(hx_memcpy_d2d((float*)y.data() + off, t.data(), t.nbytes(), nullptr), "hx_memcpy_d2d");
        off += t.numel();
    }
    return y;
}

HipTensor HipTensor::stack(const std::vector<HipTensor>& ts, size_t dim) {
    if (ts.empty()) unsupported("stacking of empty tensor list");  // lib.rs:255-259
    if (ts.size() == 1) return ts[0].clone();                      // lib.rs:261-263
    const Shape& f = ts[0].shape();
    for (size_t k = 1; k < ts.size(); ++k)  // lib.rs:266-273
        if (ts[k].shape() != f) shape_mismatch(f.as_slice(), ts[k].shape().as_slice());
    std::vector<size_t> out(f.as_slice());
    if (dim > out.size()) invalid_dimension(dim, out);  // Vec::insert panics past the end
    out.insert(out.begin() + (long)dim, ts.size());
    const size_t each = f.numel();
    HipTensor y(Shape(out), Storage::F32, ts[0].device_);
    const size_t nd = f.ndim();
    if (nd >= 1 && nd <= 3) {
        // lib.rs:278-333: the inputs' data back to back, whatever `dim` (only the shape field
        // carries it)
        for (size_t k = 0; k < ts.size(); ++k) {
            need_f32(ts[k]);
            need_standard_layout(ts[k], "stack");  // lib.rs:284, 301, 318
            if (each)
                check(hx_memcpy_d2d((float*)y.data() + k * each, ts[k].data(), each * 4, nullptr),
                      "hx_memcpy_d2d");
        }
        return y;
    }
    if (nd == 0) invalid_dimension(0, f.as_slice());  // generic_stack's stride loop underflows (panic)
    // generic_stack (lib.rs:390-467): input k's element at coordinates c goes to the output at
    // c with k inserted at `dim`
    size_t outer = 1, inner = 1;
    for (size_t i = 0; i < dim; ++i) outer *= f.dim(i);
    for (size_t i = dim; i < nd; ++i) inner *= f.dim(i);
    for (size_t k = 0; k < ts.size(); ++k) {
        need_f32(ts[k]);
        need_standard_layout(ts[k], "stack");  // lib.rs:413
        if (!each) continue;
        strided_copy({outer, inner}, (const float*)ts[k].data(), {(int64_t)inner, 1},
                     (float*)y.data() + k * inner, {(int64_t)(ts.size() * inner), 1});
    }
    return y;
}

// ----------------------------------------------------------------------------- exported S4Block
ExportedS4Block::ExportedS4Block(size_t d_model, size_t d_state, Rng& rng, int device)
    : d_model_(d_model), d_state_(d_state) {
    // crates/nn/src/lib.rs:687-726, same draw order
    A = HipTensor::random_normal(Shape({d_state, d_state}), 0.0f, 0.1f, rng, Storage::F32, device);
    B = HipTensor::random_normal(Shape({d_state, d_model}), 0.0f, 0.1f, rng, Storage::F32, device);
    C = HipTensor::random_normal(Shape({d_model, d_state}), 0.0f, 0.1f, rng, Storage::F32, device);
    D = HipTensor::zeros(Shape({d_model}), Storage::F32, device);
    delta = HipTensor::random_uniform(Shape({d_model}), 0.001f, 0.1f, rng, Storage::F32, device);
    Lambda = HipTensor::random_normal(Shape({d_state}), 0.0f, 1.0f, rng, Storage::F32, device);
}

HipTensor ExportedS4Block::forward_ssm(const HipTensor& x) const {
    // lib.rs:742-756: dim(0).unwrap(), dim(1).unwrap(), then Ok(input.clone())
    if (x.shape().ndim() < 2) invalid_dimension(x.shape().ndim(), x.shape().as_slice());
    return x.clone();
}

// ----------------------------------------------------------------------------- ssm::S4Block::forward
HipTensor S4Block::forward_conv(const HipTensor& input) const {
    // ssm.rs:189-229, statement for statement over HipTensor ops
    if (input.shape().ndim() < 2) invalid_dimension(input.shape().ndim(), input.shape().as_slice());
    const size_t batch_size = input.shape().dim(0), seq_len = input.shape().dim(1);
    // compute_conv_kernel (ssm.rs:232-251)
    std::vector<HipTensor> kernel;
    HipTensor a_power = HipTensor::eye(d_state_);
    HipTensor kernel_t = C.matmul(B);
    kernel.push_back(kernel_t);
    for (size_t k = 1; k < seq_len; ++k) {
        a_power = a_power.matmul(A_real);
        kernel_t = C.matmul(a_power).matmul(B);
        kernel.push_back(kernel_t);
    }
    const HipTensor K = HipTensor::stack(kernel, 0);
    std::vector<HipTensor> outputs;
    for (size_t b = 0; b < batch_size; ++b) {
        std::vector<HipTensor> output_seq;
        for (size_t t = 0; t < seq_len; ++t) {
            HipTensor output_t = HipTensor::zeros(Shape({d_model_}));
            for (size_t s = 0; s <= t; ++s) {
                HipTensor input_s = input.slice({b, s}, {b + 1, s + 1}).reshape(Shape({d_model_}));
                HipTensor kernel_ts = K.slice({t - s}, {t - s + 1}).reshape(Shape({d_state_}));
                HipTensor contribution = C.matmul(kernel_ts).mul(input_s);
                output_t = output_t.add(contribution);
            }
            output_seq.push_back(output_t);
        }
        outputs.push_back(HipTensor::stack(output_seq, 0));
    }
    return HipTensor::stack(outputs, 0);
}

// ----------------------------------------------------------------------------- generic nn bodies
namespace generic {

HipTensor linear(const HipTensor& x, const HipTensor& weight, const HipTensor* bias) {
    // Linear::forward (crates/nn/src/lib.rs:120-134)
    HipTensor output = x.matmul(weight.transpose(0, 1));
    if (bias) return output.add(bias->broadcast_to(output.shape()));
    return output;
}

HipTensor mamba_mlp(const HipTensor& x, const Linear& gate, const Linear& out_proj) {
    // exported MambaBlock::forward_mamba (lib.rs:888-906)
    if (x.shape().ndim() < 2) invalid_dimension(x.shape().ndim(), x.shape().as_slice());
    const HipTensor xz = linear(x, gate.weight(), &gate.bias());
    const HipTensor activated = xz.silu();
    return linear(activated, out_proj.weight(), &out_proj.bias());
}

HipTensor rmsnorm(const HipTensor& input, const HipTensor& weight, float eps) {
    // RMSNorm::forward (lib.rs:258-285); eps' = eps instead of a draw from U[eps, eps + 1e-8)
    const std::vector<size_t> last = {input.shape().ndim() - 1};
    const HipTensor mean_squared = input.mul(input).mean(&last, true);
    const HipTensor eps_tensor = HipTensor::from_scalar(eps, mean_squared.shape());
    const HipTensor rms = mean_squared.add(eps_tensor).sqrt();
    std::vector<size_t> expanded(rms.shape().as_slice());
    expanded.push_back(1);
    const HipTensor rms_b = rms.reshape(Shape(expanded)).broadcast_to(input.shape());
    const HipTensor normalized = input.div(rms_b);
    return normalized.mul(weight.broadcast_to(input.shape()));
}

HipTensor s4_forward_ssm(const S4Block& s4, const HipTensor& input) {
    // ssm::S4Block::forward_ssm (ssm.rs:138-186) with discretize(0.1) (ssm.rs:103-135)
    if (input.shape().ndim() < 2) invalid_dimension(input.shape().ndim(), input.shape().as_slice());
    const size_t batch_size = input.shape().dim(0), seq_len = input.shape().dim(1);
    const size_t d_model = s4.d_model(), d_state = s4.d_state();
    if (batch_size != d_model) shape_mismatch({d_model}, {batch_size});
    const float dt = 0.1f;
    const HipTensor dt_real = s4.A_real.mul_scalar(dt), dt_imag = s4.A_imag.mul_scalar(dt);
    const HipTensor A_d = dt_real.exp().mul(dt_imag.cos());
    const HipTensor B_d = s4.B.mul_scalar(dt);
    HipTensor state = HipTensor::zeros(Shape({d_state}));
    std::vector<HipTensor> outputs;
    for (size_t t = 0; t < seq_len; ++t) {
        const HipTensor input_t = input.slice({0, t}, {d_model, t + 1}).reshape(Shape({d_model}));
        const HipTensor state_update = A_d.mul(state);
        const HipTensor input_contribution = B_d.matmul(input_t);
        state = state_update.add(input_contribution);
        const HipTensor output_t = s4.C.matmul(state);
        const HipTensor feedthrough = s4.D.mul(input_t);
        outputs.push_back(output_t.add(feedthrough));
    }
    return HipTensor::stack(outputs, 1);
}

}  // namespace generic
}  // namespace helix
