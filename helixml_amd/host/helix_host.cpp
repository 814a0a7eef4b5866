// helix_host.cpp — the native host layer of include/helix/helix.hpp over the C ABI.
// Host code only (no kernels): shapes are checked here with the reference's error variants,
// then every computation is one or more hx_* calls.
#include "helix/helix.hpp"
#include "ndlayout.hpp"

#include <cmath>
#include <cstring>
#include <fstream>

#include "helix_hip.h"
#include "helix_detail.h"

namespace helix {

// ----------------------------------------------------------------------------- errors
TensorError TensorError::from_status(int status, const std::string& what) {
    ErrorKind k;
    switch (status) {
        case HX_ERR_SHAPE_MISMATCH: k = ErrorKind::ShapeMismatch; break;
        case HX_ERR_INVALID_DIMENSION: k = ErrorKind::InvalidDimension; break;
        case HX_ERR_DEVICE_MISMATCH: k = ErrorKind::DeviceMismatch; break;
        case HX_ERR_DTYPE_MISMATCH: k = ErrorKind::DTypeMismatch; break;
        case HX_ERR_UNSUPPORTED: k = ErrorKind::UnsupportedOperation; break;
        case HX_ERR_ALLOCATION: k = ErrorKind::AllocationFailed; break;
        case HX_ERR_SERIALIZATION: k = ErrorKind::SerializationError; break;
        case HX_ERR_INVALID_INPUT: k = ErrorKind::InvalidInput; break;
        case HX_ERR_INVALID_CHECKPOINT: k = ErrorKind::InvalidCheckpoint; break;
        default: k = ErrorKind::BackendError; break;
    }
    return TensorError(k, what);
}

void check(int status, const char* what) {
    if (status != HX_OK) throw TensorError::from_status(status, std::string(what) + ": " + hx_last_error());
}

namespace {
using detail::shape_mismatch;

uint16_t f32_to_bf16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    if ((x & 0x7f800000u) == 0x7f800000u && (x & 0x007fffffu)) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}
float bf16_to_f32(uint16_t b) {
    uint32_t x = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}
}  // namespace

// ----------------------------------------------------------------------------- Shape, Rng
size_t Shape::dim(size_t i) const {
    if (i >= dims_.size())
        throw TensorError(ErrorKind::InvalidDimension, "Invalid dimension: " + std::to_string(i) +
                                                           " is out of bounds");
    return dims_[i];
}

size_t Shape::numel() const {
    size_t n = 1;
    for (size_t d : dims_) n *= d;
    return n;
}

uint64_t Rng::next_u64() {  // SplitMix64 (Steele, Lea, Flood 2014)
    uint64_t z = (s_ += 0x9e3779b97f4a7c15ULL);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

float Rng::uniform(float lo, float hi) {
    const double u = (double)(next_u64() >> 11) * (1.0 / 9007199254740992.0);  // [0, 1)
    return (float)(lo + (hi - lo) * u);
}

float Rng::normal(float mean, float std) {  // Box-Muller, both values used
    if (have_spare_) {
        have_spare_ = false;
        return (float)(mean + std * spare_);
    }
    double u1;
    do {
        u1 = (double)(next_u64() >> 11) * (1.0 / 9007199254740992.0);
    } while (u1 <= 0.0);
    const double u2 = (double)(next_u64() >> 11) * (1.0 / 9007199254740992.0);
    const double r = std::sqrt(-2.0 * std::log(u1));
    spare_ = r * std::sin(2.0 * M_PI * u2);
    have_spare_ = true;
    return (float)(mean + std * r * std::cos(2.0 * M_PI * u2));
}

// ----------------------------------------------------------------------------- HipTensor
HipTensor::Buffer::Buffer(size_t bytes) {
    check(hx_malloc(&ptr, bytes ? bytes : 4), "hx_malloc");
}
HipTensor::Buffer::~Buffer() {
    if (ptr) (void)hx_free(ptr);
}

HipTensor::HipTensor(Shape shape, Storage st, int device)
    : shape_(std::move(shape)), storage_(st), device_(device) {
    buf_ = std::make_shared<Buffer>(nbytes());
}

HipTensor HipTensor::from_host(const std::vector<float>& values, Shape shape, Storage st, int device) {
    if (values.size() != shape.numel()) shape_mismatch({shape.numel()}, {values.size()});
    HipTensor t(std::move(shape), st, device);
    if (t.numel() == 0) return t;
    if (st == Storage::F32) {
        check(hx_memcpy_h2d(t.data(), values.data(), t.nbytes()), "hx_memcpy_h2d");
    } else {
        std::vector<uint16_t> b(values.size());
        for (size_t i = 0; i < b.size(); ++i) b[i] = f32_to_bf16(values[i]);
        check(hx_memcpy_h2d(t.data(), b.data(), t.nbytes()), "hx_memcpy_h2d");
    }
    return t;
}

HipTensor HipTensor::zeros(Shape shape, Storage st, int device) {
    std::vector<float> v(shape.numel(), 0.0f);
    return from_host(v, std::move(shape), st, device);
}

HipTensor HipTensor::ones(Shape shape, Storage st, int device) {
    std::vector<float> v(shape.numel(), 1.0f);
    return from_host(v, std::move(shape), st, device);
}

HipTensor HipTensor::random_normal(Shape shape, float mean, float std, Rng& rng, Storage st, int device) {
    std::vector<float> v(shape.numel());
    for (float& x : v) x = rng.normal(mean, std);
    return from_host(v, std::move(shape), st, device);
}

HipTensor HipTensor::random_uniform(Shape shape, float lo, float hi, Rng& rng, Storage st, int device) {
    std::vector<float> v(shape.numel());
    for (float& x : v) x = rng.uniform(lo, hi);
    return from_host(v, std::move(shape), st, device);
}

std::vector<float> HipTensor::to_host() const {
    std::vector<float> v(numel());
    if (v.empty()) return v;
    check(hx_sync(), "hx_sync");
    if (storage_ == Storage::F32) {
        check(hx_memcpy_d2h(v.data(), data(), nbytes()), "hx_memcpy_d2h");
    } else {
        std::vector<uint16_t> b(numel());
        check(hx_memcpy_d2h(b.data(), data(), nbytes()), "hx_memcpy_d2h");
        for (size_t i = 0; i < b.size(); ++i) v[i] = bf16_to_f32(b[i]);
    }
    return v;
}

HipTensor HipTensor::to_storage(Storage st) const {
    if (st == storage_) return *this;
    return from_host(to_host(), shape_, st, device_);
}

HipTensor HipTensor::reshape(Shape s) const {
    if (s.numel() != numel()) shape_mismatch({numel()}, {s.numel()});
    HipTensor t = *this;
    // lib.rs:94-113: to_shape(..).to_owned() keeps the strides a copy-free view has, else row-major
    std::vector<int64_t> st = ndlayout::reshaped(shape_.as_slice(), ref_strides(), s.as_slice());
    t.shape_ = std::move(s);
    t.strides_.clear();
    t.set_ref_strides(std::move(st));
    return t;
}

HipTensor HipTensor::clone() const {
    HipTensor t(shape_, storage_, device_);
    if (numel()) check(hx_memcpy_d2d(t.data(), data(), nbytes(), nullptr), "hx_memcpy_d2d");
    t.strides_ = strides_;  // an ndarray clone keeps its strides
    return t;
}

std::vector<int64_t> HipTensor::ref_strides() const {
    return strides_.empty() ? ndlayout::c_strides(shape_.as_slice()) : strides_;
}

void HipTensor::set_ref_strides(std::vector<int64_t> strides) {
    if (strides.size() != shape_.ndim())
        throw TensorError(ErrorKind::InvalidInput, "strides of rank " + std::to_string(strides.size()) +
                                                       " for a tensor of rank " +
                                                       std::to_string(shape_.ndim()));
    if (strides == ndlayout::c_strides(shape_.as_slice())) strides.clear();
    strides_ = std::move(strides);
}

bool HipTensor::is_contiguous() const {
    return strides_.empty() || ndlayout::is_standard_layout(shape_.as_slice(), strides_);
}

// ----------------------------------------------------------------------------- nn
Linear::Linear(size_t in_f, size_t out_f, Rng& rng, int device)
    : weight_(HipTensor::random_normal(Shape({out_f, in_f}), 0.0f, std::sqrt(2.0f / (float)in_f), rng,
                                       Storage::F32, device)),
      bias_(HipTensor::zeros(Shape({out_f}), Storage::F32, device)) {}

namespace {
HipTensor linear_impl(const HipTensor& x, const HipTensor& w, const HipTensor& b, int act) {
    if (x.shape().ndim() != 2)
        throw TensorError(ErrorKind::UnsupportedOperation, "Operation not supported: Linear on rank " +
                                                               std::to_string(x.shape().ndim()));
    const size_t R = x.shape().dim(0), IN = x.shape().dim(1), OUT = w.shape().dim(0);
    if (w.shape().dim(1) != IN) shape_mismatch({IN}, {w.shape().dim(1)});
    HipTensor y(Shape({R, OUT}), Storage::F32, 0);
    check(hx_linear_f32((int64_t)R, (int64_t)IN, (int64_t)OUT, (const float*)x.data(),
                        (const float*)w.data(), b.defined() ? (const float*)b.data() : nullptr, act,
                        (float*)y.data(), nullptr),
          "hx_linear_f32");
    return y;
}
}  // namespace

HipTensor Linear::forward(const HipTensor& x) const { return linear_impl(x, weight_, bias_, 0); }
HipTensor Linear::forward_silu(const HipTensor& x) const { return linear_impl(x, weight_, bias_, 1); }

RMSNorm::RMSNorm(size_t d_model, float eps, int device)
    : weight_(HipTensor::ones(Shape({d_model}), Storage::F32, device)), eps_(eps) {}

HipTensor RMSNorm::forward(const HipTensor& x, Storage out) const {
    const size_t dim = weight_.numel();
    if (x.shape().ndim() == 0 || x.shape().dim(x.shape().ndim() - 1) != dim)
        shape_mismatch({dim}, {x.shape().ndim() ? x.shape().dim(x.shape().ndim() - 1) : 0});
    HipTensor y(x.shape(), out, 0);
    check(hx_rmsnorm_fwd((int64_t)(x.numel() / dim), (int64_t)dim, (const float*)x.data(),
                         (const float*)weight_.data(), eps_, out == Storage::BF16 ? HX_BF16 : HX_F32,
                         y.data(), nullptr),
          "hx_rmsnorm_fwd");
    return y;
}

MambaBlock::MambaBlock(size_t d_model, size_t /*d_state*/, size_t /*d_conv*/, size_t expand, Rng& rng,
                       int device)
    : gate_(d_model, d_model * expand, rng, device), out_proj_(d_model * expand, d_model, rng, device) {}

HipTensor MambaBlock::forward(const HipTensor& x) const {
    // forward_mamba (lib.rs:888-906): xz = gate(x); silu; out_proj — SiLU fused into the first GEMM
    return out_proj_.forward(gate_.forward_silu(x));
}

S4Block::S4Block(size_t d_model, size_t d_state, Rng& rng, int device)
    : d_model_(d_model), d_state_(d_state) {
    // ssm.rs:39-83, same order of draws
    A_real = HipTensor::zeros(Shape({d_state}), Storage::F32, device);
    A_imag = HipTensor::random_normal(Shape({d_state}), 0.0f, 1.0f, rng, Storage::F32, device);
    B = HipTensor::random_normal(Shape({d_state, d_model}), 0.0f, 0.1f, rng, Storage::F32, device);
    C = HipTensor::random_normal(Shape({d_model, d_state}), 0.0f, 0.1f, rng, Storage::F32, device);
    D = HipTensor::zeros(Shape({d_model}), Storage::F32, device);
    delta = HipTensor::random_uniform(Shape({d_model}), 0.001f, 0.1f, rng, Storage::F32, device);
    Lambda = HipTensor::random_normal(Shape({d_state}), 0.0f, 1.0f, rng, Storage::F32, device);
}

HipTensor S4Block::forward_ssm(const HipTensor& x, const HipTensor* gate, bool parallel) const {
    const size_t M = x.shape().dim(0), L = x.shape().dim(1);
    if (M != d_model_) shape_mismatch({d_model_}, {M});  // ssm.rs:142-147
    // y memory is [L, d_model]; the reference's shape field is [d_model, L] (CpuTensor::stack(., 1),
    // backend-cpu/src/lib.rs:277-296), or [d_model] when L == 1 (lib.rs:261-263)
    HipTensor y(L == 1 ? Shape({M}) : Shape({M, L}), Storage::F32, 0);
    const float dt = 0.1f;  // ssm.rs:151
    if (!a_disc_.defined() || a_src_[0] != A_real.data() || a_src_[1] != A_imag.data()) {
        // discretize(dt) (ssm.rs:113-120) on the host with the reference's libm, once per
        // parameter buffer rather than per forward
        const std::vector<float> ar = A_real.to_host(), ai = A_imag.to_host();
        std::vector<float> a(d_state_);
        check(hx_s4_discretize((int64_t)d_state_, dt, ar.data(), ai.data(), a.data()),
              "hx_s4_discretize");
        a_disc_ = HipTensor::from_host(a, Shape({d_state_}), Storage::F32, 0);
        a_src_[0] = A_real.data();
        a_src_[1] = A_imag.data();
    }
    const size_t need = parallel ? hx_s4_ref_parallel_workspace_size((int64_t)M, (int64_t)d_state_, (int64_t)L)
                                 : hx_s4_ref_workspace_size((int64_t)M, (int64_t)d_state_, (int64_t)L);
    if (!workspace_.defined() || workspace_.nbytes() < need)
        workspace_ = HipTensor(Shape({(need + 3) / 4}), Storage::F32, 0);
    auto fn = parallel ? hx_s4_ref_fwd_parallel : hx_s4_ref_fwd;
    check(fn((int64_t)M, (int64_t)d_state_, (int64_t)L, dt, (const float*)x.data(),
             (const float*)a_disc_.data(), (const float*)B.data(), (const float*)C.data(),
             (const float*)D.data(), gate ? (const float*)gate->data() : nullptr, (float*)y.data(),
             workspace_.data(), workspace_.nbytes(), nullptr),
          parallel ? "hx_s4_ref_fwd_parallel" : "hx_s4_ref_fwd");
    return y;
}

std::vector<HipTensor> S4Block::checkpoint() const {
    return {A_real.clone(), A_imag.clone(), B.clone(), C.clone(), D.clone(), delta.clone(), Lambda.clone()};
}

void S4Block::restore(const std::vector<HipTensor>& ck) {
    if (ck.size() != 7)  // ssm.rs:345-350
        throw TensorError(ErrorKind::InvalidCheckpoint, "Invalid checkpoint: expected 7 parameters, got " +
                                                            std::to_string(ck.size()));
    A_real = ck[0].clone();
    A_imag = ck[1].clone();
    parameters_changed();  // a new buffer may reuse a freed one's address
    B = ck[2].clone();
    C = ck[3].clone();
    D = ck[4].clone();
    delta = ck[5].clone();
    Lambda = ck[6].clone();
}

SsmMambaBlock::SsmMambaBlock(size_t d_model, size_t d_state, Rng& rng, int device)
    : s4(d_model, d_state, rng, device) {
    // ssm.rs:385-418
    delta_proj = HipTensor::random_normal(Shape({d_model, d_model}), 0.0f, 0.1f, rng, Storage::F32, device);
    B_proj = HipTensor::random_normal(Shape({d_model, d_state}), 0.0f, 0.1f, rng, Storage::F32, device);
    C_proj = HipTensor::random_normal(Shape({d_model, d_state}), 0.0f, 0.1f, rng, Storage::F32, device);
    gate = HipTensor::random_normal(Shape({d_model}), 0.0f, 0.1f, rng, Storage::F32, device);
}

HipTensor SsmMambaBlock::forward_mamba(const HipTensor& x) const {
    // ssm.rs:435-464: delta = X . delta_proj; the B and C projections are computed and discarded
    // there (same shape constraint as delta's, so skipping them changes no result or error);
    // y = S4.forward_ssm(delta) * broadcast(gate)
    const HipTensor delta_ = x.matmul(delta_proj);
    return s4.forward_ssm(delta_, &gate);
}

MambaBlockFused::MambaBlockFused(size_t dm, size_t ds, size_t dc, size_t expand, Rng& rng, int device,
                                 size_t r)
    : d_model(dm), d_state(ds), d_conv(dc), d_inner(dm * expand), dt_rank(r ? r : (dm + 15) / 16) {
    const size_t di = d_inner;
    w_in = HipTensor::random_normal(Shape({2 * di, dm}), 0.0f, std::sqrt(2.0f / dm), rng, Storage::BF16, device);
    const float cb = 1.0f / std::sqrt((float)dc);
    conv_w = HipTensor::random_uniform(Shape({di, dc}), -cb, cb, rng, Storage::F32, device);
    conv_b = HipTensor::random_uniform(Shape({di}), -cb, cb, rng, Storage::F32, device);
    w_x = HipTensor::random_normal(Shape({dt_rank + 2 * ds, di}), 0.0f, std::sqrt(2.0f / di), rng,
                                   Storage::BF16, device);
    w_dt = HipTensor::random_normal(Shape({di, dt_rank}), 0.0f, 1.0f / std::sqrt((float)dt_rank), rng,
                                    Storage::BF16, device);
    std::vector<float> bias(di), a(di * ds), dv(di, 1.0f);
    for (size_t i = 0; i < di; ++i) {  // dt = softplus(dt_bias) log-uniform in [1e-3, 1e-1]
        const double dt0 = std::exp(std::log(1e-3) + rng.uniform(0.0f, 1.0f) * (std::log(0.1) - std::log(1e-3)));
        bias[i] = (float)(dt0 + std::log(-std::expm1(-dt0)));
        for (size_t n = 0; n < ds; ++n) a[i * ds + n] = -(float)(n + 1);
    }
    dt_bias = HipTensor::from_host(bias, Shape({di}), Storage::F32, device);
    A = HipTensor::from_host(a, Shape({di, ds}), Storage::F32, device);
    D = HipTensor::from_host(dv, Shape({di}), Storage::F32, device);
    w_out = HipTensor::random_normal(Shape({dm, di}), 0.0f, std::sqrt(2.0f / di), rng, Storage::BF16, device);
}

HipTensor MambaBlockFused::forward(const HipTensor& x) const {
    if (x.shape().ndim() != 3 || x.shape().dim(2) != d_model) shape_mismatch({d_model}, x.shape().as_slice());
    if (x.storage() != Storage::BF16)
        throw TensorError(ErrorKind::DTypeMismatch, "DType mismatch: expected bf16 storage");
    const size_t bt = x.shape().dim(0), L = x.shape().dim(1);
    const size_t need = hx_mamba_block_workspace_size((int64_t)bt, (int64_t)L, (int64_t)d_inner,
                                                      (int64_t)dt_rank, (int64_t)d_state);
    if (!workspace_.defined() || workspace_.nbytes() < need)
        workspace_ = HipTensor(Shape({(need + 3) / 4}), Storage::F32, 0);
    HipTensor out(x.shape(), Storage::BF16, 0);
    check(hx_mamba_block_fwd((int64_t)bt, (int64_t)L, (int64_t)d_model, (int64_t)d_inner,
                             (int64_t)d_state, (int64_t)dt_rank, (int64_t)d_conv, x.data(), w_in.data(),
                             (const float*)conv_w.data(), (const float*)conv_b.data(), w_x.data(),
                             w_dt.data(), (const float*)dt_bias.data(), (const float*)A.data(),
                             (const float*)D.data(), w_out.data(), out.data(), workspace_.data(),
                             workspace_.nbytes(), nullptr),
          "hx_mamba_block_fwd");
    return out;
}

HipTensor selective_scan(const HipTensor& u, const HipTensor& delta, const HipTensor& A,
                         const HipTensor& B, const HipTensor& C, const HipTensor* D, const HipTensor* z,
                         const HipTensor* dt_bias, bool softplus, HipTensor* last_state) {
    if (u.shape().ndim() != 3) shape_mismatch({3}, {u.shape().ndim()});
    const size_t bt = u.shape().dim(0), L = u.shape().dim(1), dim = u.shape().dim(2);
    const size_t N = A.shape().dim(1);
    if (delta.shape() != u.shape()) shape_mismatch(u.shape().as_slice(), delta.shape().as_slice());
    if (B.shape() != Shape({bt, L, N})) shape_mismatch({bt, L, N}, B.shape().as_slice());
    if (C.shape() != Shape({bt, L, N})) shape_mismatch({bt, L, N}, C.shape().as_slice());
    HipTensor out(u.shape(), u.storage(), 0);
    if (last_state) *last_state = HipTensor(Shape({bt, dim, N}), Storage::F32, 0);
    const int dt = u.storage() == Storage::BF16 ? HX_BF16 : HX_F32;
    // the long-sequence path (time segments with a carry) needs scratch: kept per thread and
    // grown on demand (this thread's calls are ordered on the default stream, so they share it)
    thread_local HipTensor ws;
    const size_t need = hx_selective_scan_workspace_size((int64_t)bt, (int64_t)L, (int64_t)dim, (int64_t)N, dt);
    if (need && (!ws.defined() || ws.nbytes() < need)) ws = HipTensor(Shape({(need + 3) / 4}), Storage::F32, 0);
    check(hx_selective_scan_fwd_ws((int64_t)bt, (int64_t)L, (int64_t)dim, (int64_t)N, dt, softplus ? 1 : 0,
                                   u.data(), delta.data(), (const float*)A.data(), B.data(), C.data(),
                                   D ? (const float*)D->data() : nullptr, z ? z->data() : nullptr,
                                   dt_bias ? (const float*)dt_bias->data() : nullptr, out.data(), nullptr,
                                   last_state ? (float*)last_state->data() : nullptr,
                                   need ? ws.data() : nullptr, need ? ws.nbytes() : 0, nullptr),
          "hx_selective_scan_fwd_ws");
    return out;
}

// ----------------------------------------------------------------------------- checkpoint
// bincode 1.x default options (as `bincode::serialize`): little-endian, fixed-width integers,
// sequence lengths as u64, enum variants as u32 indices, structs as their fields in order.
// CpuTensor (backend-cpu/src/lib.rs:23-29) = { data: ArrayD<f32>, shape: Shape, dtype: DType,
// device: Device }; ndarray 0.15 serialises an array as { v: u8 = 1, dim: [usize], data: [elem] }.
namespace {
struct Writer {
    std::vector<uint8_t> b;
    template <typename T>
    void put(T v) {
        const size_t o = b.size();
        b.resize(o + sizeof(T));
        std::memcpy(b.data() + o, &v, sizeof(T));  // little-endian host (x86-64)
    }
};

struct Reader {
    const std::vector<uint8_t>& b;
    size_t o = 0;
    template <typename T>
    T get() {
        if (b.size() - o < sizeof(T))
            throw TensorError(ErrorKind::SerializationError, "Serialization error: truncated parameters");
        T v;
        std::memcpy(&v, b.data() + o, sizeof(T));
        o += sizeof(T);
        return v;
    }
    uint64_t len(size_t elem_bytes) {
        const uint64_t n = get<uint64_t>();
        if (elem_bytes && n > (b.size() - o) / elem_bytes)
            throw TensorError(ErrorKind::SerializationError, "Serialization error: length past end");
        return n;
    }
};
}  // namespace

std::vector<uint8_t> encode_params(const std::vector<HostTensor>& params) {
    Writer w;
    w.put<uint64_t>(params.size());
    for (const HostTensor& t : params) {
        size_t n = 1;
        for (size_t d : t.shape) n *= d;
        if (n != t.values.size()) shape_mismatch({n}, {t.values.size()});
        w.put<uint8_t>(1);                   // ndarray format version
        w.put<uint64_t>(t.shape.size());     // dim: IxDyn
        for (size_t d : t.shape) w.put<uint64_t>(d);
        w.put<uint64_t>(t.values.size());    // data, logical order
        for (float f : t.values) w.put<float>(f);
        w.put<uint64_t>(t.shape.size());     // shape: Shape { dims: Vec<usize> }
        for (size_t d : t.shape) w.put<uint64_t>(d);
        w.put<uint32_t>((uint32_t)DType::F32);          // dtype
        w.put<uint32_t>((uint32_t)Device::Kind::Cpu);   // device: the bytes CpuTensor writes
    }
    return w.b;
}

std::vector<HostTensor> decode_params(const std::vector<uint8_t>& bytes) {
    Reader r{bytes};
    auto bad = [](const std::string& m) {
        return TensorError(ErrorKind::SerializationError, "Serialization error: " + m);
    };
    const uint64_t count = r.len(1);
    std::vector<HostTensor> out;
    for (uint64_t i = 0; i < count; ++i) {
        if (r.get<uint8_t>() != 1) throw bad("unknown ndarray format version");
        const uint64_t nd = r.len(8);
        std::vector<size_t> dims(nd);
        for (auto& d : dims) d = (size_t)r.get<uint64_t>();
        const uint64_t n = r.len(4);
        HostTensor t;
        t.values.resize(n);
        for (auto& f : t.values) f = r.get<float>();
        const uint64_t nd2 = r.len(8);
        t.shape.resize(nd2);
        for (auto& d : t.shape) d = (size_t)r.get<uint64_t>();
        if (r.get<uint32_t>() != (uint32_t)DType::F32) throw bad("only F32 tensors are supported");
        const uint32_t dev = r.get<uint32_t>();
        switch ((Device::Kind)dev) {
            case Device::Kind::Cpu: case Device::Kind::Metal: case Device::Kind::Wgpu: break;
            case Device::Kind::Cuda: case Device::Kind::Qpu: case Device::Kind::Npu:
            case Device::Kind::Tpu: (void)r.get<uint64_t>(); break;
            case Device::Kind::Custom: {
                const uint64_t sl = r.len(1);
                r.o += sl;
                break;
            }
            default: throw bad("unknown device variant");
        }
        size_t nd_el = 1, ns_el = 1;
        for (size_t d : dims) nd_el *= d;
        for (size_t d : t.shape) ns_el *= d;
        // the array dim is the storage layout and the Shape field the logical shape; they hold
        // the same number of elements (they differ only for the reference's S4 output quirk)
        if (nd_el != n || ns_el != n) throw bad("dims do not match the data length");
        out.push_back(std::move(t));
    }
    if (r.o != bytes.size()) throw bad("trailing bytes after the parameters");
    return out;
}

void save_checkpoint(const std::string& path, const std::string& metadata_json,
                     const std::vector<HostTensor>& params) {
    const std::vector<uint8_t> body = encode_params(params);
    std::ofstream f(path, std::ios::binary | std::ios::trunc);
    if (!f) throw TensorError(ErrorKind::SerializationError, "Serialization error: cannot open " + path);
    const uint32_t n = (uint32_t)metadata_json.size();
    const uint8_t be[4] = {(uint8_t)(n >> 24), (uint8_t)(n >> 16), (uint8_t)(n >> 8), (uint8_t)n};
    f.write((const char*)be, 4);  // tokio write_u32: big-endian (checkpoint.rs:161-162)
    f.write(metadata_json.data(), (std::streamsize)metadata_json.size());
    f.write((const char*)body.data(), (std::streamsize)body.size());
    if (!f) throw TensorError(ErrorKind::SerializationError, "Serialization error: write failed " + path);
}

std::pair<std::string, std::vector<HostTensor>> load_checkpoint_host(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw TensorError(ErrorKind::SerializationError, "Serialization error: cannot open " + path);
    std::vector<uint8_t> all((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    if (all.size() < 4) throw TensorError(ErrorKind::SerializationError, "Serialization error: short file");
    const uint32_t n = ((uint32_t)all[0] << 24) | ((uint32_t)all[1] << 16) | ((uint32_t)all[2] << 8) | all[3];
    if (all.size() - 4 < n) throw TensorError(ErrorKind::SerializationError, "Serialization error: short metadata");
    std::string meta((const char*)all.data() + 4, n);
    std::vector<uint8_t> body(all.begin() + 4 + n, all.end());
    return {meta, decode_params(body)};
}

void save_checkpoint(const std::string& path, const std::string& metadata_json,
                     const std::vector<HipTensor>& params) {
    std::vector<HostTensor> h;
    for (const HipTensor& t : params) h.push_back({t.shape().as_slice(), t.to_host()});
    save_checkpoint(path, metadata_json, h);
}

std::pair<std::string, std::vector<HipTensor>> load_checkpoint(const std::string& path, int device) {
    auto [meta, h] = load_checkpoint_host(path);
    std::vector<HipTensor> out;
    for (const HostTensor& t : h) out.push_back(HipTensor::from_host(t.values, Shape(t.shape), Storage::F32, device));
    return {meta, std::move(out)};
}

}  // namespace helix
