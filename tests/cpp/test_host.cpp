// test_host.cpp — tests of the native C++ host layer (include/helix/helix.hpp), written the way
// the reference's own Rust tests read (crates/backend-cpu/src/lib.rs:1733-1758,
// crates/training/src/checkpoint.rs:290+, crates/nn tests): construct modules, run forward,
// compare. GPU results are checked against the C oracle (oracle/hx_oracle.c, linked here as test
// infrastructure), bit for bit where the device path reproduces the reference's f32 order.
//
//   helix_host_tests --cpu [checkpoint_path]   host-only tests (no GPU touched); writes a
//                                               checkpoint of known tensors for the Python
//                                               cross-check of the byte format
//   helix_host_tests --gpu                     device tests
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "helix/helix.hpp"
#include "helix_hip.h"
#include "ndlayout.hpp"

extern "C" {
void oracle_matmul(int64_t M, int64_t K, int64_t N, const float* A, const float* B, float* Y);
void oracle_linear(int64_t R, int64_t IN, int64_t OUT, const float* X, const float* W,
                   const float* bias, int act, float* Y);
void oracle_mamba_mlp(int64_t R, int64_t d_model, int64_t d_inner, const float* X, const float* Wg,
                      const float* bg, const float* Wo, const float* bo, float* tmp, float* Y);
void oracle_rmsnorm(int64_t R, int64_t Dm, const float* X, const float* w, float eps, float* Y);
void oracle_s4_ref_fwd(int64_t M, int64_t N, int64_t L, float dt, const float* x,
                       const float* a_real, const float* a_imag, const float* B, const float* C,
                       const float* D, const float* gate, float* y, float* work);
void oracle_ssm_mamba_fwd(int64_t M, int64_t N, float dt, const float* X, const float* delta_proj,
                          const float* a_real, const float* a_imag, const float* B, const float* C,
                          const float* D, const float* gate, float* y, float* work);
void oracle_unary(int op, int64_t n, const float* x, float s, float* y);
void oracle_mean_axis(int64_t outer, int64_t len, int64_t inner, int lane_fold, const float* x,
                      float* y);
void oracle_rmsnorm_ref(int64_t R, int64_t Dm, const float* X, const float* w, float eps, float* Y,
                        float* work);
void oracle_selective_scan(int64_t Bt, int64_t L, int64_t Dd, int64_t N, int delta_softplus,
                           const float* u, const float* delta, const float* A, const float* Bm,
                           const float* Cm, const float* D, const float* z, const float* dt_bias,
                           float* out, const float* init_state, float* last_state);
}

using namespace helix;

namespace {
int g_fail = 0, g_run = 0;
std::string g_cur;

#define CHECK(cond)                                                                        \
    do {                                                                                   \
        if (!(cond)) {                                                                     \
            std::printf("  FAIL %s: %s (line %d)\n", g_cur.c_str(), #cond, __LINE__);      \
            ++g_fail;                                                                      \
            return;                                                                        \
        }                                                                                  \
    } while (0)

template <typename F>
bool throws_kind(F&& f, ErrorKind k, std::string* msg = nullptr) {
    try {
        f();
    } catch (const TensorError& e) {
        if (msg) *msg = e.what();
        return e.kind() == k;
    }
    return false;
}

bool bits_equal(const std::vector<float>& a, const std::vector<float>& b) {
    return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * 4) == 0;
}

double rel_err(const std::vector<float>& g, const std::vector<float>& r) {
    double amax = 0.0, e = 0.0;
    for (float v : r) amax = std::fmax(amax, std::fabs(v));
    const double floor = 1e-3 * (amax > 0 ? amax : 1e-30);
    for (size_t i = 0; i < g.size(); ++i)
        e = std::fmax(e, std::fabs((double)g[i] - r[i]) / std::fmax(std::fabs((double)r[i]), floor));
    return e;
}

struct Case {
    const char* name;
    bool gpu;
    std::function<void()> fn;
};
std::vector<Case>& cases() {
    static std::vector<Case> c;
    return c;
}
struct Reg {
    Reg(const char* n, bool gpu, std::function<void()> f) { cases().push_back({n, gpu, std::move(f)}); }
};
#define TEST_CPU(name) static void name(); static Reg reg_##name(#name, false, name); static void name()
#define TEST_GPU(name) static void name(); static Reg reg_##name(#name, true, name); static void name()

std::vector<float> randn(size_t n, uint64_t seed, float std = 1.0f) {
    Rng r(seed);
    std::vector<float> v(n);
    for (auto& x : v) x = r.normal(0.0f, std);
    return v;
}

std::string g_ckpt_path;
}  // namespace

// ============================================================================ host-only tests
TEST_CPU(shape_dim_out_of_range_is_invalid_dimension) {
    Shape s({2, 3});
    CHECK(s.numel() == 6 && s.dim(1) == 3);
    CHECK(throws_kind([&] { (void)s.dim(2); }, ErrorKind::InvalidDimension));
}

TEST_CPU(rng_normal_and_uniform_moments) {
    Rng r(0x48454C49);
    double s = 0, s2 = 0, umin = 1e9, umax = -1e9;
    const int n = 200000;
    for (int i = 0; i < n; ++i) {
        const double x = r.normal(0.0f, 0.1f);
        s += x;
        s2 += x * x;
        const double u = r.uniform(0.001f, 0.1f);
        umin = std::fmin(umin, u);
        umax = std::fmax(umax, u);
    }
    const double mean = s / n, sd = std::sqrt(s2 / n - mean * mean);
    CHECK(std::fabs(mean) < 1e-3 && std::fabs(sd - 0.1) < 1e-3);
    CHECK(umin >= 0.001 && umax < 0.1 && umin < 0.0011 && umax > 0.0999);
}

TEST_CPU(status_codes_map_to_tensor_error_variants) {
    CHECK(TensorError::from_status(1, "").kind() == ErrorKind::ShapeMismatch);
    CHECK(TensorError::from_status(5, "").kind() == ErrorKind::UnsupportedOperation);
    CHECK(TensorError::from_status(8, "").kind() == ErrorKind::SerializationError);
    CHECK(TensorError::from_status(9, "").kind() == ErrorKind::InvalidInput);
    CHECK(TensorError::from_status(10, "").kind() == ErrorKind::InvalidCheckpoint);
    CHECK(TensorError::from_status(7, "").kind() == ErrorKind::BackendError);
}

TEST_CPU(checkpoint_bytes_round_trip) {
    std::vector<HostTensor> p = {{{3}, {1.0f, -2.5f, 3.25f}},
                                 {{2, 2}, {0.0f, -0.0f, 1e-30f, 7.0f}},
                                 {{}, {42.0f}},
                                 {{0, 4}, {}}};
    const auto bytes = encode_params(p);
    // Vec length 4 (u64 LE) first
    CHECK(bytes.size() > 8 && bytes[0] == 4 && bytes[1] == 0 && bytes[7] == 0);
    const auto q = decode_params(bytes);
    CHECK(q.size() == p.size());
    for (size_t i = 0; i < p.size(); ++i) {
        CHECK(q[i].shape == p[i].shape);
        CHECK(bits_equal(q[i].values, p[i].values));
    }
    // truncation and trailing bytes are serialization errors
    auto cut = bytes;
    cut.pop_back();
    CHECK(throws_kind([&] { (void)decode_params(cut); }, ErrorKind::SerializationError));
    auto extra = bytes;
    extra.push_back(0);
    CHECK(throws_kind([&] { (void)decode_params(extra); }, ErrorKind::SerializationError));
    // a count that cannot fit the buffer is refused before allocating
    auto huge = bytes;
    huge[6] = 0x7f;
    CHECK(throws_kind([&] { (void)decode_params(huge); }, ErrorKind::SerializationError));
}

TEST_CPU(checkpoint_file_layout) {
    const std::string meta = "{\"epoch\":3,\"step\":120}";
    std::vector<HostTensor> p = {{{2, 3}, {1, 2, 3, 4, 5, 6}}, {{4}, {0.5f, -0.5f, 0.25f, 8.0f}}};
    const std::string path = g_ckpt_path.empty() ? "/tmp/helix_ckpt_test.bin" : g_ckpt_path;
    save_checkpoint(path, meta, p);
    auto [m2, q] = load_checkpoint_host(path);
    CHECK(m2 == meta);
    CHECK(q.size() == 2 && q[0].shape == p[0].shape && bits_equal(q[1].values, p[1].values));
    FILE* f = std::fopen(path.c_str(), "rb");
    CHECK(f);
    unsigned char hdr[4];
    CHECK(std::fread(hdr, 1, 4, f) == 4);
    std::fclose(f);
    CHECK(hdr[0] == 0 && hdr[1] == 0 && hdr[2] == 0 && hdr[3] == meta.size());  // u32 big-endian
}

TEST_CPU(operation_type_is_the_reference_enum) {
    // hal/src/device.rs:129-210: 57 variants, this order
    CHECK(std::string(operation_name(OperationType::Add)) == "Add");
    CHECK(std::string(operation_name(OperationType::SSMForward)) == "SSMForward");
    CHECK((int)OperationType::SSMForward == 44 && (int)OperationType::StateUpdate == 46);
    CHECK((int)OperationType::SignalFiltering == 56);
    CHECK(std::string(operation_name(OperationType::SignalFiltering)) == "SignalFiltering");
    CHECK(std::string(operation_name(OperationType::Log10)) == "Log10");
}

TEST_CPU(compute_graph_build_sort_and_cycle) {
    // operations.rs:88-231: edges from -> to; inputs have no incoming edge, outputs no outgoing
    ComputeGraph g;
    for (int i = 0; i < 5; ++i) g.add_operation(Operation(OperationType::Add));
    g.add_dependency(3, 1);
    g.add_dependency(1, 0);
    g.add_dependency(3, 4);
    g.add_dependency(4, 0);
    g.build();
    CHECK((g.input_nodes() == std::vector<size_t>{2, 3}));
    CHECK((g.output_nodes() == std::vector<size_t>{0, 2}));
    const auto order = g.topological_sort();
    CHECK(order.size() == 5);
    auto pos = [&](size_t n) { return std::find(order.begin(), order.end(), n) - order.begin(); };
    CHECK(pos(3) < pos(1) && pos(1) < pos(0) && pos(3) < pos(4) && pos(4) < pos(0));
    CHECK(throws_kind([&] { g.add_dependency(0, 9); }, ErrorKind::InvalidInput));
    g.add_dependency(0, 3);  // closes 3 -> 1 -> 0 -> 3
    std::string msg;
    CHECK(throws_kind([&] { (void)g.topological_sort(); }, ErrorKind::InvalidInput, &msg));
    CHECK(msg.find("Circular dependency detected") != std::string::npos);
}

// ndarray 0.15's layout rules as the mirror restates them, on hand-derived cases
TEST_CPU(ndarray_layout_rules) {
    namespace L = helix::ndlayout;
    using S = L::Strides;
    // row-major [2, 3]: the last axis is the minimum-stride axis and folds its lanes
    CHECK((L::c_strides({2, 3}) == S{3, 1}) && (L::f_strides({2, 3}) == S{1, 2}));
    CHECK(L::min_stride_axis({2, 3}, {3, 1}) == 1);
    CHECK(L::sums_with_lane_fold({2, 3}, {3, 1}, 1) && !L::sums_with_lane_fold({2, 3}, {3, 1}, 0));
    // transpose of row-major [3, 2] -> [2, 3] with strides (1, 2): F order, contiguous in memory
    // order, not standard; axis 0 now folds its lanes and axis 1 sums in order
    const S t = L::transposed({2, 1}, 0, 1);
    CHECK((t == S{1, 2}));
    CHECK(L::is_contiguous({2, 3}, t) && !L::is_standard_layout({2, 3}, t));
    CHECK(L::array_layout({2, 3}, t) == (L::kFOrder | L::kFPrefer));
    CHECK(L::min_stride_axis({2, 3}, t) == 0);
    CHECK(L::sums_with_lane_fold({2, 3}, t, 0) && !L::sums_with_lane_fold({2, 3}, t, 1));
    // a length-1 axis carries any stride: [3, 1] -> [1, 3] stays standard
    CHECK(L::is_standard_layout({1, 3}, L::transposed({1, 1}, 0, 1)));
    // ties in |stride| go to the later axis
    CHECK(L::min_stride_axis({3, 1}, {1, 1}) == 1 && L::min_stride_axis({3, 1}, {1, 3}) == 0);
    // binary ops collect F only when the Zip prefers F: F + F -> F, F + C -> C (tendencies cancel)
    CHECK((L::collect({2, 3}, {t, t}) == S{1, 2}));
    CHECK((L::collect({2, 3}, {t, {3, 1}}) == S{3, 1}));
    // 3-D: full reversal is F; swapping the outer two axes of [2, 3, 4] leaves only a C
    // preference (last stride 1), and F + that prefers F (tendency -2 + 1)
    const S f3 = L::transposed({12, 4, 1}, 0, 2);  // [4, 3, 2]
    CHECK((f3 == S{1, 4, 12}) && L::array_layout({4, 3, 2}, f3) == (L::kFOrder | L::kFPrefer));
    const S p3 = L::transposed({12, 4, 1}, 0, 1);  // [3, 2, 4] strides (4, 12, 1)
    CHECK(L::array_layout({3, 2, 4}, p3) == L::kCPrefer);
    CHECK((L::collect({3, 2, 4}, {p3, p3}) == L::c_strides({3, 2, 4})));
    CHECK((L::collect({3, 2, 4}, {L::f_strides({3, 2, 4}), p3}) == L::f_strides({3, 2, 4})));
    // mean_axis over the minimum-stride axis collects the remaining view: (4, 12) -> row-major
    CHECK((L::mean_axis_result({4, 3, 2}, f3, 0) == S{2, 1}));
    CHECK((L::mean_axis_result({2, 3}, t, 1) == S{1}));
    // reshape: the same shape keeps F; [2, 3] F -> [6] needs a copy (row-major); C [2, 3] ->
    // [3, 2] is a view; F [4, 6] -> [4, 2, 3] splits the outer axis as a view (1, 12, 4)
    CHECK((L::reshaped({2, 3}, t, {2, 3}) == S{1, 2}));
    CHECK((L::reshaped({2, 3}, t, {6}) == S{1}));
    CHECK((L::reshaped({2, 3}, {3, 1}, {3, 2}) == S{2, 1}));
    CHECK((L::reshaped({4, 6}, {1, 4}, {4, 2, 3}) == S{1, 12, 4}));
    CHECK(L::is_contiguous({4, 2, 3}, {1, 12, 4}));
    // to_owned of a sliced view keeps its strides only when it is contiguous in memory order
    CHECK((L::owned({4, 2}, {1, 4}) == S{1, 4}));     // full columns of an F [4, n] array
    CHECK((L::owned({3, 2}, {1, 4}) == S{2, 1}));     // partial columns: a row-major copy
}

TEST_CPU(validate_operation_rejects_handles_the_launch_would_overrun) {
    // RocmBackend::execute_op checks every input against what its launch touches before anything
    // runs; the addresses below are never dereferenced
    auto h = [](size_t bytes, std::vector<size_t> shape, DataType dt = DataType::F32) {
        MemoryHandle m;
        m.address = 0x10000;
        m.size = bytes;
        m.shape = std::move(shape);
        m.dtype = dt;
        return m;
    };
    std::string msg;
    Operation add(OperationType::Add);
    add.inputs = {h(24, {2, 3}), h(20, {2, 3})};  // second holds 5 floats, shape says 6
    CHECK(throws_kind([&] { validate_operation(add); }, ErrorKind::InvalidInput, &msg));
    CHECK(msg.find("input 1 holds 20 bytes") != std::string::npos);
    add.inputs[1] = h(24, {2, 3});
    validate_operation(add);  // well-formed: no throw
    add.inputs[1].address = 0;
    CHECK(throws_kind([&] { validate_operation(add); }, ErrorKind::InvalidInput));
    Operation mm(OperationType::MatMul);
    mm.inputs = {h(2 * 3 * 2, {2, 3}, DataType::BF16), h(3 * 4 * 4, {3, 4})};  // bf16 read as f32
    CHECK(throws_kind([&] { validate_operation(mm); }, ErrorKind::DTypeMismatch));
    mm.inputs[0] = h(2 * 3 * 4, {2, 3});
    mm.inputs[1] = h(3 * 4 * 4 - 4, {3, 4});
    CHECK(throws_kind([&] { validate_operation(mm); }, ErrorKind::InvalidInput));
    Operation tr(OperationType::Transpose);
    tr.inputs = {h(16, {3, 2})};
    CHECK(throws_kind([&] { validate_operation(tr); }, ErrorKind::InvalidInput));
    // SSMForward: u, delta, A, B, C[, D, z, dt_bias]
    const size_t bt = 2, L = 5, dim = 8, N = 16;
    auto ssm = [&](DataType st) {
        const size_t es = st == DataType::BF16 ? 2 : 4;
        Operation op(OperationType::SSMForward);
        op.inputs = {h(bt * L * dim * es, {}, st), h(bt * L * dim * es, {}, st), h(dim * N * 4, {}),
                     h(bt * L * N * es, {}, st), h(bt * L * N * es, {}, st), h(dim * 4, {}),
                     h(bt * L * dim * es, {}, st), h(dim * 4, {})};
        op.params = {{"batch", (double)bt}, {"seqlen", (double)L}, {"dim", (double)dim}, {"dstate", (double)N}};
        return op;
    };
    validate_operation(ssm(DataType::F32));
    validate_operation(ssm(DataType::BF16));
    auto bad = ssm(DataType::F32);
    bad.inputs[3].dtype = DataType::BF16;  // B not in u's storage type
    CHECK(throws_kind([&] { validate_operation(bad); }, ErrorKind::DTypeMismatch, &msg));
    CHECK(msg.find("SSMForward B") != std::string::npos);
    bad = ssm(DataType::BF16);
    bad.inputs[2].dtype = DataType::BF16;  // A must be F32
    CHECK(throws_kind([&] { validate_operation(bad); }, ErrorKind::DTypeMismatch));
    bad = ssm(DataType::F32);
    bad.inputs[6].size -= 4;  // z one element short
    CHECK(throws_kind([&] { validate_operation(bad); }, ErrorKind::InvalidInput, &msg));
    CHECK(msg.find("SSMForward: z holds") != std::string::npos);
    bad = ssm(DataType::F32);
    bad.params["seqlen"] = 6;  // more steps than the buffers hold
    CHECK(throws_kind([&] { validate_operation(bad); }, ErrorKind::InvalidInput));
    bad = ssm(DataType::F32);
    bad.params["dim"] = -1;
    CHECK(throws_kind([&] { validate_operation(bad); }, ErrorKind::InvalidInput));
    bad = ssm(DataType::F32);
    bad.inputs[0].dtype = DataType::F16;
    CHECK(throws_kind([&] { validate_operation(bad); }, ErrorKind::DTypeMismatch));
    bad = ssm(DataType::F32);
    bad.inputs[6].address = 0;  // an absent optional operand (z) is allowed
    validate_operation(bad);
    // StateUpdate: state, u, delta, A, B, C[, D, z, dt_bias]
    Operation su(OperationType::StateUpdate);
    su.inputs = {h(bt * dim * N * 4 - 4, {}), h(bt * dim * 4, {}), h(bt * dim * 4, {}), h(dim * N * 4, {}),
                 h(bt * N * 4, {}), h(bt * N * 4, {})};
    su.params = {{"batch", (double)bt}, {"dim", (double)dim}};
    CHECK(throws_kind([&] { validate_operation(su); }, ErrorKind::InvalidInput, &msg));
    CHECK(msg.find("state holds") != std::string::npos);
    su.inputs[0].size += 4;
    validate_operation(su);
    su.inputs[5].dtype = DataType::BF16;
    CHECK(throws_kind([&] { validate_operation(su); }, ErrorKind::DTypeMismatch));
}

// ============================================================================ device tests
TEST_GPU(reference_kat_matmul_ones) {
    // backend-cpu/src/lib.rs:1747-1758: ones[2,3] . ones[3,4] == 3
    auto a = HipTensor::ones(Shape({2, 3}));
    auto b = HipTensor::ones(Shape({3, 4}));
    auto y = a.matmul(b);
    CHECK((y.shape() == Shape({2, 4})));
    for (float v : y.to_host()) CHECK(std::fabs(v - 3.0f) < 1e-6f);
    std::string msg;
    CHECK(throws_kind([&] { (void)a.matmul(HipTensor::ones(Shape({4, 2}))); }, ErrorKind::ShapeMismatch, &msg));
    CHECK(msg.find("expected [3], got [4]") != std::string::npos);
}

TEST_GPU(matmul_bit_exact_vs_cpu_tensor_order) {
    const size_t M = 37, K = 129, N = 70;
    auto av = randn(M * K, 1), bv = randn(K * N, 2);
    auto y = HipTensor::from_host(av, Shape({M, K})).matmul(HipTensor::from_host(bv, Shape({K, N})));
    std::vector<float> r(M * N);
    oracle_matmul(M, K, N, av.data(), bv.data(), r.data());
    CHECK(bits_equal(y.to_host(), r));
}

TEST_GPU(linear_and_exported_mamba_block_vs_oracle) {
    Rng rng(7);
    MambaBlock blk(64, 16, 4, 2, rng);  // README example shape (config 1)
    auto xv = randn(100 * 64, 3);
    for (auto& v : xv) v = std::fmod(v, 1.0f);
    auto x = HipTensor::from_host(xv, Shape({100, 64}));
    auto y = blk.forward(x).to_host();
    std::vector<float> tmp(100 * 128), r(100 * 64);
    auto wg = blk.gate().weight().to_host(), bg = blk.gate().bias().to_host();
    auto wo = blk.out_proj().weight().to_host(), bo = blk.out_proj().bias().to_host();
    oracle_mamba_mlp(100, 64, 128, xv.data(), wg.data(), bg.data(), wo.data(), bo.data(), tmp.data(), r.data());
    CHECK(rel_err(y, r) < 1e-4);  // the fp32 bar (device SiLU vs libm expf differ by ulps)
    std::vector<float> r2(100 * 128);
    oracle_linear(100, 64, 128, xv.data(), wg.data(), bg.data(), 0, r2.data());
    CHECK(bits_equal(blk.gate().forward(x).to_host(), r2));
}

TEST_GPU(rmsnorm_vs_oracle) {
    RMSNorm norm(512, 1e-5f);
    auto xv = randn(33 * 512, 4, 2.0f);
    auto y = norm.forward(HipTensor::from_host(xv, Shape({33, 512}))).to_host();
    std::vector<float> w(512, 1.0f), r(33 * 512);
    oracle_rmsnorm(33, 512, xv.data(), w.data(), 1e-5f, r.data());
    CHECK(rel_err(y, r) < 1e-5);
}

TEST_GPU(s4block_forward_ssm_bit_exact_and_shape_rules) {
    Rng rng(11);
    S4Block s4(64, 16, rng);  // ssm::S4Block::new(64, 16) distributions
    const size_t L = 100;
    auto xv = randn(64 * L, 5);
    auto y = s4.forward_ssm(HipTensor::from_host(xv, Shape({64, L})));
    CHECK((y.shape() == Shape({64, L})));  // the reference's shape field; memory is [L, 64]
    std::vector<float> r(L * 64), work(3 * 16 + 64);
    auto ar = s4.A_real.to_host(), ai = s4.A_imag.to_host(), B = s4.B.to_host(), C = s4.C.to_host(),
         D = s4.D.to_host();
    oracle_s4_ref_fwd(64, 16, L, 0.1f, xv.data(), ar.data(), ai.data(), B.data(), C.data(), D.data(),
                      nullptr, r.data(), work.data());
    CHECK(bits_equal(y.to_host(), r));
    // ssm.rs:142-147: dim 0 must be d_model
    std::string msg;
    CHECK(throws_kind([&] { (void)s4.forward_ssm(HipTensor::zeros(Shape({100, 64}))); },
                      ErrorKind::ShapeMismatch, &msg));
    CHECK(msg.find("expected [64], got [100]") != std::string::npos);
    // the time-parallel form agrees to rounding on a decaying system
    S4Block s4b(64, 16, rng);
    std::vector<float> are(16, -0.5f), aim(16);
    for (int n = 0; n < 16; ++n) aim[n] = (float)(M_PI * n);
    s4b.A_real = HipTensor::from_host(are, Shape({16}));
    s4b.A_imag = HipTensor::from_host(aim, Shape({16}));
    auto xp = HipTensor::from_host(xv, Shape({64, L}));
    // D = 0 in this init, so outputs cross zero: compared normwise
    auto yp = s4b.forward_ssm(xp, nullptr, true).to_host(), ye = s4b.forward_ssm(xp).to_host();
    double num = 0, den = 0;
    for (size_t i = 0; i < yp.size(); ++i) {
        num = std::fmax(num, std::fabs((double)yp[i] - ye[i]));
        den = std::fmax(den, std::fabs((double)ye[i]));
    }
    CHECK(num <= 1e-5 * den);
}

TEST_GPU(s4block_checkpoint_restore_through_file) {
    Rng rng(13);
    S4Block a(32, 8, rng), b(32, 8, rng);
    auto x = HipTensor::from_host(randn(32 * 50, 6), Shape({32, 50}));
    const std::string path = "/tmp/helix_s4_ckpt.bin";
    save_checkpoint(path, "{\"epoch\":0}", a.checkpoint());
    auto [meta, params] = load_checkpoint(path);
    CHECK(meta == "{\"epoch\":0}" && params.size() == 7);
    b.restore(params);
    CHECK(bits_equal(a.forward_ssm(x).to_host(), b.forward_ssm(x).to_host()));
    params.pop_back();  // ssm.rs:345-350
    std::string msg;
    CHECK(throws_kind([&] { b.restore(params); }, ErrorKind::InvalidCheckpoint, &msg));
    CHECK(msg.find("expected 7 parameters, got 6") != std::string::npos);
}

TEST_GPU(ssm_mamba_block_forward_bit_exact) {
    Rng rng(17);
    SsmMambaBlock m(32, 16, rng);
    auto xv = randn(32 * 32, 8);
    auto y = m.forward_mamba(HipTensor::from_host(xv, Shape({32, 32}))).to_host();
    std::vector<float> r(32 * 32), work(32 * 32 + 3 * 16 + 32);
    auto dp = m.delta_proj.to_host(), ar = m.s4.A_real.to_host(), ai = m.s4.A_imag.to_host(),
         B = m.s4.B.to_host(), C = m.s4.C.to_host(), D = m.s4.D.to_host(), g = m.gate.to_host();
    oracle_ssm_mamba_fwd(32, 16, 0.1f, xv.data(), dp.data(), ar.data(), ai.data(), B.data(), C.data(),
                         D.data(), g.data(), r.data(), work.data());
    CHECK(bits_equal(y, r));
}

TEST_GPU(selective_scan_and_backend_ssm_forward) {
    const size_t bt = 2, L = 300, dim = 128, N = 16;
    auto u = randn(bt * L * dim, 20), dl = randn(bt * L * dim, 21), Bv = randn(bt * L * N, 22),
         Cv = randn(bt * L * N, 23), Dv = randn(dim, 24), zv = randn(bt * L * dim, 25);
    for (auto& v : dl) v = v * 0.5f - 4.0f;
    std::vector<float> Av(dim * N);
    for (size_t d = 0; d < dim; ++d)
        for (size_t n = 0; n < N; ++n) Av[d * N + n] = -(float)(n + 1);
    auto tu = HipTensor::from_host(u, Shape({bt, L, dim})), td = HipTensor::from_host(dl, Shape({bt, L, dim}));
    auto tA = HipTensor::from_host(Av, Shape({dim, N})), tB = HipTensor::from_host(Bv, Shape({bt, L, N}));
    auto tC = HipTensor::from_host(Cv, Shape({bt, L, N})), tD = HipTensor::from_host(Dv, Shape({dim}));
    auto tz = HipTensor::from_host(zv, Shape({bt, L, dim}));
    auto y = selective_scan(tu, td, tA, tB, tC, &tD, &tz, nullptr, true);
    std::vector<float> r(bt * L * dim);
    oracle_selective_scan(bt, L, dim, N, 1, u.data(), dl.data(), Av.data(), Bv.data(), Cv.data(), Dv.data(),
                          zv.data(), nullptr, r.data(), nullptr, nullptr);
    auto yh = y.to_host();
    CHECK(rel_err(yh, r) < 1e-4);

    // hal::ComputeBackend for ROCm: SSMForward through execute_op is the same kernel
    RocmBackend be(0);
    CHECK(be.device_type() == DeviceType::ROCm && be.is_available());
    CHECK(be.supports_operation(OperationType::SSMForward) && be.supports_operation(OperationType::MatMul));
    CHECK(!be.supports_operation(OperationType::SSMBackward));
    CHECK(be.compute_units() > 0 && be.memory_bandwidth() > 0 && be.optimal_batch_size() >= 1);
    auto handle = [&](const HipTensor& t, std::vector<size_t> shape) {
        MemoryHandle h;
        h.address = (uintptr_t)t.data();
        h.size = t.nbytes();
        h.shape = std::move(shape);
        return h;
    };
    Operation op(OperationType::SSMForward);
    op.inputs = {handle(tu, {bt, L, dim}), handle(td, {bt, L, dim}), handle(tA, {dim, N}),
                 handle(tB, {bt, L, N}), handle(tC, {bt, L, N}), handle(tD, {dim}), handle(tz, {bt, L, dim})};
    op.params = {{"batch", (double)bt}, {"seqlen", (double)L}, {"dim", (double)dim}, {"dstate", (double)N},
                 {"softplus", 1.0}};
    MemoryHandle out = be.execute_op(op);
    std::vector<float> yb(bt * L * dim);
    be.copy_to_host(yb.data(), out, yb.size() * 4);
    CHECK(bits_equal(yb, yh));
    be.deallocate(out);
    CHECK(throws_kind([&] { be.deallocate(out); }, ErrorKind::InvalidInput));
    Operation bad(OperationType::SSMForward);
    bad.inputs = op.inputs;
    CHECK(throws_kind([&] { (void)be.execute_op(bad); }, ErrorKind::InvalidInput));  // no params
    CHECK(throws_kind([&] { (void)be.execute_op(Operation(OperationType::SSMBackward)); },
                      ErrorKind::UnsupportedOperation));
    // MatMul through the backend equals HipTensor::matmul
    auto a = HipTensor::from_host(randn(12 * 20, 30), Shape({12, 20}));
    auto b = HipTensor::from_host(randn(20 * 9, 31), Shape({20, 9}));
    Operation mm(OperationType::MatMul);
    mm.inputs = {handle(a, {12, 20}), handle(b, {20, 9})};
    MemoryHandle mo = be.execute_op(mm);
    std::vector<float> mh(12 * 9);
    be.copy_to_host(mh.data(), mo, mh.size() * 4);
    CHECK(bits_equal(mh, a.matmul(b).to_host()));
}

TEST_GPU(long_sequence_scan_on_every_surface) {
    // 1 x 16384 x 512: 8 (batch, 64-channel) tiles cannot fill the GPU, so the library cuts the
    // sequence into time segments with a carry (a workspace is needed). helix::selective_scan and
    // the HAL's SSMForward take that path and give the C ABI's hx_selective_scan_fwd_ws result
    // bit for bit (the call the Python layer makes), within 1e-4 of the sequential oracle.
    const size_t bt = 1, L = 16384, dim = 512, N = 16;
    const size_t need = hx_selective_scan_workspace_size(bt, L, dim, N, HX_F32);
    CHECK(need > 0);
    auto u = randn(bt * L * dim, 60), dl = randn(bt * L * dim, 61), Bv = randn(bt * L * N, 62),
         Cv = randn(bt * L * N, 63), Dv = randn(dim, 64), zv = randn(bt * L * dim, 65);
    for (auto& v : dl) v = v * 0.5f - 4.0f;
    std::vector<float> Av(dim * N);
    for (size_t d = 0; d < dim; ++d)
        for (size_t n = 0; n < N; ++n) Av[d * N + n] = -(float)(n + 1);
    auto tu = HipTensor::from_host(u, Shape({bt, L, dim})), td = HipTensor::from_host(dl, Shape({bt, L, dim}));
    auto tA = HipTensor::from_host(Av, Shape({dim, N})), tB = HipTensor::from_host(Bv, Shape({bt, L, N}));
    auto tC = HipTensor::from_host(Cv, Shape({bt, L, N})), tD = HipTensor::from_host(Dv, Shape({dim}));
    auto tz = HipTensor::from_host(zv, Shape({bt, L, dim}));
    // the C ABI's segmented path
    HipTensor ws(Shape({(need + 3) / 4}), Storage::F32, 0), yc(Shape({bt, L, dim}), Storage::F32, 0);
    CHECK(hx_selective_scan_fwd_ws(bt, L, dim, N, HX_F32, 1, tu.data(), td.data(), (const float*)tA.data(),
                                   tB.data(), tC.data(), (const float*)tD.data(), tz.data(), nullptr, yc.data(),
                                   nullptr, nullptr, ws.data(), ws.nbytes(), nullptr) == HX_OK);
    const auto ych = yc.to_host();
    // the C++ host layer
    const auto yh = selective_scan(tu, td, tA, tB, tC, &tD, &tz, nullptr, true).to_host();
    CHECK(bits_equal(yh, ych));
    // the HAL
    RocmBackend be(0);
    auto handle = [&](const HipTensor& t) {
        MemoryHandle m;
        m.address = (uintptr_t)t.data();
        m.size = t.nbytes();
        return m;
    };
    Operation op(OperationType::SSMForward);
    op.inputs = {handle(tu), handle(td), handle(tA), handle(tB), handle(tC), handle(tD), handle(tz)};
    op.params = {{"batch", (double)bt}, {"seqlen", (double)L}, {"dim", (double)dim}, {"dstate", (double)N}};
    MemoryHandle out = be.execute_op(op);
    std::vector<float> yb(bt * L * dim);
    be.copy_to_host(yb.data(), out, yb.size() * 4);
    be.deallocate(out);
    CHECK(bits_equal(yb, ych));
    // and a second, shorter call reuses the backend's workspace
    Operation op2 = op;
    op2.params["seqlen"] = 8192.0;
    MemoryHandle out2 = be.execute_op(op2);
    std::vector<float> yb2(bt * 8192 * dim);
    be.copy_to_host(yb2.data(), out2, yb2.size() * 4);
    be.deallocate(out2);
    std::vector<float> r(bt * L * dim);
    oracle_selective_scan(bt, L, dim, N, 1, u.data(), dl.data(), Av.data(), Bv.data(), Cv.data(), Dv.data(),
                          zv.data(), nullptr, r.data(), nullptr, nullptr);
    const double e = rel_err(yh, r);
    std::printf("  1x16384x512 segmented scan: max rel err %.3e vs oracle\n", e);
    CHECK(e < 1e-4);
    // the first 8192 steps of a sequence do not depend on what follows
    std::vector<float> r2(r.begin(), r.begin() + bt * 8192 * dim);
    CHECK(rel_err(yb2, r2) < 1e-4);
}

TEST_GPU(fused_mamba_block_runs_and_regrows_workspace) {
    Rng rng(19);
    MambaBlockFused blk(64, 16, 4, 2, rng);
    auto x1 = HipTensor::from_host(randn(2 * 40 * 64, 40), Shape({2, 40, 64}), Storage::BF16);
    auto x2 = HipTensor::from_host(randn(1 * 300 * 64, 41), Shape({1, 300, 64}), Storage::BF16);
    auto y1 = blk.forward(x1).to_host();
    auto y2 = blk.forward(x2).to_host();
    auto y1b = blk.forward(x1).to_host();
    CHECK(y1.size() == 2 * 40 * 64 && y2.size() == 300 * 64);
    CHECK(bits_equal(y1, y1b));  // deterministic, workspace reuse is safe
    for (float v : y2) CHECK(std::isfinite(v));
    CHECK(throws_kind([&] { (void)blk.forward(x1.to_storage(Storage::F32)); }, ErrorKind::DTypeMismatch));
}

// ---------------------------------------------------------------------------- tensor primitives
TEST_GPU(hiptensor_elementwise_ops_vs_cpu_tensor) {
    const size_t n = 1031;
    auto av = randn(n, 50), bv = randn(n, 51);
    auto a = HipTensor::from_host(av, Shape({n})), b = HipTensor::from_host(bv, Shape({n}));
    std::vector<float> r(n);
    for (size_t i = 0; i < n; ++i) r[i] = av[i] + bv[i];
    CHECK(bits_equal(a.add(b).to_host(), r));
    for (size_t i = 0; i < n; ++i) r[i] = av[i] - bv[i];
    CHECK(bits_equal(a.sub(b).to_host(), r));
    for (size_t i = 0; i < n; ++i) r[i] = av[i] * bv[i];
    CHECK(bits_equal(a.mul(b).to_host(), r));
    for (size_t i = 0; i < n; ++i) r[i] = av[i] / bv[i];
    CHECK(bits_equal(a.div(b).to_host(), r));
    for (size_t i = 0; i < n; ++i) r[i] = av[i] * 0.1f;
    CHECK(bits_equal(a.mul_scalar(0.1f).to_host(), r));
    for (size_t i = 0; i < n; ++i) r[i] = std::sqrt(std::fabs(av[i]));
    CHECK(bits_equal(a.abs().sqrt().to_host(), r));
    const int ops[] = {0, 1, 2, 4, 10};  // exp, cos, sin, silu, sigmoid: device libm, <= 1e-6
    for (int op : ops) {
        oracle_unary(op, (int64_t)n, av.data(), 0.0f, r.data());
        HipTensor g = op == 0 ? a.exp() : op == 1 ? a.cos() : op == 2 ? a.sin() : op == 4 ? a.silu() : a.sigmoid();
        CHECK(rel_err(g.to_host(), r) <= 1e-6);
    }
    std::string msg;
    CHECK(throws_kind([&] { (void)a.add(HipTensor::ones(Shape({n, 1}))); }, ErrorKind::ShapeMismatch, &msg));
    CHECK(msg == "Shape mismatch: expected [1031], got [1031, 1]");
    CHECK(std::fabs(HipTensor::from_scalar(2.5f, Shape({1})).to_scalar() - 2.5f) == 0.0f);
    CHECK(throws_kind([&] { (void)a.to_scalar(); }, ErrorKind::InvalidInput));
    CHECK(bits_equal(HipTensor::eye(3).to_host(), {1, 0, 0, 0, 1, 0, 0, 0, 1}));
}

TEST_GPU(hiptensor_shape_ops_and_mean) {
    auto xv = randn(6 * 10, 60);
    auto x = HipTensor::from_host(xv, Shape({6, 10}));
    // transpose (lib.rs:115-137)
    auto t = x.transpose(0, 1);
    CHECK((t.shape() == Shape({10, 6})));
    auto th = t.to_host();
    bool ok = true;
    for (size_t i = 0; i < 6; ++i)
        for (size_t j = 0; j < 10; ++j) ok = ok && th[j * 6 + i] == xv[i * 10 + j];
    CHECK(ok);
    CHECK(throws_kind([&] { (void)x.transpose(0, 2); }, ErrorKind::InvalidDimension));
    // slice (lib.rs:139-183)
    auto sl = x.slice({1, 2}, {4, 5}).to_host();
    CHECK(sl.size() == 9 && sl[0] == xv[12] && sl[8] == xv[3 * 10 + 4]);
    CHECK(throws_kind([&] { (void)x.slice({0}, {1}); }, ErrorKind::ShapeMismatch));
    CHECK(throws_kind([&] { (void)x.slice({0, 5}, {1, 5}); }, ErrorKind::InvalidDimension));
    CHECK(throws_kind([&] { (void)HipTensor::ones(Shape({2, 2, 2})).slice({0, 0, 0}, {1, 1, 1}); },
                      ErrorKind::UnsupportedOperation));
    // stack(., 1) of 1-D steps: data back to back, shape field [d, L] (lib.rs:277-296)
    std::vector<HipTensor> steps;
    for (int k = 0; k < 4; ++k) steps.push_back(HipTensor::from_scalar((float)k, Shape({3})));
    auto st = HipTensor::stack(steps, 1);
    CHECK((st.shape() == Shape({3, 4})));
    CHECK(bits_equal(st.to_host(), {0, 0, 0, 1, 1, 1, 2, 2, 2, 3, 3, 3}));
    CHECK(throws_kind([&] { (void)HipTensor::stack({}, 0); }, ErrorKind::UnsupportedOperation));
    CHECK(throws_kind([&] { (void)HipTensor::stack({steps[0], x}, 0); }, ErrorKind::ShapeMismatch));
    // a 4-D stack is a true stack (generic_stack, lib.rs:390-467)
    auto q0 = HipTensor::from_host(randn(16, 61), Shape({2, 2, 2, 2}));
    auto q1 = HipTensor::from_host(randn(16, 62), Shape({2, 2, 2, 2}));
    auto qs = HipTensor::stack({q0, q1}, 1);
    CHECK((qs.shape() == Shape({2, 2, 2, 2, 2})));
    auto qh = qs.to_host(), q0h = q0.to_host(), q1h = q1.to_host();
    CHECK(qh[0] == q0h[0] && qh[8] == q1h[0] && qh[16] == q0h[8] && qh[31] == q1h[15]);
    // cat of 1-D (lib.rs:185-252)
    auto c = HipTensor::cat({steps[0], steps[3]}, 0);
    CHECK(bits_equal(c.to_host(), {0, 0, 0, 3, 3, 3}));
    CHECK(throws_kind([&] { (void)HipTensor::cat({x, x}, 0); }, ErrorKind::UnsupportedOperation));
    // broadcast_to repeat rows (lib.rs:1388-1404) and the [R, 1] -> [R, C] generic case
    auto w = HipTensor::from_host({1, 2, 3}, Shape({3}));
    CHECK(bits_equal(w.broadcast_to(Shape({2, 3})).to_host(), {1, 2, 3, 1, 2, 3}));
    CHECK(bits_equal(w.reshape(Shape({3, 1})).broadcast_to(Shape({3, 2})).to_host(), {1, 1, 2, 2, 3, 3}));
    CHECK(throws_kind([&] { (void)w.broadcast_to(Shape({2, 4})); }, ErrorKind::ShapeMismatch));
    // mean over the last axis and over axis 0: ndarray's orders, bit for bit
    std::vector<float> r0(6), r1(10);
    const std::vector<size_t> last = {1}, first = {0};
    oracle_mean_axis(6, 10, 1, 1, xv.data(), r0.data());
    oracle_mean_axis(1, 6, 10, 0, xv.data(), r1.data());
    CHECK(bits_equal(x.mean(&last).to_host(), r0));
    CHECK(bits_equal(x.mean(&first).to_host(), r1));
    const std::vector<size_t> bad = {2};
    CHECK(throws_kind([&] { (void)x.mean(&bad); }, ErrorKind::InvalidDimension));
}

// A transposed tensor keeps the reference array's permuted strides: mean sums its axes in the
// order ndarray uses for that layout, cat/stack/broadcast_to fail where the reference's
// as_slice().unwrap() panics, and the operations that keep or drop the order do so.
TEST_GPU(transposed_tensor_follows_the_reference_layout) {
    const size_t R = 13, C = 11;  // both >= 9: the lane fold and the in-order sum differ
    auto xv = randn(R * C, 81);
    auto x = HipTensor::from_host(xv, Shape({R, C}));
    std::vector<float> rows_fold(R), rows_seq(R), cols_fold(C), cols_seq(C);
    oracle_mean_axis(R, C, 1, 1, xv.data(), rows_fold.data());  // each row of x, lane fold
    oracle_mean_axis(R, C, 1, 0, xv.data(), rows_seq.data());   // each row of x, in order
    oracle_mean_axis(1, R, C, 0, xv.data(), cols_seq.data());   // each column of x, in order
    {
        std::vector<float> xt(R * C);  // each column of x by the lane fold (x^T row-major)
        for (size_t r = 0; r < R; ++r)
            for (size_t c = 0; c < C; ++c) xt[c * R + r] = xv[r * C + c];
        oracle_mean_axis(C, R, 1, 1, xt.data(), cols_fold.data());
    }
    CHECK(!bits_equal(rows_fold, rows_seq) && !bits_equal(cols_fold, cols_seq));
    auto xT = x.transpose(0, 1);  // [C, R], strides (1, C) in the reference
    CHECK(x.is_contiguous() && !xT.is_contiguous());
    const std::vector<size_t> last = {1}, first = {0};
    // over xT's last axis (x's columns): not the minimum-stride axis -> in order
    CHECK(bits_equal(xT.mean(&last).to_host(), cols_seq));
    // over xT's axis 0 (x's rows): the minimum-stride axis with contiguous lanes -> lane fold
    CHECK(bits_equal(xT.mean(&first).to_host(), rows_fold));
    // both axes, last first: in-order column means, then a 1-D lane fold
    std::vector<float> all(1);
    oracle_mean_axis(1, C, 1, 1, cols_seq.data(), all.data());
    CHECK(bits_equal(xT.mean().to_host(), all));
    // elementwise maps keep the order, F + F stays F, F + C collects row-major
    CHECK(!xT.exp().is_contiguous() && !xT.mul(xT).is_contiguous());
    auto mixed = xT.add(HipTensor::ones(Shape({C, R})));
    CHECK(mixed.is_contiguous());
    std::vector<float> mv = mixed.to_host(), mixed_rows(C);
    oracle_mean_axis(C, R, 1, 1, mv.data(), mixed_rows.data());
    CHECK(bits_equal(mixed.mean(&last).to_host(), mixed_rows));
    // contiguous() is to_owned(): it keeps the order; a reshape that needs a copy drops it
    CHECK(!xT.contiguous().is_contiguous());
    CHECK(!xT.reshape(Shape({C, R})).is_contiguous() && xT.reshape(Shape({C * R})).is_contiguous());
    // a slice of whole columns stays F; one of part of them is a row-major copy
    CHECK(!xT.slice({0, 0}, {C, 2}).is_contiguous() && xT.slice({0, 0}, {3, 2}).is_contiguous());
    // as_slice().unwrap() panics in the reference: stack, broadcast_to
    CHECK(throws_kind([&] { (void)HipTensor::stack({xT, xT}, 0); }, ErrorKind::UnsupportedOperation));
    CHECK(throws_kind([&] { (void)xT.broadcast_to(Shape({2, C, R})); }, ErrorKind::UnsupportedOperation));
    CHECK((xT.broadcast_to(Shape({C, R})).shape() == Shape({C, R})));  // same shape: a clone
    // a transpose of a length-1 axis stays standard
    CHECK(HipTensor::ones(Shape({1, 5})).transpose(0, 1).is_contiguous());
}

TEST_GPU(matmul_vector_forms_and_rank_errors) {
    const size_t M = 9, K = 33, N = 7;
    auto mv = randn(M * K, 70), vv = randn(K, 71), wv = randn(K * N, 72);
    auto m = HipTensor::from_host(mv, Shape({M, K})), v = HipTensor::from_host(vv, Shape({K}));
    auto w = HipTensor::from_host(wv, Shape({K, N}));
    std::vector<float> r(M);
    oracle_matmul(M, K, 1, mv.data(), vv.data(), r.data());  // 2-D x 1-D (lib.rs:715-746)
    auto mvp = m.matmul(v);
    CHECK((mvp.shape() == Shape({M})) && bits_equal(mvp.to_host(), r));
    std::vector<float> r2(N);
    oracle_matmul(1, K, N, vv.data(), wv.data(), r2.data());  // 1-D x 2-D (lib.rs:681-712)
    auto vw = v.matmul(w);
    CHECK((vw.shape() == Shape({N})) && bits_equal(vw.to_host(), r2));
    std::string msg;
    CHECK(throws_kind([&] { (void)v.matmul(v); }, ErrorKind::UnsupportedOperation, &msg));
    CHECK(msg.find("batch matrix multiplication for >2D tensors not implemented yet") != std::string::npos);
    CHECK(throws_kind([&] { (void)m.matmul(HipTensor::ones(Shape({K + 1}))); }, ErrorKind::ShapeMismatch));
}

TEST_GPU(generic_nn_bodies_over_primitives_vs_oracle) {
    // Linear::forward (lib.rs:120-134) as x.matmul(W^T) + broadcast(bias): bit-exact
    Rng rng(80);
    Linear g(64, 128, rng), o(128, 64, rng);
    auto bias_g = HipTensor::from_host(randn(128, 81), Shape({128}));
    auto xv = randn(100 * 64, 82);
    auto x = HipTensor::from_host(xv, Shape({100, 64}));
    const auto wg = g.weight().to_host(), bg = bias_g.to_host();
    std::vector<float> r(100 * 128);
    oracle_linear(100, 64, 128, xv.data(), wg.data(), bg.data(), 0, r.data());
    CHECK(bits_equal(generic::linear(x, g.weight(), &bias_g).to_host(), r));
    // the exported MambaBlock body (lib.rs:888-906): linear -> silu -> linear
    const auto wo = o.weight().to_host(), bo = o.bias().to_host(), b0 = g.bias().to_host();
    std::vector<float> tmp(100 * 128), r2(100 * 64);
    oracle_mamba_mlp(100, 64, 128, xv.data(), wg.data(), b0.data(), wo.data(), bo.data(), tmp.data(), r2.data());
    const double e_mlp = rel_err(generic::mamba_mlp(x, g, o).to_host(), r2);
    std::printf("  generic mamba_mlp vs oracle: max rel err %.3e\n", e_mlp);
    CHECK(e_mlp <= 1e-4);
    // RMSNorm::forward (lib.rs:258-285) over primitives: bit-exact with the oracle's
    // primitive-order restatement
    auto wv = randn(64, 83);
    std::vector<float> r3(100 * 64), work(64);
    oracle_rmsnorm_ref(100, 64, xv.data(), wv.data(), 1e-5f, r3.data(), work.data());
    CHECK(bits_equal(generic::rmsnorm(x, HipTensor::from_host(wv, Shape({64})), 1e-5f).to_host(), r3));
    // 3-D input [2, 50, 64] takes the (3,3) generic broadcast and the (1,3) weight broadcast
    CHECK(bits_equal(generic::rmsnorm(x.reshape(Shape({2, 50, 64})), HipTensor::from_host(wv, Shape({64})),
                                      1e-5f).to_host(), r3));
}

TEST_GPU(generic_s4_forward_ssm_over_primitives) {
    // ssm::S4Block::forward_ssm (ssm.rs:138-186) step by step over HipTensor ops. With
    // A_real = A_imag = 0 the device exp/cos give exactly 1 (as libm does), so the result is the
    // oracle's bit for bit; with the reference's init (A_imag ~ N(0,1)) within 2e-4.
    Rng rng(90);
    S4Block s4(16, 8, rng);
    auto xv = randn(16 * 40, 91);
    auto x = HipTensor::from_host(xv, Shape({16, 40}));
    auto run_oracle = [&](const S4Block& b) {
        const auto ar = b.A_real.to_host(), ai = b.A_imag.to_host(), Bv = b.B.to_host(),
                   Cv = b.C.to_host(), Dv = b.D.to_host();
        std::vector<float> y(16 * 40), work(3 * 8 + 16);
        oracle_s4_ref_fwd(16, 8, 40, 0.1f, xv.data(), ar.data(), ai.data(), Bv.data(), Cv.data(), Dv.data(),
                          nullptr, y.data(), work.data());
        return y;
    };
    auto y = generic::s4_forward_ssm(s4, x);
    CHECK((y.shape() == Shape({16, 40})));
    const double e_s4 = rel_err(y.to_host(), run_oracle(s4));
    std::printf("  generic S4 forward_ssm vs oracle (reference init): max rel err %.3e\n", e_s4);
    // measured 1.04e-4: device and host cosf differ by an ulp in a = cos(0.1 A_imag), which the
    // |a| ~ 1 recurrence carries into every later step
    CHECK(e_s4 <= 2e-4);
    s4.A_imag = HipTensor::zeros(Shape({8}));
    s4.D = HipTensor::from_host(randn(16, 92), Shape({16}));
    CHECK(bits_equal(generic::s4_forward_ssm(s4, x).to_host(), run_oracle(s4)));
    CHECK(bits_equal(generic::s4_forward_ssm(s4, x).to_host(), s4.forward_ssm(x).to_host()));
    CHECK(throws_kind([&] { (void)generic::s4_forward_ssm(s4, HipTensor::ones(Shape({8, 4}))); },
                      ErrorKind::ShapeMismatch));
}

TEST_GPU(exported_s4block_forward_is_identity) {
    // nn::S4Block::forward_ssm (crates/nn/src/lib.rs:742-756): Ok(input.clone())
    Rng rng(100);
    ExportedS4Block blk(64, 16, rng);
    CHECK((blk.A.shape() == Shape({16, 16})) && (blk.B.shape() == Shape({16, 64})) &&
          (blk.C.shape() == Shape({64, 16})) && (blk.Lambda.shape() == Shape({16})));
    CHECK(blk.parameters().size() == 6);
    auto xv = randn(100 * 64, 101);
    auto x = HipTensor::from_host(xv, Shape({100, 64}));
    auto y = blk.forward(x);
    CHECK(y.data() != x.data() && (y.shape() == x.shape()) && bits_equal(y.to_host(), xv));
    CHECK(throws_kind([&] { (void)blk.forward(HipTensor::ones(Shape({64}))); }, ErrorKind::InvalidDimension));
}

TEST_GPU(ssm_s4block_forward_conv_reproduces_reference_errors) {
    // ssm::S4Block::forward = forward_conv (ssm.rs:189-273): no input shape completes in the
    // reference; each case below fails where and how the reference fails
    auto expect = [&](size_t dm, size_t ds, std::vector<size_t> shape, ErrorKind k, const char* text) {
        Rng rng(110);
        S4Block b(dm, ds, rng);
        size_t n = 1;
        for (size_t d : shape) n *= d;
        auto x = HipTensor::from_host(randn(n, 111), Shape(shape));
        std::string msg;
        const bool got = throws_kind([&] { (void)b.forward(x); }, k, &msg);
        if (!got || msg.find(text) == std::string::npos)
            std::printf("  forward_conv d_model %zu d_state %zu: got \"%s\"\n", dm, ds, msg.c_str());
        return got && msg.find(text) != std::string::npos;
    };
    // L = 1: the [1, 1] input slice does not reshape to [d_model] (ssm.rs:210-211)
    CHECK(expect(4, 4, {2, 1}, ErrorKind::ShapeMismatch, "expected [1], got [4]"));
    // d_model = 1: the 2-D kernel sliced with one index (ssm.rs:213)
    CHECK(expect(1, 1, {2, 1}, ErrorKind::ShapeMismatch, "expected [2], got [1]"));
    // L = 2, d_model != d_state: C.(A^1) [d_model] . B [d_state, d_model] (ssm.rs:246)
    CHECK(expect(4, 2, {1, 2}, ErrorKind::ShapeMismatch, "expected [4], got [2]"));
    // L = 2, d_model == d_state: stack of K_0 [d, d] with K_1 [d] (ssm.rs:250)
    CHECK(expect(3, 3, {1, 2}, ErrorKind::ShapeMismatch, "expected [3, 3], got [3]"));
    // L = 3: A_power [d_state] . A_real [d_state] is 1-D x 1-D (ssm.rs:244)
    CHECK(expect(3, 3, {1, 3}, ErrorKind::UnsupportedOperation, "batch matrix multiplication"));
    // batch 0: stack of no outputs (ssm.rs:228)
    CHECK(expect(2, 2, {0, 1}, ErrorKind::UnsupportedOperation, "stacking of empty tensor list"));
    // 3-D input: two-index slice of a 3-D tensor (ssm.rs:210)
    CHECK(expect(4, 4, {2, 1, 4}, ErrorKind::ShapeMismatch, "expected [3], got [2]"));
    // rank 1: the reference's unwrap of dim(1) panics
    CHECK(expect(4, 4, {4}, ErrorKind::InvalidDimension, "out of bounds"));
}

TEST_GPU(rocm_backend_graph_async_copy_and_elementwise_ops) {
    RocmBackend be(0);
    CHECK(be.supports_operation(OperationType::Add) && be.supports_operation(OperationType::Mean) &&
          be.supports_operation(OperationType::Transpose) && !be.supports_operation(OperationType::FFT));
    const size_t n = 300;
    auto av = randn(n, 120), bv = randn(n, 121), cv = randn(n, 122);
    auto up = [&](const std::vector<float>& v, uint64_t id) {
        MemoryHandle h = be.allocate(v.size() * 4, DataType::F32);
        be.copy_from_host(h, v.data(), v.size() * 4);
        h.id = id;  // graph wiring uses ids; the backend keeps its own record
        return h;
    };
    MemoryHandle a = up(av, 1001), b = up(bv, 1002), c = up(cv, 1003);
    // graph: t0 = a + b -> t1 = exp(t0) -> t2 = t1 * c; t3 = sqrt(|c|) is a second output
    MemoryHandle t0;
    t0.id = 2000;
    MemoryHandle t1;
    t1.id = 2001;
    ComputeGraph g;
    Operation add(OperationType::Add);
    add.inputs = {a, b};
    add.output = &t0;
    Operation ex(OperationType::Exp);
    ex.inputs = {t0};
    ex.output = &t1;
    Operation mul(OperationType::Mul);
    mul.inputs = {t1, c};
    const size_t n0 = g.add_operation(add), n1 = g.add_operation(ex), n2 = g.add_operation(mul);
    g.add_dependency(n0, n1);
    g.add_dependency(n1, n2);
    g.build();
    // t0 and t1 carry ids only (no memory): execute_op allocates, the graph wires by id
    std::vector<MemoryHandle> outs = be.execute_graph(g);
    CHECK(outs.size() == 1);
    std::vector<float> got(n), sum(n), e(n), r(n);
    be.copy_to_host(got.data(), outs[0], n * 4);
    for (size_t i = 0; i < n; ++i) sum[i] = av[i] + bv[i];
    oracle_unary(0, (int64_t)n, sum.data(), 0.0f, e.data());
    for (size_t i = 0; i < n; ++i) r[i] = e[i] * cv[i];
    CHECK(rel_err(got, r) <= 1e-6);
    // execute_async / wait
    Operation sq(OperationType::Abs);
    sq.inputs = {c};
    AsyncHandle h = be.execute_async(sq);
    CHECK(h.device_id == be.device_id() && h.operation == OperationType::Abs);
    MemoryHandle ab = be.wait(h);
    std::vector<float> abh(n);
    be.copy_to_host(abh.data(), ab, n * 4);
    for (size_t i = 0; i < n; ++i) r[i] = std::fabs(cv[i]);
    CHECK(bits_equal(abh, r));
    CHECK(throws_kind([&] { (void)be.wait(h); }, ErrorKind::InvalidInput));
    // Mean (all elements) and Transpose
    Operation mean(OperationType::Mean);
    mean.inputs = {c};
    MemoryHandle mh = be.execute_op(mean);
    float mval = 0;
    be.copy_to_host(&mval, mh, 4);
    float rm = 0;
    oracle_mean_axis(1, (int64_t)n, 1, 1, cv.data(), &rm);
    CHECK(mval == rm);
    MemoryHandle cm = c;
    cm.shape = {15, 20};
    Operation tr(OperationType::Transpose);
    tr.inputs = {cm};
    MemoryHandle th = be.execute_op(tr);
    std::vector<float> tv(n);
    be.copy_to_host(tv.data(), th, n * 4);
    CHECK((th.shape == std::vector<size_t>{20, 15}) && tv[1] == cv[20] && tv[15] == cv[1]);
    // copy_to another backend instance on the device
    RocmBackend other(0);
    MemoryHandle cc = be.copy_to(c, other);
    std::vector<float> ch(n);
    other.copy_to_host(ch.data(), cc, n * 4);
    CHECK(bits_equal(ch, cv));
    const double u = be.utilization();
    CHECK(u >= 0.0 && u <= 1.0);
    const TopologicalFeatures tf = be.compute_topological_features(c);
    CHECK(tf.stability == 0.5 && tf.entropy == 0.0 && tf.motif_hashes.empty() && tf.cycles.empty());
    CHECK(throws_kind([&] { (void)be.execute_op(Operation(OperationType::FFT)); }, ErrorKind::UnsupportedOperation));
}

int main(int argc, char** argv) {
    bool want_gpu = false, want_cpu = false;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        if (a == "--gpu") want_gpu = true;
        else if (a == "--cpu") want_cpu = true;
        else g_ckpt_path = a;
    }
    if (!want_cpu && !want_gpu) want_cpu = want_gpu = true;
    for (auto& c : cases()) {
        if ((c.gpu && !want_gpu) || (!c.gpu && !want_cpu)) continue;
        g_cur = c.name;
        ++g_run;
        const int before = g_fail;
        std::printf("RUN  %s\n", c.name);
        std::fflush(stdout);
        try {
            c.fn();
        } catch (const std::exception& e) {
            std::printf("  FAIL %s: exception %s\n", c.name, e.what());
            ++g_fail;
        }
        std::printf("%s %s\n", g_fail == before ? "OK  " : "FAIL", c.name);
        std::fflush(stdout);
    }
    std::printf("%d run, %d failed\n", g_run, g_fail);
    return g_fail ? 1 : 0;
}
