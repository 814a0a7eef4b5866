// helix_hal.cpp — hal::ComputeBackend (crates/hal/src/backend.rs:13-70) and hal::ComputeGraph
// (crates/hal/src/operations.rs:88-231) for one ROCm device over the C ABI. Host code only.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <initializer_list>
#include <functional>

#include "helix/helix.hpp"
#include "helix_detail.h"
#include "helix_hip.h"

namespace helix {

using detail::invalid_input;
using detail::shape_mismatch;
using detail::unsupported;

const char* operation_name(OperationType op) {
    static const char* const names[] = {
        "Add", "Sub", "Mul", "Div", "Pow", "Sqrt", "Abs",
        "Sin", "Cos", "Tan", "Asin", "Acos", "Atan",
        "Exp", "Log", "Log2", "Log10",
        "MatMul", "Transpose", "Inverse", "Determinant", "Eigenvalues", "SVD",
        "Conv1D", "Conv2D", "Conv3D", "MaxPool", "AvgPool",
        "FFT", "IFFT", "RFFT", "IRFFT",
        "Sum", "Mean", "Max", "Min", "Var", "Std",
        "ReLU", "Sigmoid", "Tanh", "SiLU", "GELU", "Softmax",
        "SSMForward", "SSMBackward", "StateUpdate",
        "TopologicalAnalysis", "MotifDetection", "CycleDetection", "StabilityCalculation",
        "QuantumGate", "QuantumMeasurement", "QuantumEntanglement",
        "SpikeEncoding", "SpikeDecoding", "SignalFiltering",
    };
    const size_t i = (size_t)op;
    return i < sizeof(names) / sizeof(names[0]) ? names[i] : "?";
}

// ----------------------------------------------------------------------------- ComputeGraph
size_t ComputeGraph::add_operation(Operation op) {
    nodes_.push_back(std::move(op));
    return nodes_.size() - 1;
}

void ComputeGraph::add_dependency(size_t from, size_t to) {
    if (from >= nodes_.size() || to >= nodes_.size()) invalid_input("Invalid node ID");  // operations.rs:125-131
    deps_[from].push_back(to);
}

const std::vector<size_t>* ComputeGraph::dependencies(size_t node) const {
    auto it = deps_.find(node);
    return it == deps_.end() ? nullptr : &it->second;
}

void ComputeGraph::build() {
    // operations.rs:161-181: inputs have no incoming edge, outputs no outgoing edge
    inputs_.clear();
    outputs_.clear();
    for (size_t i = 0; i < nodes_.size(); ++i) {
        bool incoming = false;
        for (const auto& kv : deps_)
            if (std::find(kv.second.begin(), kv.second.end(), i) != kv.second.end()) incoming = true;
        if (!incoming) inputs_.push_back(i);
        if (!deps_.count(i)) outputs_.push_back(i);
    }
}

std::vector<size_t> ComputeGraph::topological_sort() const {
    // operations.rs:184-231: DFS from each unvisited node in index order, post-order, reversed;
    // a node met again while on the DFS path is a cycle
    std::vector<char> visited(nodes_.size(), 0), on_path(nodes_.size(), 0);
    std::vector<size_t> post;
    std::function<void(size_t)> dfs = [&](size_t n) {
        if (on_path[n]) invalid_input("Circular dependency detected");
        if (visited[n]) return;
        on_path[n] = 1;
        if (const auto* d = dependencies(n))
            for (size_t m : *d) dfs(m);
        on_path[n] = 0;
        visited[n] = 1;
        post.push_back(n);
    };
    for (size_t i = 0; i < nodes_.size(); ++i)
        if (!visited[i]) dfs(i);
    std::reverse(post.begin(), post.end());
    return post;
}

// ----------------------------------------------------------------------------- RocmBackend
RocmBackend::RocmBackend(int device) : device_(device) {
    check(hx_init(device), "hx_init");
    caps_.device_type = DeviceType::ROCm;
    caps_.device_id = device_id();
    caps_.supported_operations = {
        OperationType::Add,     OperationType::Sub,        OperationType::Mul,  OperationType::Div,
        OperationType::Sqrt,    OperationType::Abs,        OperationType::Sin,  OperationType::Cos,
        OperationType::Exp,     OperationType::Log,        OperationType::MatMul,
        OperationType::Transpose, OperationType::Mean,     OperationType::Sigmoid,
        OperationType::SiLU,    OperationType::SSMForward, OperationType::StateUpdate};
    caps_.supported_precisions = {DataType::F32, DataType::BF16};
    int cus = 0;
    size_t mem = 0;
    check(hx_device_info(device, &cus, &mem), "hx_device_info");
    caps_.compute_units = (size_t)cus;
    caps_.memory_bytes = mem;
    caps_.available_memory = mem;
    caps_.memory_bandwidth_gbs = 8000.0;  // MI355X HBM3E, published
}

RocmBackend::~RocmBackend() {
    (void)hx_sync();
    for (auto& kv : live_) (void)hx_free(kv.second);
    if (scan_ws_) (void)hx_free(scan_ws_);
}

std::string RocmBackend::device_id() const { return "rocm:" + std::to_string(device_); }

bool RocmBackend::supports_operation(OperationType op) const {
    return std::find(caps_.supported_operations.begin(), caps_.supported_operations.end(), op) !=
           caps_.supported_operations.end();
}

size_t RocmBackend::optimal_batch_size() const {
    // the scan runs one block per (batch row, 64 channels): at d_inner 1536 (24 tiles per row)
    // compute_units / 32 rows (8 on 256 CUs) give every CU a tile
    return caps_.compute_units >= 32 ? caps_.compute_units / 32 : 1;
}

MemoryHandle RocmBackend::allocate(size_t size, DataType dtype) {
    void* p = nullptr;
    check(hx_malloc(&p, size ? size : 4), "hx_malloc");
    MemoryHandle h;
    h.id = next_id_++;
    h.size = size;
    h.dtype = dtype;
    h.address = (uintptr_t)p;
    live_[h.id] = p;
    caps_.available_memory -= std::min(caps_.available_memory, size);
    return h;
}

void RocmBackend::deallocate(const MemoryHandle& h) {
    auto it = live_.find(h.id);
    if (it == live_.end()) invalid_input("unknown memory handle");
    check(hx_sync(), "hx_sync");  // work queued on the buffer finishes first
    check(hx_free(it->second), "hx_free");
    live_.erase(it);
    caps_.available_memory = std::min(caps_.memory_bytes, caps_.available_memory + h.size);
}

void RocmBackend::copy_from_host(const MemoryHandle& dst, const void* src, size_t bytes) {
    if (bytes > dst.size) invalid_input("copy past handle");
    check(hx_memcpy_h2d((void*)dst.address, src, bytes), "hx_memcpy_h2d");
}

void RocmBackend::copy_to_host(void* dst, const MemoryHandle& src, size_t bytes) const {
    if (bytes > src.size) invalid_input("copy past handle");
    check(hx_sync(), "hx_sync");
    check(hx_memcpy_d2h(dst, (const void*)src.address, bytes), "hx_memcpy_d2h");
}

MemoryHandle RocmBackend::copy_to(const MemoryHandle& src, ComputeBackend& dst) {
    // backend.rs:45: a new buffer of the same size and type on `dst` holding src's bytes
    MemoryHandle out = dst.allocate(src.size, src.dtype);
    out.shape = src.shape;
    if (src.size == 0) return out;
    if (dst.device_type() == DeviceType::ROCm) {
        check(hx_memcpy_d2d((void*)out.address, (const void*)src.address, src.size, nullptr),
              "hx_memcpy_d2d");  // device to device (peer copies go through the same call)
    } else {
        std::vector<unsigned char> host(src.size);
        copy_to_host(host.data(), src, src.size);
        dst.copy_from_host(out, host.data(), src.size);
    }
    return out;
}

namespace {
size_t elem_bytes(DataType t) {
    switch (t) {
        case DataType::I8: case DataType::U8: case DataType::BF8: case DataType::Bool: return 1;
        case DataType::I16: case DataType::U16: case DataType::F16: case DataType::BF16: return 2;
        case DataType::I64: case DataType::U64: case DataType::F64: case DataType::C32: return 8;
        case DataType::C64: return 16;
        default: return 4;
    }
}
size_t elements(const MemoryHandle& h) {
    if (!h.shape.empty()) {
        size_t n = 1;
        for (size_t d : h.shape) {
            if (d != 0 && n > SIZE_MAX / d) invalid_input("handle shape overflows size_t");
            n *= d;
        }
        return n;
    }
    return h.size / elem_bytes(h.dtype);
}
size_t mul_checked(std::initializer_list<size_t> f) {
    size_t n = 1;
    for (size_t v : f) {
        if (v != 0 && n > SIZE_MAX / v) invalid_input("operation sizes overflow size_t");
        n *= v;
    }
    return n;
}
void need_f32(const MemoryHandle& h, const char* op) {
    if (h.dtype != DataType::F32)
        throw TensorError(ErrorKind::DTypeMismatch,
                          std::string("DType mismatch: expected \"F32\", got another type for ") + op);
}
void need_dtype(const MemoryHandle& h, DataType want, const char* op, const char* what) {
    if (h.dtype != want)
        throw TensorError(ErrorKind::DTypeMismatch, std::string("DType mismatch: expected \"") +
                                                        (want == DataType::BF16 ? "BF16" : "F32") +
                                                        "\", got another type for " + op + " " + what);
}
// A handle the operation reads or writes `bytes` of: it must have a device address and hold them.
void need_bytes(const MemoryHandle& h, size_t bytes, const char* op, const char* what) {
    if (h.address == 0) invalid_input(std::string(op) + ": " + what + " has no device address");
    if (h.size < bytes)
        invalid_input(std::string(op) + ": " + what + " holds " + std::to_string(h.size) +
                      " bytes, the operation touches " + std::to_string(bytes));
}
// Whether optional input i is given (present with a device address).
bool given(const Operation& op, size_t i) { return i < op.inputs.size() && op.inputs[i].address != 0; }
int64_t size_param(const Operation& op, const char* k, double dflt, bool required) {
    auto it = op.params.find(k);
    double v = dflt;
    if (it == op.params.end()) {
        if (required) invalid_input(std::string("missing parameter ") + k);
    } else {
        v = it->second;
    }
    if (!(v >= 0.0) || v != std::floor(v) || v > 9.0e15)
        invalid_input(std::string("parameter ") + k + " must be a non-negative integer");
    return (int64_t)v;
}
void need_inputs(const Operation& op, size_t n) {
    if (op.inputs.size() < n)
        invalid_input(std::string(operation_name(op.op_type)) + " requires " + std::to_string(n) +
                      " input" + (n > 1 ? "s" : ""));
}
}  // namespace

void validate_operation(const Operation& op) {
    const OperationType t = op.op_type;
    const char* name = operation_name(t);
    switch (t) {
        case OperationType::Add: case OperationType::Sub: case OperationType::Mul:
        case OperationType::Div: {
            need_inputs(op, 2);
            need_f32(op.inputs[0], "binary op");
            need_f32(op.inputs[1], "binary op");
            const size_t n = elements(op.inputs[0]);
            if (elements(op.inputs[1]) != n) shape_mismatch({n}, {elements(op.inputs[1])});
            need_bytes(op.inputs[0], n * 4, name, "input 0");
            need_bytes(op.inputs[1], n * 4, name, "input 1");
            return;
        }
        case OperationType::Sqrt: case OperationType::Abs: case OperationType::Sin:
        case OperationType::Cos: case OperationType::Exp: case OperationType::Log:
        case OperationType::Sigmoid: case OperationType::SiLU:
            need_inputs(op, 1);
            need_f32(op.inputs[0], "unary op");
            need_bytes(op.inputs[0], elements(op.inputs[0]) * 4, name, "input 0");
            return;
        case OperationType::Mean: {
            need_inputs(op, 1);
            need_f32(op.inputs[0], "Mean");
            const size_t n = elements(op.inputs[0]);
            if (n == 0) invalid_input("Mean of an empty buffer");
            need_bytes(op.inputs[0], n * 4, name, "input 0");
            return;
        }
        case OperationType::Transpose: {
            need_inputs(op, 1);
            need_f32(op.inputs[0], "Transpose");
            const auto& sh = op.inputs[0].shape;
            if (sh.size() != 2) unsupported("Transpose needs a 2-D input shape");
            need_bytes(op.inputs[0], mul_checked({sh[0], sh[1], 4}), name, "input 0");
            return;
        }
        case OperationType::MatMul: {
            need_inputs(op, 2);
            need_f32(op.inputs[0], "MatMul");
            need_f32(op.inputs[1], "MatMul");
            const auto& a = op.inputs[0].shape;
            const auto& b = op.inputs[1].shape;
            if (a.size() != 2 || b.size() != 2) unsupported("MatMul needs 2-D input shapes");
            if (a[1] != b[0]) shape_mismatch({a[1]}, {b[0]});
            need_bytes(op.inputs[0], mul_checked({a[0], a[1], 4}), name, "input 0");
            need_bytes(op.inputs[1], mul_checked({b[0], b[1], 4}), name, "input 1");
            return;
        }
        case OperationType::SSMForward: {
            // inputs u, delta, A, B, C[, D, z, dt_bias]; u, delta, B, C, z in u's storage type
            if (op.inputs.size() < 5) invalid_input("SSMForward takes u, delta, A, B, C[, D, z, dt_bias]");
            const size_t bt = (size_t)size_param(op, "batch", 0, true), L = (size_t)size_param(op, "seqlen", 0, true);
            const size_t dim = (size_t)size_param(op, "dim", 0, true), N = (size_t)size_param(op, "dstate", 16, false);
            (void)size_param(op, "softplus", 1, false);
            const DataType st = op.inputs[0].dtype;
            if (st != DataType::F32 && st != DataType::BF16)
                throw TensorError(ErrorKind::DTypeMismatch,
                                  "DType mismatch: expected \"F32\" or \"BF16\", got another type for SSMForward u");
            const size_t es = st == DataType::BF16 ? 2 : 4;
            const size_t seq = mul_checked({bt, L, dim, es}), bc = mul_checked({bt, L, N, es});
            need_bytes(op.inputs[0], seq, name, "u");
            need_dtype(op.inputs[1], st, name, "delta");
            need_bytes(op.inputs[1], seq, name, "delta");
            need_dtype(op.inputs[2], DataType::F32, name, "A");
            need_bytes(op.inputs[2], mul_checked({dim, N, 4}), name, "A");
            need_dtype(op.inputs[3], st, name, "B");
            need_bytes(op.inputs[3], bc, name, "B");
            need_dtype(op.inputs[4], st, name, "C");
            need_bytes(op.inputs[4], bc, name, "C");
            if (given(op, 5)) { need_dtype(op.inputs[5], DataType::F32, name, "D"); need_bytes(op.inputs[5], dim * 4, name, "D"); }
            if (given(op, 6)) { need_dtype(op.inputs[6], st, name, "z"); need_bytes(op.inputs[6], seq, name, "z"); }
            if (given(op, 7)) { need_dtype(op.inputs[7], DataType::F32, name, "dt_bias"); need_bytes(op.inputs[7], dim * 4, name, "dt_bias"); }
            return;
        }
        case OperationType::StateUpdate: {
            // inputs state, u, delta, A, B, C[, D, z, dt_bias]; u, delta, B, C, z in u's storage type
            if (op.inputs.size() < 6) invalid_input("StateUpdate takes state, u, delta, A, B, C[, D, z, dt_bias]");
            const size_t bt = (size_t)size_param(op, "batch", 0, true), dim = (size_t)size_param(op, "dim", 0, true);
            const size_t N = (size_t)size_param(op, "dstate", 16, false);
            (void)size_param(op, "softplus", 1, false);
            const DataType st = op.inputs[1].dtype;
            if (st != DataType::F32 && st != DataType::BF16)
                throw TensorError(ErrorKind::DTypeMismatch,
                                  "DType mismatch: expected \"F32\" or \"BF16\", got another type for StateUpdate u");
            const size_t es = st == DataType::BF16 ? 2 : 4;
            const size_t row = mul_checked({bt, dim, es}), bc = mul_checked({bt, N, es});
            need_dtype(op.inputs[0], DataType::F32, name, "state");
            need_bytes(op.inputs[0], mul_checked({bt, dim, N, 4}), name, "state");
            need_bytes(op.inputs[1], row, name, "u");
            need_dtype(op.inputs[2], st, name, "delta");
            need_bytes(op.inputs[2], row, name, "delta");
            need_dtype(op.inputs[3], DataType::F32, name, "A");
            need_bytes(op.inputs[3], mul_checked({dim, N, 4}), name, "A");
            need_dtype(op.inputs[4], st, name, "B");
            need_bytes(op.inputs[4], bc, name, "B");
            need_dtype(op.inputs[5], st, name, "C");
            need_bytes(op.inputs[5], bc, name, "C");
            if (given(op, 6)) { need_dtype(op.inputs[6], DataType::F32, name, "D"); need_bytes(op.inputs[6], dim * 4, name, "D"); }
            if (given(op, 7)) { need_dtype(op.inputs[7], st, name, "z"); need_bytes(op.inputs[7], row, name, "z"); }
            if (given(op, 8)) { need_dtype(op.inputs[8], DataType::F32, name, "dt_bias"); need_bytes(op.inputs[8], dim * 4, name, "dt_bias"); }
            return;
        }
        default:
            return;  // execute_op reports the operation as unsupported
    }
}

void* RocmBackend::scan_workspace(size_t bytes) {
    if (bytes == 0) return nullptr;
    if (bytes > scan_ws_bytes_) {
        if (scan_ws_) {
            check(hx_sync(), "hx_sync");  // work queued on the old buffer finishes first
            check(hx_free(scan_ws_), "hx_free");
            scan_ws_ = nullptr;
            scan_ws_bytes_ = 0;
        }
        check(hx_malloc(&scan_ws_, bytes), "hx_malloc");
        scan_ws_bytes_ = bytes;
    }
    return scan_ws_;
}

MemoryHandle RocmBackend::execute_op(const Operation& op) {
    // every input is checked against what the launch will touch before anything is launched
    validate_operation(op);
    auto param = [&](const char* k, double dflt) {
        auto it = op.params.find(k);
        return it == op.params.end() ? dflt : it->second;
    };
    auto ptr = [&](size_t i) -> void* {
        return i < op.inputs.size() && op.inputs[i].address ? (void*)op.inputs[i].address : nullptr;
    };
    auto out_for = [&](size_t bytes, DataType dt) {
        if (op.output && op.output->address) {  // an id-only handle declares an output (graphs)
            if (op.output->size < bytes) invalid_input("output handle too small");
            return *op.output;
        }
        return allocate(bytes, dt);
    };
    const OperationType t = op.op_type;
    switch (t) {
        case OperationType::Add: case OperationType::Sub: case OperationType::Mul:
        case OperationType::Div: {
            const size_t n = elements(op.inputs[0]);
            MemoryHandle o = out_for(n * 4, DataType::F32);
            o.shape = op.inputs[0].shape;
            const int code = t == OperationType::Add ? HX_ADD : t == OperationType::Sub ? HX_SUB
                             : t == OperationType::Mul ? HX_MUL : HX_DIV;
            check(hx_binary_f32(code, (int64_t)n, (const float*)ptr(0), (const float*)ptr(1),
                                (float*)o.address, nullptr),
                  "hx_binary_f32");
            return o;
        }
        case OperationType::Sqrt: case OperationType::Abs: case OperationType::Sin:
        case OperationType::Cos: case OperationType::Exp: case OperationType::Log:
        case OperationType::Sigmoid: case OperationType::SiLU: {
            const size_t n = elements(op.inputs[0]);
            MemoryHandle o = out_for(n * 4, DataType::F32);
            o.shape = op.inputs[0].shape;
            const int code = t == OperationType::Sqrt ? HX_SQRT : t == OperationType::Abs ? HX_ABS
                             : t == OperationType::Sin ? HX_SIN : t == OperationType::Cos ? HX_COS
                             : t == OperationType::Exp ? HX_EXP : t == OperationType::Log ? HX_LOG
                             : t == OperationType::Sigmoid ? HX_SIGMOID : HX_SILU;
            check(hx_unary_f32(code, (int64_t)n, (const float*)ptr(0), 0.0f, (float*)o.address, nullptr),
                  "hx_unary_f32");
            return o;
        }
        case OperationType::Mean: {
            // all elements -> one value (the reference backends' Mean, e.g.
            // backend-cpu/src/cpu_backend.rs:703-734)
            const size_t n = elements(op.inputs[0]);
            MemoryHandle o = out_for(4, DataType::F32);
            o.shape = {1};
            check(hx_mean_axis_f32(1, (int64_t)n, 1, 1, (const float*)ptr(0), (float*)o.address, nullptr),
                  "hx_mean_axis_f32");
            return o;
        }
        case OperationType::Transpose: {
            const auto& s = op.inputs[0].shape;
            MemoryHandle o = out_for(s[0] * s[1] * 4, DataType::F32);
            o.shape = {s[1], s[0]};
            const int64_t shp[2] = {(int64_t)s[1], (int64_t)s[0]};
            const int64_t src[2] = {1, (int64_t)s[1]}, dst[2] = {(int64_t)s[0], 1};
            check(hx_copy_strided_f32(2, shp, (const float*)ptr(0), src, (float*)o.address, dst, nullptr),
                  "hx_copy_strided_f32");
            return o;
        }
        case OperationType::MatMul: {
            const auto& a = op.inputs[0].shape;
            const auto& b = op.inputs[1].shape;
            MemoryHandle o = out_for(a[0] * b[1] * 4, DataType::F32);
            o.shape = {a[0], b[1]};
            check(hx_matmul_f32((int64_t)a[0], (int64_t)a[1], (int64_t)b[1], (const float*)ptr(0),
                                (const float*)ptr(1), (float*)o.address, nullptr),
                  "hx_matmul_f32");
            return o;
        }
        case OperationType::SSMForward: {
            // the library's long-sequence path (time segments with a carry) through a workspace
            // this backend keeps, as the fused scan of hal/src/device.rs:191 would run
            const int64_t bt = (int64_t)param("batch", 0), L = (int64_t)param("seqlen", 0);
            const int64_t dim = (int64_t)param("dim", 0), N = (int64_t)param("dstate", 16);
            const int sp = (int)param("softplus", 1);
            const bool bf = op.inputs[0].dtype == DataType::BF16;
            const int dt = bf ? HX_BF16 : HX_F32;
            MemoryHandle o = out_for((size_t)(bt * L * dim) * (bf ? 2 : 4), op.inputs[0].dtype);
            o.shape = {(size_t)bt, (size_t)L, (size_t)dim};
            const size_t need = hx_selective_scan_workspace_size(bt, L, dim, N, dt);
            void* ws = scan_workspace(need);
            check(hx_selective_scan_fwd_ws(bt, L, dim, N, dt, sp, ptr(0), ptr(1), (const float*)ptr(2), ptr(3),
                                           ptr(4), (const float*)ptr(5), ptr(6), (const float*)ptr(7),
                                           (void*)o.address, nullptr, nullptr, ws, need, nullptr),
                  "hx_selective_scan_fwd_ws");
            return o;
        }
        case OperationType::StateUpdate: {
            const int64_t bt = (int64_t)param("batch", 0), dim = (int64_t)param("dim", 0);
            const int64_t N = (int64_t)param("dstate", 16);
            const int sp = (int)param("softplus", 1);
            const bool bf = op.inputs[1].dtype == DataType::BF16;
            MemoryHandle o = out_for((size_t)(bt * dim) * (bf ? 2 : 4), op.inputs[1].dtype);
            o.shape = {(size_t)bt, (size_t)dim};
            check(hx_selective_state_update(bt, dim, N, bf ? HX_BF16 : HX_F32, sp, (float*)ptr(0), ptr(1),
                                            ptr(2), (const float*)ptr(3), ptr(4), ptr(5), (const float*)ptr(6),
                                            ptr(7), (const float*)ptr(8), (void*)o.address, nullptr),
                  "hx_selective_state_update");
            return o;
        }
        default:
            unsupported(std::string(operation_name(t)) + " on " + device_id());
    }
}

std::vector<MemoryHandle> RocmBackend::execute_graph(const ComputeGraph& graph) {
    // Nodes run in topological order; an input whose id is a node's declared output id reads
    // what that node produced (the substitution rule of the reference backends' execute_graph,
    // backend-cpu/src/cpu_backend.rs:1014-1066); the outputs of the graph's output nodes return
    // in node order. The graph must have been built (ComputeGraph::build).
    std::map<uint64_t, MemoryHandle> produced;
    std::map<size_t, MemoryHandle> result_of;
    for (size_t n : graph.topological_sort()) {
        Operation op = graph.nodes()[n];
        for (MemoryHandle& in : op.inputs) {
            auto it = produced.find(in.id);
            if (it != produced.end()) in = it->second;
        }
        MemoryHandle out = execute_op(op);
        if (graph.nodes()[n].output) produced[graph.nodes()[n].output->id] = out;
        result_of[n] = out;
    }
    std::vector<MemoryHandle> outs;
    for (size_t n : graph.output_nodes()) outs.push_back(result_of.at(n));
    return outs;
}

TopologicalFeatures RocmBackend::compute_topological_features(const MemoryHandle& /*data*/) {
    // The reference defines no algorithm for this: both of its backends return no motifs or
    // cycles, stability 0.5 and entropy 0.0 (backend-cpu/src/cpu_backend.rs:1069-1078,
    // backend-cuda/src/cuda_backend.rs:1213-1222); the same answer is returned here.
    TopologicalFeatures f;
    f.stability = 0.5;
    f.entropy = 0.0;
    return f;
}

AsyncHandle RocmBackend::execute_async(const Operation& op) {
    // every operation above is enqueued on the device stream without a host wait, so the launch
    // itself is the asynchronous part; the output is held until wait()
    MemoryHandle out = execute_op(op);
    AsyncHandle h;
    h.id = next_id_++;
    h.device_id = device_id();
    h.operation = op.op_type;
    pending_[h.id] = out;
    return h;
}

MemoryHandle RocmBackend::wait(const AsyncHandle& h) {
    auto it = pending_.find(h.id);
    if (it == pending_.end()) invalid_input("unknown async handle");
    check(hx_sync(), "hx_sync");
    MemoryHandle out = it->second;
    pending_.erase(it);
    return out;
}

bool RocmBackend::is_available() const { return hx_init(device_) == HX_OK; }

double RocmBackend::utilization() const {
    double frac = 0.0;
    return hx_device_utilization(device_, &frac) == HX_OK ? frac : 0.0;
}

void RocmBackend::synchronize() { check(hx_sync(), "hx_sync"); }

}  // namespace helix
