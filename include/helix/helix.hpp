// helix.hpp — native C++ host layer over libhelix_hip.so's C ABI, mirroring the reference's
// Rust interface for the SSM path so a C++ caller writes what a HelixML caller writes:
//
//   tensor_core:  Shape, DType, Device, TensorError (crates/tensor-core/src/{shape,dtype,device,
//                 error}.rs), the Tensor trait's constructors and to/from host copies
//                 (tensor.rs:7-59, TensorRandom 212-233) on a device tensor, HipTensor;
//   nn:           Linear (crates/nn/src/lib.rs:53-134), RMSNorm (lib.rs:219-285), the exported
//                 MambaBlock (Linear -> SiLU -> Linear, lib.rs:846-906), ssm::S4Block
//                 (ssm.rs:37-186, checkpoint/restore 331-360), ssm::MambaBlock (ssm.rs:435-483),
//                 and the full selective Mamba block (MambaBlockFused);
//   training:     the checkpoint file of CheckpointManager (training/src/checkpoint.rs:137-198):
//                 u32 big-endian metadata length, metadata JSON, then bincode 1.x of
//                 Vec<CpuTensor> — HipTensors are written in exactly the bytes a CpuTensor with
//                 the same values writes, and read back from them;
//   hal:          ComputeBackend for ROCm (crates/hal/src/backend.rs:13-70) with SSMForward,
//                 StateUpdate and MatMul operations (hal/src/device.rs:129-210).
//
// Errors are thrown as helix::TensorError carrying the reference's variant; nothing here
// computes on the host: every value comes from the HIP kernels behind include/helix_hip.h.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace helix {

// ----------------------------------------------------------------------------- tensor_core
// tensor_core::TensorError variants (crates/tensor-core/src/error.rs:7-37), declaration order.
enum class ErrorKind {
    ShapeMismatch,
    InvalidDimension,
    DeviceMismatch,
    DTypeMismatch,
    UnsupportedOperation,
    AllocationFailed,
    BackendError,
    SerializationError,
    InvalidCheckpoint,
    InvalidInput,
};

class TensorError : public std::runtime_error {
public:
    TensorError(ErrorKind k, const std::string& msg) : std::runtime_error(msg), kind_(k) {}
    ErrorKind kind() const { return kind_; }
    // The variant for a libhelix_hip status code (include/helix_hip.h hx_status).
    static TensorError from_status(int status, const std::string& what);

private:
    ErrorKind kind_;
};

// Throws the TensorError for a non-zero hx status, with the library's last error text.
void check(int status, const char* what);

// tensor_core::DType (dtype.rs:8-37), same variant order (it is the bincode tag).
enum class DType : uint32_t { I8, I16, I32, I64, U8, U16, U32, U64, F16, F32, F64, Bool, C32, C64 };

// tensor_core::Shape (shape.rs:8-97): row-major dims.
class Shape {
public:
    Shape() = default;
    explicit Shape(std::vector<size_t> dims) : dims_(std::move(dims)) {}
    const std::vector<size_t>& as_slice() const { return dims_; }
    size_t ndim() const { return dims_.size(); }
    size_t dim(size_t i) const;
    size_t numel() const;
    bool operator==(const Shape& o) const { return dims_ == o.dims_; }
    bool operator!=(const Shape& o) const { return dims_ != o.dims_; }

private:
    std::vector<size_t> dims_;
};

// tensor_core::Device (device.rs:8-25). The reference has no ROCm variant; a HipTensor lives on
// Custom("rocm:<id>").
struct Device {
    enum class Kind : uint32_t { Cpu, Cuda, Metal, Wgpu, Qpu, Npu, Tpu, Custom } kind = Kind::Cpu;
    uint64_t index = 0;
    std::string name;
    static Device cpu() { return Device{}; }
    static Device rocm(int id) { return Device{Kind::Custom, 0, "rocm:" + std::to_string(id)}; }
    bool operator==(const Device& o) const { return kind == o.kind && index == o.index && name == o.name; }
};

// Storage of a device tensor: fp32, or bf16 (the north-star block's storage; DType has no BF16,
// so such a tensor reports DType::F32 values when copied to the host or serialised).
enum class Storage { F32, BF16 };

// Seeded host generator for the reference's TensorRandom distributions (SplitMix64 with
// Box-Muller normals): the reference's own generator is unseeded thread_rng
// (backend-cpu/src/lib.rs:1209-1257), so only the distributions can match.
class Rng {
public:
    explicit Rng(uint64_t seed) : s_(seed) {}
    uint64_t next_u64();
    float uniform(float lo, float hi);
    float normal(float mean, float std);

private:
    uint64_t s_;
    bool have_spare_ = false;
    double spare_ = 0.0;
};

// A device tensor: the HipTensor a crates/backend-hip would define. Owns device memory
// (hx_malloc/hx_free), row-major contiguous.
class HipTensor {
public:
    HipTensor() = default;
    HipTensor(Shape shape, Storage st, int device = 0);  // uninitialised
    static HipTensor zeros(Shape shape, Storage st = Storage::F32, int device = 0);
    static HipTensor ones(Shape shape, Storage st = Storage::F32, int device = 0);
    static HipTensor from_host(const std::vector<float>& values, Shape shape,
                               Storage st = Storage::F32, int device = 0);
    static HipTensor random_normal(Shape shape, float mean, float std, Rng& rng,
                                   Storage st = Storage::F32, int device = 0);
    static HipTensor random_uniform(Shape shape, float lo, float hi, Rng& rng,
                                    Storage st = Storage::F32, int device = 0);

    const Shape& shape() const { return shape_; }
    Storage storage() const { return storage_; }
    DType dtype() const { return DType::F32; }
    Device device() const { return Device::rocm(device_); }
    size_t numel() const { return shape_.numel(); }
    size_t nbytes() const { return numel() * (storage_ == Storage::BF16 ? 2 : 4); }
    void* data() const { return buf_ ? buf_->ptr : nullptr; }
    bool defined() const { return buf_ != nullptr; }

    std::vector<float> to_host() const;  // values as f32 (bf16 widened exactly)
    HipTensor to_storage(Storage st) const;
    HipTensor reshape(Shape s) const;  // shares storage
    HipTensor clone() const;

    // Tensor ops on the path (TensorOps, tensor.rs:62-134)
    HipTensor matmul(const HipTensor& other) const;  // 2-D x 2-D, CpuTensor::matmul bit-exact

private:
    struct Buffer {
        void* ptr = nullptr;
        explicit Buffer(size_t bytes);
        ~Buffer();
        Buffer(const Buffer&) = delete;
        Buffer& operator=(const Buffer&) = delete;
    };
    std::shared_ptr<Buffer> buf_;
    Shape shape_;
    Storage storage_ = Storage::F32;
    int device_ = 0;
};

// ----------------------------------------------------------------------------- nn
// nn::Linear (lib.rs:53-134): weight [out, in] ~ N(0, sqrt(2/in)), bias zeros; y = x . W^T + b.
class Linear {
public:
    Linear(size_t in_features, size_t out_features, Rng& rng, int device = 0);
    Linear(HipTensor weight, HipTensor bias) : weight_(std::move(weight)), bias_(std::move(bias)) {}
    HipTensor forward(const HipTensor& x) const;             // fp32, [rows, in]
    HipTensor forward_silu(const HipTensor& x) const;        // silu(x . W^T + b), one launch
    const HipTensor& weight() const { return weight_; }
    const HipTensor& bias() const { return bias_; }

private:
    HipTensor weight_, bias_;
};

// nn::RMSNorm (lib.rs:219-285): weight ones; y = x / sqrt(mean(x^2) + eps) * w over the last dim.
class RMSNorm {
public:
    RMSNorm(size_t d_model, float eps, int device = 0);
    HipTensor forward(const HipTensor& x, Storage out = Storage::F32) const;
    HipTensor& weight() { return weight_; }
    float eps() const { return eps_; }

private:
    HipTensor weight_;
    float eps_;
};

// Exported nn::MambaBlock (lib.rs:846-906): forward = out_proj(silu(gate(x))).
class MambaBlock {
public:
    MambaBlock(size_t d_model, size_t d_state, size_t d_conv, size_t expand, Rng& rng, int device = 0);
    HipTensor forward(const HipTensor& x) const;  // x [seq_len, d_model] fp32
    const Linear& gate() const { return gate_; }
    const Linear& out_proj() const { return out_proj_; }

private:
    Linear gate_, out_proj_;
};

// nn::ssm::S4Block (ssm.rs:37-186): shared-state S4 recurrence, dt = 0.1.
class S4Block {
public:
    S4Block(size_t d_model, size_t d_state, Rng& rng, int device = 0);
    // forward_ssm (ssm.rs:138-186): x [d_model, L] -> y with the reference's memory [L, d_model]
    // and shape field [d_model, L]. parallel = the time-parallel form (equal to rounding).
    HipTensor forward_ssm(const HipTensor& x, const HipTensor* gate = nullptr,
                          bool parallel = false) const;
    // checkpoint()/restore() (ssm.rs:331-360): A_real, A_imag, B, C, D, delta, Lambda.
    std::vector<HipTensor> checkpoint() const;
    void restore(const std::vector<HipTensor>& ck);
    size_t d_model() const { return d_model_; }
    size_t d_state() const { return d_state_; }
    HipTensor A_real, A_imag, B, C, D, delta, Lambda;

private:
    size_t d_model_, d_state_;
    // discretize(dt)'s decay (hx_s4_discretize, host libm) for the A_real / A_imag buffers it was
    // computed from (parameters are immutable buffers, so their addresses identify them)
    mutable HipTensor a_disc_;
    mutable const void* a_src_[2] = {nullptr, nullptr};
    mutable HipTensor workspace_;
};

// nn::ssm::MambaBlock::forward_mamba (ssm.rs:435-464): delta = X . delta_proj; y =
// S4.forward_ssm(delta) gated by `gate`. X must be [d_model, d_model] as in the reference.
class SsmMambaBlock {
public:
    SsmMambaBlock(size_t d_model, size_t d_state, Rng& rng, int device = 0);
    HipTensor forward_mamba(const HipTensor& x) const;
    S4Block s4;
    HipTensor delta_proj, B_proj, C_proj, gate;
};

// The selective Mamba block the exported MambaBlock's parameters describe (bf16 storage, fp32
// arithmetic): in_proj -> conv1d+SiLU -> x_proj -> dt_proj -> selective scan -> out_proj.
class MambaBlockFused {
public:
    MambaBlockFused(size_t d_model, size_t d_state, size_t d_conv, size_t expand, Rng& rng,
                    int device = 0, size_t dt_rank = 0);
    HipTensor forward(const HipTensor& x) const;  // x [batch, L, d_model] bf16
    size_t d_model, d_state, d_conv, d_inner, dt_rank;
    HipTensor w_in, conv_w, conv_b, w_x, w_dt, dt_bias, A, D, w_out;

private:
    mutable HipTensor workspace_;
};

// Fused selective scan on HipTensors (hx_selective_scan_fwd).
HipTensor selective_scan(const HipTensor& u, const HipTensor& delta, const HipTensor& A,
                         const HipTensor& B, const HipTensor& C, const HipTensor* D,
                         const HipTensor* z, const HipTensor* dt_bias, bool softplus,
                         HipTensor* last_state = nullptr);

// ----------------------------------------------------------------------------- training
// CheckpointManager's file (training/src/checkpoint.rs:137-198): u32 big-endian metadata
// length, metadata JSON, bincode of Vec<CpuTensor>. The tensor bytes are those a CpuTensor with
// the same values writes (device Cpu, dtype F32), so files move between the two backends.
struct HostTensor {
    std::vector<size_t> shape;
    std::vector<float> values;
};
std::vector<uint8_t> encode_params(const std::vector<HostTensor>& params);
std::vector<HostTensor> decode_params(const std::vector<uint8_t>& bytes);
void save_checkpoint(const std::string& path, const std::string& metadata_json,
                     const std::vector<HostTensor>& params);
std::pair<std::string, std::vector<HostTensor>> load_checkpoint_host(const std::string& path);
// HipTensor forms (device <-> host copies around the above)
void save_checkpoint(const std::string& path, const std::string& metadata_json,
                     const std::vector<HipTensor>& params);
std::pair<std::string, std::vector<HipTensor>> load_checkpoint(const std::string& path,
                                                               int device = 0);

// ----------------------------------------------------------------------------- hal
// hal::DeviceType and DataType (hal/src/device.rs:8-100) in the reference's declaration order;
// OperationType (device.rs:129-210) holds the reference's names for the operations on this path.
enum class DeviceType { CPU, CUDA, Metal, ROCm, NPU, TPU, QPU, BCI };
enum class DataType { I8, I16, I32, I64, U8, U16, U32, U64, F16, F32, F64, BF8, BF16, C32, C64, Bool };
enum class OperationType { Add, MatMul, Conv1D, SiLU, SSMForward, SSMBackward, StateUpdate };

// hal::MemoryHandle (hal/src/memory.rs:11-24).
struct MemoryHandle {
    uint64_t id = 0;
    DeviceType device = DeviceType::ROCm;
    size_t size = 0;
    DataType dtype = DataType::F32;
    uintptr_t address = 0;
    std::vector<size_t> shape;  // logical shape of the buffer
};

// hal::Operation (hal/src/operations.rs:9-28): type, inputs, output, numeric parameters.
struct Operation {
    OperationType op_type;
    std::vector<MemoryHandle> inputs;
    MemoryHandle* output = nullptr;  // optional preallocated output
    std::map<std::string, double> params;
    explicit Operation(OperationType t) : op_type(t) {}
};

struct DeviceCapabilities {
    DeviceType device_type = DeviceType::ROCm;
    std::string device_id;
    std::vector<OperationType> supported_operations;
    std::vector<DataType> supported_precisions;
    size_t compute_units = 0;
    size_t memory_bytes = 0;
    double memory_bandwidth_gbs = 0.0;
};

// hal::ComputeBackend (hal/src/backend.rs:13-70) for one ROCm device.
class RocmBackend {
public:
    explicit RocmBackend(int device = 0);
    ~RocmBackend();
    DeviceType device_type() const { return DeviceType::ROCm; }
    std::string device_id() const;
    const DeviceCapabilities& capabilities() const { return caps_; }
    bool supports_operation(OperationType op) const;
    size_t optimal_batch_size() const;
    std::vector<DataType> supported_precisions() const { return caps_.supported_precisions; }
    double memory_bandwidth() const { return caps_.memory_bandwidth_gbs; }
    size_t compute_units() const { return caps_.compute_units; }
    MemoryHandle allocate(size_t size, DataType dtype);
    void deallocate(const MemoryHandle& h);
    void copy_from_host(const MemoryHandle& dst, const void* src, size_t bytes);
    void copy_to_host(void* dst, const MemoryHandle& src, size_t bytes) const;
    // SSMForward: inputs u, delta, A, B, C [, D, z, dt_bias as present] with params batch, seqlen,
    // dim, dstate, softplus; StateUpdate: state, u, delta, A, B, C [, D, z, dt_bias];
    // MatMul: a [M,K], b [K,N] (fp32). The output is allocated unless op.output is given.
    MemoryHandle execute_op(const Operation& op);
    bool is_available() const;
    double utilization() const { return 0.0; }
    void synchronize();

private:
    int device_;
    DeviceCapabilities caps_;
    uint64_t next_id_ = 1;
    std::map<uint64_t, void*> live_;
};

}  // namespace helix
