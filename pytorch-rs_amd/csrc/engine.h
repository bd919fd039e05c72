// engine.h -- C++ host engine: the Tensor / Storage / autograd layer of the
// torch_rs hot path, restated from the reference's src/tensor.rs for device
// tensors.  All arithmetic goes through libtrs_hip.so's C ABI (trs_hip.h);
// this layer owns metadata (shape, strides, offset), output-layout planning,
// and the reverse-mode graph.
//
// Device model: "cuda" tensors (ROCm PyTorch's spelling) live in HBM and run
// every op on the GPU.  "cpu" tensors are host staging only (creation, views,
// .to(), .numpy()); arithmetic on them raises, because the CPU path is the
// reference's own and this library has no CPU fallback.
#pragma once

#include <cstdint>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "trs_hip.h"

namespace trs_engine {

using Dims = std::vector<int64_t>;

// TensorError (src/tensor_error.rs:7-108) -> Python RuntimeError;
// indexing errors -> IndexError (src/python_tensor_errors.rs:8-49).
struct TensorError : std::runtime_error {
    explicit TensorError(const std::string &m) : std::runtime_error(m) {}
};
struct IndexError : std::runtime_error {
    explicit IndexError(const std::string &m) : std::runtime_error(m) {}
};

enum class DeviceType { CPU, CUDA };

struct Device {
    DeviceType type = DeviceType::CPU;
    int index = -1;
    bool is_cuda() const { return type == DeviceType::CUDA; }
    bool operator==(const Device &o) const { return type == o.type && (type == DeviceType::CPU || index == o.index); }
    std::string str() const;
    static Device parse(const std::string &s);
};

// Refcounted flat f32 buffer (Storage, src/storage.rs:7-18): a host vector
// for cpu tensors or an HBM allocation for cuda tensors.
struct Storage {
    Device device;
    int64_t numel = 0;
    std::vector<float> host;
    float *dptr = nullptr;
    // A leaf's accumulated gradient (StorageData::SharedGradient,
    // src/storage.rs:7-18): later backward passes add into it in place.
    bool shared_gradient = false;
    ~Storage();
    float *data() { return device.is_cuda() ? dptr : host.data(); }
    static std::shared_ptr<Storage> allocate(Device device, int64_t numel);
};
using StoragePtr = std::shared_ptr<Storage>;

// ---- layout planning (src/tensor.rs:3695-4458), restated ----
namespace layout {
Dims contiguous_strides(const Dims &shape);
bool is_contiguous(const Dims &shape, const Dims &strides, int64_t numel);
bool is_non_overlapping_and_dense(const Dims &shape, const Dims &strides, int64_t numel);
bool is_channels_last_contiguous(const Dims &shape, const Dims &strides);
Dims channels_last_strides(const Dims &shape);
Dims elementwise_output_strides(const Dims &shape, const std::vector<std::pair<Dims, Dims>> &ops);
Dims unary_output_strides(const Dims &shape, const Dims &strides, int64_t numel);
Dims scalar_output_strides(const Dims &shape, const Dims &strides);
void binary_output_layout(const Dims &ls, const Dims &lt, const Dims &rs, const Dims &rt, Dims &oshape, Dims &ostr);
bool reshape_view_strides(const Dims &old_shape, const Dims &old_strides, const Dims &new_shape, int64_t numel,
                          Dims &out);
Dims reshape_strides(const Dims &shape, int64_t numel);
int64_t numel_of(const Dims &shape);
std::string shape_str(const Dims &d);
}  // namespace layout

struct AutogradMeta;
using MetaPtr = std::shared_ptr<AutogradMeta>;

// Python-visible node names (src/autograd_node.rs:5-59) plus the nodes this
// backend adds for device tensors.
enum class Node {
    Add, Alias, Clone, Multiply, Negate, Permute, Relu, ReflectedSubtract, Subtract, Sum, MatrixTranspose,
    Transpose, View, Select, Exp, Mm, Bmm, AddTensor, SubTensor, Squeeze, SqueezeDimension, SqueezeDimensions,
    Unsqueeze, Fused
};
const char *node_name(Node n);

struct SavedTensor {
    StoragePtr values;  // kept only when a derivative needs the values
    Dims shape, strides;
    int64_t offset = 0, numel = 0;
    int64_t output_nr = 0;
    MetaPtr autograd;
    bool values_required = false;
};

enum class GradKind {
    Multiply, MultiplyScalar, Negate, Relu, Sum, Identity, Permute, Index, AddTensor, SubTensor, Matmul, Exp,
    MaskApply, Transfer, Fused
};

// The backward of a fused node: one compiled pointwise program whose
// arguments are saved forward inputs (index into GradFn::inputs) or the
// upstream gradient (-1), and whose output o, over the node's output shape,
// is the gradient of input targets[o].
struct FusedBackward {
    uint64_t program = 0;
    std::vector<int> args;
    std::vector<int> targets;
};

// One byte per element in HBM (a dropout keep-mask).
struct ByteBuffer {
    Device device;
    Dims shape;
    int64_t numel = 0;
    uint8_t *dptr = nullptr;
    ~ByteBuffer();
    static std::shared_ptr<ByteBuffer> from_host(const uint8_t *data, const Dims &shape, Device device);
};
using BytePtr = std::shared_ptr<ByteBuffer>;

struct GradFn {
    GradKind kind;
    Node node;
    std::vector<SavedTensor> inputs;
    float scalar = 0.0f;
    bool scalar_live = false;
    Dims dims;            // permute: the permutation
    int64_t index_start = 0;  // select: first input element of the output
    Dims out_shape;       // output shape of the recorded op
    SavedTensor output;   // exp: its own output (values saved)
    BytePtr mask;         // mask-apply: the keep-mask
    FusedBackward fused;  // fused: the gradient program
    std::vector<BytePtr> fused_bytes;  // fused: byte-buffer inputs by position (null for tensors)
};

struct AutogradMeta {
    bool leaf = true;
    // leaf
    Dims leaf_shape;
    Device device;
    std::mutex grad_mu;
    StoragePtr grad;
    // non-leaf
    std::mutex fn_mu;
    std::unique_ptr<GradFn> fn;
    ~AutogradMeta();
};

class Tensor {
public:
    StoragePtr storage;
    Dims shape, strides;
    int64_t offset = 0, numel = 1;
    int64_t output_nr = 0;
    bool view_requires_grad = false;
    MetaPtr autograd;

    Device device() const { return storage->device; }
    bool requires_grad() const { return autograd != nullptr || view_requires_grad; }
    bool is_leaf() const { return !(autograd && !autograd->leaf); }
    bool is_contiguous() const { return layout::is_contiguous(shape, strides, numel); }
    const char *grad_fn_name() const;
    trs_layout abi_layout() const;

    // construction
    static Tensor from_host(const float *data, const Dims &shape, Device device);
    static Tensor full(const Dims &shape, float value, Device device);
    Tensor with_requires_grad(bool flag) const;
    Tensor detach() const;
    Tensor to(Device device) const;
    std::vector<float> to_host() const;  // logical row-major values
    void copy_to_host(float *out) const;  // the same, into numel floats at `out`

    // views (src/tensor.rs:1082-1215, 2032-2189)
    Tensor permute(const Dims &dims, Node node = Node::Permute) const;
    Tensor transpose(int64_t d0, int64_t d1) const;
    Tensor squeeze() const;                                    // every size-1 dim
    Tensor squeeze_dim(int64_t dim) const;                     // that dim, if size 1
    Tensor squeeze_dims(const std::vector<int64_t> &dims) const;  // those dims that have size 1
    Tensor unsqueeze_front() const;                            // a leading size-1 dim
    Tensor matrix_transpose() const;
    Tensor reverse_dims() const;
    Tensor reshape(const std::vector<int64_t> &req) const;
    Tensor view(const std::vector<int64_t> &req) const;
    Tensor contiguous() const;
    Tensor clone() const;
    Tensor select(int64_t index) const;

    // pointwise (src/tensor.rs:2191-2411)
    Tensor add(const Tensor &o) const;
    Tensor sub(const Tensor &o) const;
    Tensor mul(const Tensor &o) const;
    Tensor div(const Tensor &o) const;
    Tensor add_scalar(float s) const;
    Tensor sub_scalar(float s) const;
    Tensor mul_scalar(float s) const;
    Tensor div_scalar(float s) const;
    Tensor scalar_sub(float s) const;
    Tensor scalar_div(float s) const;
    Tensor neg() const;
    Tensor relu() const;
    Tensor exp() const;
    Tensor sum() const;
    Tensor matmul(const Tensor &o) const;
    float item() const;
    void require_cuda(const char *what) const;

    // autograd
    void backward() const;
    bool has_grad() const;
    Tensor grad() const;       // a detached contiguous copy (Tensor::grad)
    Tensor live_grad() const;  // an alias of the accumulated storage (Tensor::live_grad)

private:
    Tensor binary_op(int op, const Tensor &o) const;
    Tensor scalar_op(int op, float s) const;
    Tensor unary_op(int op) const;
    Tensor alias_view(const Dims &shape, const Dims &strides, int64_t offset) const;
    Tensor squeeze_selected(const std::vector<bool> &selected, Node node) const;
};

// Dropout-apply with a precomputed keep-mask: (h * mask) * scale.
Tensor mask_apply(const Tensor &h, const BytePtr &mask, float scale);

// Thread-local no-grad depth (src/grad_mode.rs:5-38).
void enter_no_grad();
void exit_no_grad();
bool is_grad_enabled();

// Device helpers
int device_count();
void synchronize();
int current_device();
void set_device(int index);

// One argument of a fused program: a tensor, or (bytes set) a byte buffer
// read as an `in u8` operand, such as a dropout keep-mask.
struct FusedArg {
    Tensor tensor;
    BytePtr bytes;
};

// Fused pointwise program (compiled once, cached by IR text).
struct FusedProgram {
    uint64_t id = 0;
    int nin = 0;
    static FusedProgram compile(const std::string &ir, int nin);
    Tensor launch(const std::vector<FusedArg> &inputs, const Dims &out_shape, const Dims &out_strides) const;
    // The forward launch recorded as one graph node whose backward runs the
    // gradient program `bwd` (all input gradients in one kernel).
    Tensor launch_with_grad(const std::vector<FusedArg> &inputs, const Dims &out_shape, const Dims &out_strides,
                            const FusedBackward &bwd) const;
};

}  // namespace trs_engine
