// engine.cpp -- the C++ host engine above libtrs_hip.so: tensor metadata,
// output-layout planning, views and the reverse-mode graph of the pytorch-rs
// hot path (src/tensor.rs), with every element operation sent to the GPU
// through the C ABI in trs_hip.h.  Nothing here touches element values on
// the host except explicit host<->device transfers.
#include "engine.h"

#include <algorithm>
#include <cstring>
#include <map>
#include <sstream>
#include <utility>

namespace trs_engine {

namespace {

// Raises the library's last error as the Python-visible TensorError.
void check(int rc) {
    if (rc == TRS_OK) return;
    throw TensorError(trs_last_error());
}

// Reference-style shape rendering for messages: [2, 3].
std::string dims_str(const Dims &d) {
    std::ostringstream s;
    s << "[";
    for (size_t i = 0; i < d.size(); i++) s << (i ? ", " : "") << d[i];
    s << "]";
    return s.str();
}

thread_local int g_no_grad_depth = 0;

// BACKWARD_TRAVERSAL (src/tensor.rs:21): one reverse pass at a time, so two
// roots sharing saved values cannot each consume part of the graph.
std::mutex g_backward_mu;

}  // namespace

// ---- grad mode (src/grad_mode.rs:5-38) ------------------------------------

void enter_no_grad() { g_no_grad_depth++; }
void exit_no_grad() {
    if (g_no_grad_depth > 0) g_no_grad_depth--;
}
bool is_grad_enabled() { return g_no_grad_depth == 0; }

// ---- device ----------------------------------------------------------------

std::string Device::str() const {
    if (type == DeviceType::CPU) return "cpu";
    return "cuda:" + std::to_string(index < 0 ? 0 : index);
}

Device Device::parse(const std::string &s) {
    Device d;
    if (s == "cpu") return d;
    if (s == "cuda" || s.rfind("cuda:", 0) == 0) {
        d.type = DeviceType::CUDA;
        d.index = 0;
        if (s.size() > 5) {
            char *end = nullptr;
            long v = std::strtol(s.c_str() + 5, &end, 10);
            if (*end != '\0' || v < 0) throw TensorError("Invalid device string: '" + s + "'");
            d.index = (int)v;
        }
        return d;
    }
    throw TensorError("Expected one of cpu, cuda device type at start of device string: " + s);
}

int device_count() {
    int n = 0;
    if (trs_device_count(&n) != TRS_OK) return 0;
    return n;
}

void synchronize() { check(trs_synchronize()); }

int current_device() {
    int d = 0;
    check(trs_get_device(&d));
    return d;
}

void set_device(int index) { check(trs_set_device(index)); }

static void select_device(const Device &d) {
    if (!d.is_cuda()) return;
    int cur = -1;
    check(trs_get_device(&cur));
    if (cur != d.index) check(trs_set_device(d.index));
}

// ---- storage (src/storage.rs:7-18) ------------------------------------------

// Destructors must not throw: select the device without error checks.
static void select_device_quietly(const Device &d) {
    int cur = -1;
    if (d.is_cuda() && trs_get_device(&cur) == TRS_OK && cur != d.index) (void)trs_set_device(d.index);
}

Storage::~Storage() {
    if (dptr) {
        select_device_quietly(device);
        (void)trs_free(dptr);  // stream-ordered return to the library's block cache
    }
}

std::shared_ptr<Storage> Storage::allocate(Device device, int64_t numel) {
    auto s = std::make_shared<Storage>();
    s->device = device;
    s->numel = numel;
    if (device.is_cuda()) {
        select_device(device);
        void *p = nullptr;
        if (numel > 0) {
            int rc = trs_alloc((size_t)numel * sizeof(float), &p);
            if (rc != TRS_OK)
                throw TensorError("failed to allocate storage for " + std::to_string(numel) + " elements");
        }
        s->dptr = (float *)p;
    } else {
        try {
            s->host.assign((size_t)numel, 0.0f);
        } catch (const std::bad_alloc &) {
            throw TensorError("failed to allocate storage for " + std::to_string(numel) + " elements");
        }
    }
    return s;
}

// ---- layout planning (src/tensor.rs:3695-4458) --------------------------------

namespace layout {

int64_t numel_of(const Dims &shape) {
    int64_t n = 1;
    for (int64_t d : shape) {
        if (d != 0 && n > INT64_MAX / d) throw TensorError("tensor element count overflowed usize");
        n *= d;
    }
    return n;
}

std::string shape_str(const Dims &d) { return dims_str(d); }

// contiguous_strides (src/tensor.rs:4198-4209): the stride of axis 0 is not
// multiplied by its own size, and singleton/empty dims count as 1.
Dims contiguous_strides(const Dims &shape) {
    Dims st(shape.size(), 0);
    int64_t stride = 1;
    for (int a = (int)shape.size() - 1; a >= 0; a--) {
        st[a] = stride;
        if (a > 0) {
            const int64_t d = std::max<int64_t>(shape[a], 1);
            if (stride > INT64_MAX / d) throw TensorError("Stride calculation overflowed");
            stride *= d;
        }
    }
    return st;
}

// layout_is_contiguous (src/tensor.rs:3695-3715).
bool is_contiguous(const Dims &shape, const Dims &strides, int64_t numel) {
    if (numel == 0) return true;
    int64_t expected = 1;
    for (int a = (int)shape.size() - 1; a >= 0; a--) {
        if (shape[a] == 1) continue;
        if (strides[a] != expected) return false;
        expected *= shape[a];
    }
    return true;
}

// is_non_overlapping_and_dense (src/tensor.rs:1019-1053): every non-singleton
// dim's stride must be the product of the sizes below it, found exactly once.
bool is_non_overlapping_and_dense(const Dims &shape, const Dims &strides, int64_t numel) {
    if (numel == 0) return true;
    int dims = 0;
    for (int64_t d : shape) dims += d > 1;
    int64_t expected = 1;
    for (int m = 0; m < dims; m++) {
        int found = -1;
        for (size_t a = 0; a < shape.size(); a++) {
            if (shape[a] > 1 && strides[a] == expected) {
                if (found >= 0) return false;
                found = (int)a;
            }
        }
        if (found < 0) return false;
        expected *= shape[found];
    }
    return true;
}

// Channels-last (rank 4, physical order [1,3,2,0]) predicate and strides
// (src/tensor.rs:3717-3719, 3765-3791, 4211-4247).
bool is_channels_last_contiguous(const Dims &shape, const Dims &strides) {
    if (shape.size() != 4) return false;
    static const int order[4] = {1, 3, 2, 0};
    bool empty = false;
    for (int64_t d : shape) empty |= d == 0;
    uint64_t expected = 1;
    for (int axis : order) {
        const int64_t d = shape[axis];
        if (d == 1) continue;
        if ((uint64_t)strides[axis] != expected) return false;
        uint64_t next;
        if (__builtin_mul_overflow(expected, (uint64_t)d, &next)) {
            if (!empty) return false;
            next = expected * (uint64_t)d;
        }
        expected = next;
    }
    return true;
}

Dims channels_last_strides(const Dims &shape) {
    if (shape.size() != 4) throw TensorError("Stride calculation overflowed");
    (void)contiguous_strides(shape);
    static const int order[4] = {1, 3, 2, 0};
    Dims st(4, 0);
    int64_t stride = 1;
    for (int p = 0; p < 4; p++) {
        st[order[p]] = stride;
        if (p + 1 < 4) {
            const int64_t d = shape[order[p]];
            if (d != 0 && stride > INT64_MAX / d) throw TensorError("Stride calculation overflowed");
            stride *= d;
        }
    }
    return st;
}

namespace {

// ElementwiseLayout::aligned_broadcast_stride (src/tensor.rs:4114-4131) as
// TensorIterator's wrapping i64 byte stride (:4133-4151).
int64_t bcast_stride_bytes(const std::pair<Dims, Dims> &op, size_t out_rank, size_t axis, int64_t out_dim) {
    const size_t lead = out_rank - op.first.size();
    if (axis < lead) return 0;
    const size_t ia = axis - lead;
    const uint64_t s = (op.first[ia] == 1 && out_dim != 1) ? 0 : (uint64_t)op.second[ia];
    return (int64_t)(s * 4u);
}

// compare_elementwise_dimensions (src/tensor.rs:4315-4336).
int compare_dims(const Dims &shape, const std::vector<std::pair<Dims, Dims>> &ops, int d0, int d1) {
    for (const auto &op : ops) {
        const int64_t s0 = bcast_stride_bytes(op, shape.size(), d0, shape[d0]);
        const int64_t s1 = bcast_stride_bytes(op, shape.size(), d1, shape[d1]);
        if (s0 == 0 || s1 == 0) continue;
        if (s0 < s1) return -1;
        if (s0 > s1 || shape[d0] > shape[d1]) return 1;
    }
    return 0;
}

}  // namespace

// elementwise_output_strides (src/tensor.rs:4249-4312): insertion-sort the
// dims by operand byte strides (first operand that decides wins), then lay
// the output out densely in that order with TensorIterator's wrapping i64
// byte-stride arithmetic.
Dims elementwise_output_strides(const Dims &shape, const std::vector<std::pair<Dims, Dims>> &ops) {
    const int rank = (int)shape.size();
    std::vector<int> perm(rank);
    for (int i = 0; i < rank; i++) perm[i] = rank - 1 - i;
    for (int index = 1; index < rank; index++) {
        int d1 = index;
        for (int d0 = index - 1; d0 >= 0; d0--) {
            const int c = compare_dims(shape, ops, perm[d0], perm[d1]);
            if (c > 0) {
                std::swap(perm[d0], perm[d1]);
                d1 = d0;
            } else if (c < 0) {
                break;
            }
        }
    }
    bool identity = true;
    for (int i = 0; i < rank; i++) identity &= perm[i] == rank - i - 1;
    if (identity) return contiguous_strides(shape);
    std::vector<int64_t> bytes(rank, 0);
    int64_t next = 4;
    for (int p = 0; p < rank; p++) {
        bytes[perm[p]] = next;
        if (p + 1 < rank) next = (int64_t)((uint64_t)next * (uint64_t)shape[perm[p]]);
    }
    Dims out(rank, 0);
    for (int a = rank - 1; a >= 0; a--) {
        const int64_t s = bytes[a] / 4;
        if (s >= 0) {
            out[a] = s;
        } else if (a + 1 == rank) {
            out[a] = 1;
        } else {
            const int64_t d = std::max<int64_t>(shape[a + 1], 1);
            if (out[a + 1] > INT64_MAX / d) throw TensorError("Stride calculation overflowed");
            out[a] = out[a + 1] * d;
        }
    }
    return out;
}

// unary_output_strides (src/tensor.rs:2751-2766).
Dims unary_output_strides(const Dims &shape, const Dims &strides, int64_t numel) {
    if (is_contiguous(shape, strides, numel)) return contiguous_strides(shape);
    if (is_channels_last_contiguous(shape, strides)) return channels_last_strides(shape);
    if (is_non_overlapping_and_dense(shape, strides, numel)) return strides;
    return elementwise_output_strides(shape, {{shape, strides}});
}

// map_scalar's layout (src/tensor.rs:2718-2735).
Dims scalar_output_strides(const Dims &shape, const Dims &strides) {
    return elementwise_output_strides(shape, {{shape, strides}});
}

// zip_map's layout: zip_map_same_shape (src/tensor.rs:2629-2656) for equal
// shapes, BroadcastPlan::new (:3601-3693) otherwise.
void binary_output_layout(const Dims &ls, const Dims &lt, const Dims &rs, const Dims &rt, Dims &oshape,
                          Dims &ostr) {
    if (ls == rs) {
        const int64_t n = numel_of(ls);
        oshape = ls;
        if (is_contiguous(ls, lt, n) && is_contiguous(rs, rt, n)) {
            ostr = contiguous_strides(ls);
        } else if (is_channels_last_contiguous(ls, lt) && is_channels_last_contiguous(rs, rt)) {
            ostr = channels_last_strides(ls);
        } else if (is_non_overlapping_and_dense(ls, lt, n) && is_non_overlapping_and_dense(rs, rt, n) && lt == rt) {
            ostr = lt;
        } else {
            ostr = elementwise_output_strides(ls, {{ls, lt}, {rs, rt}});
        }
        return;
    }
    const size_t rank = std::max(ls.size(), rs.size());
    oshape.assign(rank, 0);
    for (size_t a = 0; a < rank; a++) {
        const size_t la = rank - ls.size(), ra = rank - rs.size();
        const int64_t l = a < la ? 1 : ls[a - la];
        const int64_t r = a < ra ? 1 : rs[a - ra];
        if (l == r || r == 1) oshape[a] = l;
        else if (l == 1) oshape[a] = r;
        else {
            // format_shape_mismatch (src/tensor_error.rs:217-233)
            throw TensorError("The size of tensor a (" + std::to_string(l) + ") must match the size of tensor b (" +
                              std::to_string(r) + ") at non-singleton dimension " + std::to_string(a));
        }
    }
    (void)numel_of(oshape);
    ostr = elementwise_output_strides(oshape, {{ls, lt}, {rs, rt}});
}

// compute_reshape_view_strides (src/tensor.rs:3996-4055): walks the old
// layout in contiguous chunks and assigns the new dims to them.
bool reshape_view_strides(const Dims &old_shape, const Dims &old_strides, const Dims &new_shape, int64_t numel,
                          Dims &out) {
    if (numel == 0) {
        out = (new_shape == old_shape) ? old_strides : reshape_strides(new_shape, numel);
        return true;
    }
    if (old_shape.empty()) {
        out = contiguous_strides(new_shape);
        return true;
    }
    out.assign(new_shape.size(), 0);
    int view_dim = (int)new_shape.size();
    int64_t chunk_base = old_strides.back();
    int64_t tensor_elems = 1, view_elems = 1;
    for (int td = (int)old_shape.size() - 1; td >= 0; td--) {
        tensor_elems *= old_shape[td];
        const bool chunk_ends = td == 0 || (old_shape[td - 1] != 1 && old_strides[td - 1] != tensor_elems * chunk_base);
        if (!chunk_ends) continue;
        while (view_dim > 0 && (view_elems < tensor_elems || new_shape[view_dim - 1] == 1)) {
            view_dim--;
            out[view_dim] = view_elems * chunk_base;
            view_elems *= new_shape[view_dim];
        }
        if (view_elems != tensor_elems) return false;
        if (td > 0) {
            chunk_base = old_strides[td - 1];
            tensor_elems = 1;
            view_elems = 1;
        }
    }
    return view_dim == 0;
}

// reshape_strides (src/tensor.rs:4338-4356).
Dims reshape_strides(const Dims &shape, int64_t numel) {
    if (numel != 0) return contiguous_strides(shape);
    Dims st(shape.size(), 0);
    int64_t stride = 1;
    for (int a = (int)shape.size() - 1; a >= 0; a--) {
        st[a] = stride;
        if (a > 0) stride = (int64_t)((uint64_t)stride * (uint64_t)std::max<int64_t>(shape[a], 1));
    }
    return st;
}

}  // namespace layout

// ---- node names (src/autograd_node.rs:5-59) ----------------------------------

const char *node_name(Node n) {
    switch (n) {
    case Node::Add: return "AddBackward0";
    case Node::Alias: return "AliasBackward0";
    case Node::Clone: return "CloneBackward0";
    case Node::Multiply: return "MulBackward0";
    case Node::Negate: return "NegBackward0";
    case Node::Permute: return "PermuteBackward0";
    case Node::Relu: return "ReluBackward0";
    case Node::ReflectedSubtract: return "RsubBackward1";
    case Node::Subtract: return "SubBackward0";
    case Node::Sum: return "SumBackward0";
    case Node::MatrixTranspose: return "TBackward0";
    case Node::Transpose: return "TransposeBackward0";
    case Node::View: return "ViewBackward0";
    case Node::Select: return "SelectBackward0";
    case Node::Exp: return "ExpBackward0";
    case Node::Mm: return "MmBackward0";
    case Node::Bmm: return "BmmBackward0";
    case Node::AddTensor: return "AddBackward0";
    case Node::SubTensor: return "SubBackward0";
    case Node::Squeeze: return "SqueezeBackward0";
    case Node::SqueezeDimension: return "SqueezeBackward1";
    case Node::SqueezeDimensions: return "SqueezeBackward2";
    case Node::Unsqueeze: return "UnsqueezeBackward0";
    case Node::Fused: return "FusedBackward0";
    }
    return "UnknownBackward";
}

AutogradMeta::~AutogradMeta() {
    // Iterative teardown of long chains (src/tensor.rs:189-206): detach the
    // parents of every uniquely owned node before it is destroyed, so a
    // 20k-deep graph does not recurse.
    std::vector<MetaPtr> pending;
    if (fn) {
        for (auto &in : fn->inputs)
            if (in.autograd) pending.push_back(std::move(in.autograd));
        fn.reset();
    }
    while (!pending.empty()) {
        MetaPtr p = std::move(pending.back());
        pending.pop_back();
        if (p.use_count() == 1 && p->fn) {
            for (auto &in : p->fn->inputs)
                if (in.autograd) pending.push_back(std::move(in.autograd));
            p->fn.reset();
        }
    }
}

// ---- tensor basics -----------------------------------------------------------

trs_layout Tensor::abi_layout() const {
    if (shape.size() > TRS_MAX_RANK) throw TensorError("tensors above rank " + std::to_string(TRS_MAX_RANK) + " are not supported on the device");
    trs_layout l{};
    l.rank = (int32_t)shape.size();
    for (size_t i = 0; i < shape.size(); i++) {
        l.shape[i] = shape[i];
        l.stride[i] = strides[i];
    }
    l.offset = offset;
    return l;
}

static trs_layout abi_layout_of(const Dims &shape, const Dims &strides, int64_t offset) {
    if (shape.size() > TRS_MAX_RANK) throw TensorError("tensors above rank " + std::to_string(TRS_MAX_RANK) + " are not supported on the device");
    trs_layout l{};
    l.rank = (int32_t)shape.size();
    for (size_t i = 0; i < shape.size(); i++) {
        l.shape[i] = shape[i];
        l.stride[i] = strides[i];
    }
    l.offset = offset;
    return l;
}

const char *Tensor::grad_fn_name() const {
    if (!autograd || autograd->leaf || !autograd->fn) return nullptr;
    return node_name(autograd->fn->node);
}

void Tensor::require_cuda(const char *what) const {
    if (!device().is_cuda())
        throw TensorError(std::string(what) +
                          ": this backend computes on device tensors only; move the tensor with .to(\"cuda\")");
    select_device(device());
}

static Tensor make_tensor(StoragePtr st, Dims shape, Dims strides, int64_t offset) {
    Tensor t;
    t.storage = std::move(st);
    t.numel = layout::numel_of(shape);
    t.shape = std::move(shape);
    t.strides = std::move(strides);
    t.offset = offset;
    return t;
}

// A fresh device tensor of `shape` laid out with `strides` (dense).
static Tensor empty_like_layout(Device dev, const Dims &shape, const Dims &strides) {
    const int64_t n = layout::numel_of(shape);
    return make_tensor(Storage::allocate(dev, n), shape, strides, 0);
}

Tensor Tensor::from_host(const float *data, const Dims &shape, Device device) {
    const int64_t n = layout::numel_of(shape);
    Tensor t = make_tensor(Storage::allocate(device, n), shape, layout::contiguous_strides(shape), 0);
    if (n > 0) {
        if (device.is_cuda()) check(trs_memcpy_h2d(t.storage->dptr, data, (size_t)n * sizeof(float)));
        else std::memcpy(t.storage->host.data(), data, (size_t)n * sizeof(float));
    }
    return t;
}

Tensor Tensor::full(const Dims &shape, float value, Device device) {
    const int64_t n = layout::numel_of(shape);
    Tensor t = make_tensor(Storage::allocate(device, n), shape, layout::contiguous_strides(shape), 0);
    if (n > 0) {
        if (device.is_cuda()) check(trs_fill_f32(t.storage->dptr, (size_t)n, value));
        else std::fill(t.storage->host.begin(), t.storage->host.end(), value);
    }
    return t;
}

// Tensor::with_requires_grad (src/tensor.rs:780-798).
Tensor Tensor::with_requires_grad(bool flag) const {
    Tensor t = *this;
    if (!flag) {
        t.autograd.reset();
        t.output_nr = 0;
        t.view_requires_grad = false;
    } else if (!t.autograd) {
        auto m = std::make_shared<AutogradMeta>();
        m->leaf = true;
        m->leaf_shape = shape;
        m->device = device();
        t.autograd = m;
        t.output_nr = 0;
        t.view_requires_grad = false;
    }
    return t;
}

Tensor Tensor::detach() const {
    Tensor t = *this;
    t.autograd.reset();
    t.output_nr = 0;
    t.view_requires_grad = false;
    return t;
}

// Logical row-major values written to `out` (numel floats of host memory).
void Tensor::copy_to_host(float *out) const {
    if (numel == 0) return;
    if (device().is_cuda()) {
        select_device(device());
        if (is_contiguous()) {
            check(trs_memcpy_d2h(out, storage->dptr + offset, (size_t)numel * sizeof(float)));
        } else {
            Tensor c = contiguous();
            check(trs_memcpy_d2h(out, c.storage->dptr + c.offset, (size_t)numel * sizeof(float)));
        }
        return;
    }
    // host odometer over the strided view
    const int rank = (int)shape.size();
    std::vector<int64_t> idx(rank, 0);
    int64_t off = offset;
    for (int64_t i = 0; i < numel; i++) {
        out[(size_t)i] = storage->host[(size_t)off];
        for (int a = rank - 1; a >= 0; a--) {
            if (++idx[a] < shape[a]) {
                off += strides[a];
                break;
            }
            off -= strides[a] * (shape[a] - 1);
            idx[a] = 0;
        }
    }
}

std::vector<float> Tensor::to_host() const {
    std::vector<float> out((size_t)numel);
    copy_to_host(out.data());
    return out;
}

// Device transfer: copies the logical values into a fresh contiguous tensor
// on `dev` (the same device returns this tensor).  A transfer of a tensor
// that requires grad records a Transfer edge; backward through it raises,
// because its gradient would have to be accumulated in host memory.
Tensor Tensor::to(Device dev) const {
    if (dev == device()) return *this;
    const std::vector<float> host = to_host();
    Tensor out = from_host(host.data(), shape, dev);
    if (requires_grad() && is_grad_enabled() && autograd) {
        auto m = std::make_shared<AutogradMeta>();
        m->leaf = false;
        auto fn = std::make_unique<GradFn>();
        fn->kind = GradKind::Transfer;
        fn->node = Node::Clone;
        SavedTensor s;
        s.shape = shape;
        s.strides = strides;
        s.offset = offset;
        s.numel = numel;
        s.output_nr = output_nr;
        s.autograd = autograd;
        fn->inputs.push_back(std::move(s));
        fn->out_shape = shape;
        m->fn = std::move(fn);
        out.autograd = m;
    }
    return out;
}

// ---- graph recording ----------------------------------------------------------

// SavedTensor::try_from_tensor (src/tensor.rs:2809-2825): storages are
// immutable once written and are shared, except a leaf's accumulated
// gradient, which later backward passes change in place: its values are
// snapshotted (Storage::try_clone_for_saved), in stream order.
static StoragePtr saved_values(const StoragePtr &st) {
    if (!st->shared_gradient) return st;
    StoragePtr copy = Storage::allocate(st->device, st->numel);
    if (st->numel == 0) return copy;
    if (st->device.is_cuda()) {
        select_device(st->device);
        check(trs_memcpy_d2d(copy->dptr, st->dptr, (size_t)st->numel * sizeof(float)));
    } else {
        copy->host = st->host;
    }
    return copy;
}

static SavedTensor save(const Tensor &t, bool values) {
    SavedTensor s;
    if (values) s.values = saved_values(t.storage);
    s.values_required = values;
    s.shape = t.shape;
    s.strides = t.strides;
    s.offset = t.offset;
    s.numel = t.numel;
    s.output_nr = t.output_nr;
    s.autograd = t.autograd;
    return s;
}

static bool records(const Tensor &t) { return t.requires_grad() && is_grad_enabled(); }

static void attach(Tensor &out, std::unique_ptr<GradFn> fn) {
    auto m = std::make_shared<AutogradMeta>();
    m->leaf = false;
    fn->out_shape = out.shape;
    m->fn = std::move(fn);
    out.autograd = m;
    out.output_nr = 0;
}

// record_transform (src/tensor.rs:903-922): an identity or permute edge with
// metadata only.
static void record_transform(const Tensor &in, Tensor &out, GradKind kind, Node node, const Dims &dims = {}) {
    if (!records(in)) return;
    auto fn = std::make_unique<GradFn>();
    fn->kind = kind;
    fn->node = node;
    fn->dims = dims;
    fn->inputs.push_back(save(in, false));
    attach(out, std::move(fn));
}

// ---- views (src/tensor.rs:1082-1215, 2032-2189) --------------------------------

Tensor Tensor::alias_view(const Dims &shp, const Dims &str, int64_t off) const {
    Tensor t = make_tensor(storage, shp, str, off);
    t.view_requires_grad = requires_grad();
    return t;
}

// permute_axes_with_grad_fn (src/tensor.rs:1086-1148).
Tensor Tensor::permute(const Dims &dims, Node node) const {
    const size_t rank = shape.size();
    if (dims.size() != rank)
        throw TensorError("number of dimensions in the tensor input does not match the length of the desired ordering "
                          "of dimensions i.e. input.dim() = " + std::to_string(rank) +
                          " is not equal to len(dims) = " + std::to_string(dims.size()));
    std::vector<bool> seen(rank, false);
    for (int64_t d : dims) {
        if (d < 0 || (size_t)d >= rank)
            throw TensorError("permutation dimension " + std::to_string(d) + " is out of range for tensor rank " +
                              std::to_string(rank));
        if (seen[d]) throw TensorError("permute(): duplicate dims are not allowed.");
        seen[d] = true;
    }
    Dims s, st;
    for (int64_t d : dims) {
        s.push_back(shape[d]);
        st.push_back(strides[d]);
    }
    Tensor out = alias_view(s, st, offset);
    record_transform(*this, out, GradKind::Permute, node, dims);
    return out;
}

static int64_t normalize_dim(int64_t d, size_t rank) {
    const int64_t r = std::max<int64_t>((int64_t)rank, 1);
    if (d < -r || d >= r)
        throw IndexError("Dimension out of range (expected to be in range of [-" + std::to_string(r) + ", " +
                         std::to_string(r - 1) + "], but got " + std::to_string(d) + ")");
    return d < 0 ? d + r : d;
}

// transpose (src/tensor.rs:1184-1194).
Tensor Tensor::transpose(int64_t d0, int64_t d1) const {
    const int64_t a0 = normalize_dim(d0, shape.size()), a1 = normalize_dim(d1, shape.size());
    Dims dims(shape.size());
    for (size_t i = 0; i < dims.size(); i++) dims[i] = (int64_t)i;
    if (!dims.empty()) std::swap(dims[a0], dims[a1]);
    return permute(dims, Node::Transpose);
}

// squeeze / squeeze_dim / squeeze_dims (src/tensor.rs:1305-1390): drop the
// selected size-1 dims; storage, offset and the logical order are unchanged,
// so the gradient maps back as Identity.
Tensor Tensor::squeeze_selected(const std::vector<bool> &selected, Node node) const {
    Dims s, st;
    for (size_t a = 0; a < shape.size(); a++) {
        if (selected[a] && shape[a] == 1) continue;
        s.push_back(shape[a]);
        st.push_back(strides[a]);
    }
    Tensor out = alias_view(s, st, offset);
    record_transform(*this, out, GradKind::Identity, node);
    return out;
}

Tensor Tensor::squeeze() const {
    return squeeze_selected(std::vector<bool>(shape.size(), true), Node::Squeeze);
}

Tensor Tensor::squeeze_dim(int64_t dim) const {
    const int64_t a = normalize_dim(dim, shape.size());
    std::vector<bool> sel(shape.size(), false);
    if (!sel.empty()) sel[a] = true;
    return squeeze_selected(sel, Node::SqueezeDimension);
}

Tensor Tensor::squeeze_dims(const std::vector<int64_t> &dims) const {
    if (shape.size() > 64) throw TensorError("only tensors with up to 64 dims are supported");
    std::vector<bool> sel(shape.size(), false);
    std::vector<bool> seen(std::max<size_t>(shape.size(), 1), false);
    for (int64_t d : dims) {
        const int64_t a = normalize_dim(d, shape.size());
        if (seen[a]) throw TensorError("dim " + std::to_string(a) + " appears multiple times in the list of dims");
        seen[a] = true;
        if (!sel.empty()) sel[a] = true;
    }
    return squeeze_selected(sel, Node::SqueezeDimensions);
}

// unsqueeze_front (src/tensor.rs:1218-1268): a leading size-1 dim whose
// stride is stride[0] * shape[0] (1 for a scalar); Identity mapping.
Tensor Tensor::unsqueeze_front() const {
    Dims s{1}, st;
    st.push_back(shape.empty() ? 1 : (int64_t)((uint64_t)strides[0] * (uint64_t)shape[0]));
    s.insert(s.end(), shape.begin(), shape.end());
    st.insert(st.end(), strides.begin(), strides.end());
    Tensor out = alias_view(s, st, offset);
    record_transform(*this, out, GradKind::Identity, Node::Unsqueeze);
    return out;
}

// matrix_transpose = .mT (src/tensor.rs:1209-1215).
Tensor Tensor::matrix_transpose() const {
    if (shape.empty()) {
        Tensor out = alias_view(shape, strides, offset);
        record_transform(*this, out, GradKind::Identity, Node::Alias);
        return out;
    }
    if (shape.size() == 1)
        throw TensorError("tensor.mT is only supported on matrices or batches of matrices. Got 1-D tensor.");
    return transpose(-2, -1);
}

// reverse_dimensions (.T / .t(), src/tensor.rs:1150-1167).
Tensor Tensor::reverse_dims() const {
    Dims dims;
    for (int64_t i = (int64_t)shape.size() - 1; i >= 0; i--) dims.push_back(i);
    return permute(dims, Node::MatrixTranspose);
}

// resolve_reshape_shape (src/tensor.rs:2063-2122).
static Dims resolve_reshape(const std::vector<int64_t> &req, int64_t numel) {
    int inferred = -1;
    for (size_t i = 0; i < req.size(); i++) {
        if (req[i] == -1) {
            if (inferred >= 0) throw TensorError("only one dimension can be inferred");
            inferred = (int)i;
            continue;
        }
        if (req[i] < 0)
            throw TensorError("invalid shape dimension " + std::to_string(req[i]) + " at index " + std::to_string(i) +
                              " of shape " + dims_str(req));
    }
    Dims resolved;
    for (int64_t d : req) resolved.push_back(d == -1 ? 1 : d);
    if (inferred >= 0) {
        int64_t spec = 1;
        for (int64_t d : req)
            if (d != -1) spec = (int64_t)((uint64_t)spec * (uint64_t)d);
        if (!((spec > 0 && numel % spec == 0) || numel == spec))
            throw TensorError("shape '" + dims_str(req) + "' is invalid for input of size " + std::to_string(numel));
        if (spec == 0) {
            if (numel == 0)
                throw TensorError("cannot reshape tensor of 0 elements into shape " + dims_str(req) +
                                  " because the unspecified dimension size -1 can be any value and is ambiguous");
            throw TensorError("shape '" + dims_str(req) + "' is invalid for input of size " + std::to_string(numel));
        }
        resolved[inferred] = numel / spec;
    }
    if (layout::numel_of(resolved) != numel)
        throw TensorError("shape '" + dims_str(req) + "' is invalid for input of size " + std::to_string(numel));
    return resolved;
}

Tensor Tensor::view(const std::vector<int64_t> &req) const {
    const Dims resolved = resolve_reshape(req, numel);
    Dims st;
    if (!layout::reshape_view_strides(shape, strides, resolved, numel, st))
        throw TensorError("view size is not compatible with input tensor's size and stride (at least one dimension "
                          "spans across two contiguous subspaces). Use .reshape(...) instead.");
    Tensor out = alias_view(resolved, st, offset);
    record_transform(*this, out, GradKind::Identity, Node::View);
    return out;
}

// reshape_resolved (src/tensor.rs:2124-2148): a view when the layout allows,
// else a contiguous copy recorded as the same View node.
Tensor Tensor::reshape(const std::vector<int64_t> &req) const {
    const Dims resolved = resolve_reshape(req, numel);
    Dims st;
    if (layout::reshape_view_strides(shape, strides, resolved, numel, st)) {
        Tensor out = alias_view(resolved, st, offset);
        record_transform(*this, out, GradKind::Identity, Node::View);
        return out;
    }
    Tensor packed = detach().contiguous();
    Tensor out = make_tensor(packed.storage, resolved, layout::contiguous_strides(resolved), packed.offset);
    record_transform(*this, out, GradKind::Identity, Node::View);
    return out;
}

// try_contiguous_impl (src/tensor.rs:1598-1660): an alias when already
// contiguous, else a materialised copy, both recorded as Clone.
Tensor Tensor::contiguous() const {
    if (is_contiguous()) {
        Tensor out = alias_view(shape, strides, offset);
        record_transform(*this, out, GradKind::Identity, Node::Clone);
        return out;
    }
    require_cuda("contiguous");
    Tensor out = empty_like_layout(device(), shape, layout::contiguous_strides(shape));
    const trs_layout li = abi_layout(), lo = out.abi_layout();
    check(trs_unary_f32(TRS_COPY, storage->dptr, &li, out.storage->dptr, &lo));
    record_transform(*this, out, GradKind::Identity, Node::Clone);
    return out;
}

// try_clone (Preserve, src/tensor.rs:1517-1566).
Tensor Tensor::clone() const {
    require_cuda("clone");
    Dims st = (numel == 0 || layout::is_non_overlapping_and_dense(shape, strides, numel))
                  ? strides
                  : layout::elementwise_output_strides(shape, {{shape, strides}});
    Tensor out = empty_like_layout(device(), shape, st);
    if (numel > 0) {
        const trs_layout li = abi_layout(), lo = out.abi_layout();
        check(trs_unary_f32(TRS_COPY, storage->dptr, &li, out.storage->dptr, &lo));
    }
    record_transform(*this, out, GradKind::Identity, Node::Clone);
    return out;
}

// Leading-dimension integer index (src/tensor.rs:1840-1890): a view.
Tensor Tensor::select(int64_t index) const {
    if (shape.empty())
        throw IndexError("invalid index of a 0-dim tensor. Use `tensor.item()` in Python or `tensor.item<T>()` in "
                         "C++ to convert a 0-dim tensor to a number");
    const int64_t size = shape[0];
    if (index < -size || index >= size)
        throw IndexError("index " + std::to_string(index) + " is out of bounds for dimension 0 with size " +
                         std::to_string(size));
    if (index < 0) index += size;
    Dims s(shape.begin() + 1, shape.end()), st(strides.begin() + 1, strides.end());
    Tensor out = alias_view(s, st, offset + index * strides[0]);
    if (records(*this)) {
        auto fn = std::make_unique<GradFn>();
        fn->kind = GradKind::Index;
        fn->node = Node::Select;
        fn->index_start = index * layout::numel_of(s);
        fn->inputs.push_back(save(*this, false));
        attach(out, std::move(fn));
    }
    return out;
}

// ---- pointwise (src/tensor.rs:2191-2411) ----------------------------------------

Tensor Tensor::binary_op(int op, const Tensor &o) const {
    Dims oshape, ostr;
    layout::binary_output_layout(shape, strides, o.shape, o.strides, oshape, ostr);
    require_cuda("binary op");
    if (!(o.device() == device()))
        throw TensorError("Expected all tensors to be on the same device, but found at least two devices, " +
                          device().str() + " and " + o.device().str() + "!");
    Tensor out = empty_like_layout(device(), oshape, ostr);
    if (out.numel > 0) {
        const trs_layout la = abi_layout(), lb = o.abi_layout(), lo = out.abi_layout();
        check(trs_binary_f32(op, storage->dptr, &la, o.storage->dptr, &lb, out.storage->dptr, &lo));
    }
    return out;
}

Tensor Tensor::scalar_op(int op, float s) const {
    require_cuda("scalar op");
    Dims ostr = op == TRS_S_RDIV
                    ? layout::elementwise_output_strides(shape, {{shape, layout::unary_output_strides(shape, strides, numel)}})
                    : layout::scalar_output_strides(shape, strides);
    Tensor out = empty_like_layout(device(), shape, ostr);
    if (numel > 0) {
        const trs_layout la = abi_layout(), lo = out.abi_layout();
        check(trs_binary_scalar_f32(op, storage->dptr, &la, s, out.storage->dptr, &lo));
    }
    return out;
}

Tensor Tensor::unary_op(int op) const {
    require_cuda("unary op");
    Tensor out = empty_like_layout(device(), shape, layout::unary_output_strides(shape, strides, numel));
    if (numel > 0) {
        const trs_layout la = abi_layout(), lo = out.abi_layout();
        check(trs_unary_f32(op, storage->dptr, &la, out.storage->dptr, &lo));
    }
    return out;
}

// Tensor-tensor add/sub record no edge in the reference
// (src/tensor.rs:2197-2209); this backend adds the broadcast-reducing VJP for
// device tensors.
Tensor Tensor::add(const Tensor &o) const {
    Tensor out = binary_op(TRS_ADD, o);
    if ((requires_grad() || o.requires_grad()) && is_grad_enabled()) {
        auto fn = std::make_unique<GradFn>();
        fn->kind = GradKind::AddTensor;
        fn->node = Node::AddTensor;
        fn->inputs.push_back(save(*this, false));
        fn->inputs.push_back(save(o, false));
        attach(out, std::move(fn));
    }
    return out;
}

Tensor Tensor::sub(const Tensor &o) const {
    Tensor out = binary_op(TRS_SUB, o);
    if ((requires_grad() || o.requires_grad()) && is_grad_enabled()) {
        auto fn = std::make_unique<GradFn>();
        fn->kind = GradKind::SubTensor;
        fn->node = Node::SubTensor;
        fn->inputs.push_back(save(*this, false));
        fn->inputs.push_back(save(o, false));
        attach(out, std::move(fn));
    }
    return out;
}

// mul (src/tensor.rs:2217-2236): each side saves the other's values only when
// the other side has an edge.
Tensor Tensor::mul(const Tensor &o) const {
    Tensor out = binary_op(TRS_MUL, o);
    if ((requires_grad() || o.requires_grad()) && is_grad_enabled()) {
        const bool left_edge = autograd != nullptr, right_edge = o.autograd != nullptr;
        auto fn = std::make_unique<GradFn>();
        fn->kind = GradKind::Multiply;
        fn->node = Node::Multiply;
        fn->inputs.push_back(save(*this, right_edge));
        fn->inputs.push_back(save(o, left_edge));
        attach(out, std::move(fn));
    }
    return out;
}

Tensor Tensor::div(const Tensor &o) const { return binary_op(TRS_DIV, o); }

Tensor Tensor::add_scalar(float s) const {
    Tensor out = scalar_op(TRS_S_ADD, s);
    record_transform(*this, out, GradKind::Identity, Node::Add);
    return out;
}

Tensor Tensor::sub_scalar(float s) const {
    Tensor out = scalar_op(TRS_S_SUB, s);
    record_transform(*this, out, GradKind::Identity, Node::Subtract);
    return out;
}

// mul_scalar (src/tensor.rs:2274-2286).
Tensor Tensor::mul_scalar(float s) const {
    Tensor out = scalar_op(TRS_S_MUL, s);
    if (records(*this)) {
        auto fn = std::make_unique<GradFn>();
        fn->kind = GradKind::MultiplyScalar;
        fn->node = Node::Multiply;
        fn->scalar = s;
        fn->scalar_live = autograd != nullptr;
        fn->inputs.push_back(save(*this, false));
        attach(out, std::move(fn));
    }
    return out;
}

Tensor Tensor::div_scalar(float s) const { return scalar_op(TRS_S_DIV, s); }

Tensor Tensor::scalar_sub(float s) const {
    Tensor out = scalar_op(TRS_S_RSUB, s);
    if (records(*this)) {
        auto fn = std::make_unique<GradFn>();
        fn->kind = GradKind::Negate;
        fn->node = Node::ReflectedSubtract;
        fn->inputs.push_back(save(*this, false));
        attach(out, std::move(fn));
    }
    return out;
}

Tensor Tensor::scalar_div(float s) const { return scalar_op(TRS_S_RDIV, s); }

Tensor Tensor::neg() const {
    Tensor out = unary_op(TRS_NEG);
    if (records(*this)) {
        auto fn = std::make_unique<GradFn>();
        fn->kind = GradKind::Negate;
        fn->node = Node::Negate;
        fn->inputs.push_back(save(*this, false));
        attach(out, std::move(fn));
    }
    return out;
}

// relu (src/tensor.rs:2378-2381): saves its input values.
Tensor Tensor::relu() const {
    Tensor out = unary_op(TRS_RELU);
    if (records(*this)) {
        auto fn = std::make_unique<GradFn>();
        fn->kind = GradKind::Relu;
        fn->node = Node::Relu;
        fn->inputs.push_back(save(*this, true));
        attach(out, std::move(fn));
    }
    return out;
}

// exp (src/tensor.rs:2398-2400) records nothing in the reference; on the
// device it records dx = up * exp(x), saving its own output.
Tensor Tensor::exp() const {
    Tensor out = unary_op(TRS_EXP);
    if (records(*this)) {
        auto fn = std::make_unique<GradFn>();
        fn->kind = GradKind::Exp;
        fn->node = Node::Exp;
        fn->inputs.push_back(save(*this, false));
        fn->output = save(out, true);
        fn->output.autograd.reset();
        attach(out, std::move(fn));
    }
    return out;
}

// sum (src/tensor.rs:2413-2431): a rank-0 result.
Tensor Tensor::sum() const {
    require_cuda("sum");
    Tensor out = empty_like_layout(device(), {}, {});
    const trs_layout la = abi_layout();
    check(trs_sum_f32(numel ? storage->dptr : nullptr, &la, out.storage->dptr));
    if (records(*this)) {
        auto fn = std::make_unique<GradFn>();
        fn->kind = GradKind::Sum;
        fn->node = Node::Sum;
        fn->inputs.push_back(save(*this, false));
        attach(out, std::move(fn));
    }
    return out;
}

// matmul (src/tensor.rs:2453-2533) for rank-2 operands, plus equal-batch
// rank-3 operands; on the device it records dA = dC @ B^T, dB = A^T @ dC.
// matmul (src/tensor.rs:2453-2533): shapes are validated first, with the
// reference's messages (src/tensor_error.rs:120, 243), then the device.
// Device tensors also take two rank-3 operands with equal batch (bmm).
Tensor Tensor::matmul(const Tensor &o) const {
    const size_t r = shape.size();
    const bool batched_ok = device().is_cuda() && o.device().is_cuda();
    if (r != o.shape.size() || (r != 2 && !(r == 3 && batched_ok)))
        throw TensorError("matmul currently requires two rank-2 tensors, got " + dims_str(shape) + " and " +
                          dims_str(o.shape));
    if (r == 3 && shape[0] != o.shape[0])
        throw TensorError("matmul batch sizes differ for " + dims_str(shape) + " and " + dims_str(o.shape));
    if (shape[r - 1] != o.shape[r - 2]) {
        if (r == 2)
            throw TensorError("mat1 and mat2 shapes cannot be multiplied (" + std::to_string(shape[0]) + "x" +
                              std::to_string(shape[1]) + " and " + std::to_string(o.shape[0]) + "x" +
                              std::to_string(o.shape[1]) + ")");
        throw TensorError("matmul inner dimensions differ for " + dims_str(shape) + " and " + dims_str(o.shape));
    }
    require_cuda("matmul");
    if (!(o.device() == device()))
        throw TensorError("Expected all tensors to be on the same device, but found at least two devices, " +
                          device().str() + " and " + o.device().str() + "!");
    Dims oshape = shape;
    oshape[r - 1] = o.shape[r - 1];
    Tensor out = empty_like_layout(device(), oshape, layout::contiguous_strides(oshape));
    if (out.numel > 0) {
        const trs_layout la = abi_layout(), lb = o.abi_layout(), lc = out.abi_layout();
        check(trs_matmul_f32(storage->dptr, &la, o.storage->dptr, &lb, out.storage->dptr, &lc));
    }
    if ((requires_grad() || o.requires_grad()) && is_grad_enabled()) {
        auto fn = std::make_unique<GradFn>();
        fn->kind = GradKind::Matmul;
        fn->node = r == 2 ? Node::Mm : Node::Bmm;
        fn->inputs.push_back(save(*this, o.autograd != nullptr));
        fn->inputs.push_back(save(o, autograd != nullptr));
        attach(out, std::move(fn));
    }
    return out;
}

// Dropout-apply with a uint8 keep-mask: (h * mask) * scale, recorded as the
// reference composition mul then mul_scalar (src/tensor.rs:2217, 2274) would
// be, but with the mask kept as one byte per element in HBM.
Tensor mask_apply(const Tensor &h, const BytePtr &maskp, float scale) {
    h.require_cuda("dropout");
    const ByteBuffer &mask = *maskp;
    if (!(mask.device == h.device())) throw TensorError("dropout mask is on another device");
    if (mask.numel != h.numel || mask.shape != h.shape)
        throw TensorError("dropout mask shape " + dims_str(mask.shape) + " does not match " + dims_str(h.shape));
    Tensor out = empty_like_layout(h.device(), h.shape, layout::unary_output_strides(h.shape, h.strides, h.numel));
    if (h.numel > 0) {
        const trs_layout lh = h.abi_layout(), lo = out.abi_layout();
        const trs_layout lm = abi_layout_of(mask.shape, layout::contiguous_strides(mask.shape), 0);
        check(trs_mask_apply_f32(h.storage->dptr, &lh, mask.dptr, &lm, scale, out.storage->dptr, &lo));
    }
    if (records(h)) {
        auto fn = std::make_unique<GradFn>();
        fn->kind = GradKind::MaskApply;
        fn->node = Node::Multiply;
        fn->scalar = scale;
        fn->mask = maskp;
        fn->inputs.push_back(save(h, false));
        attach(out, std::move(fn));
    }
    return out;
}

float Tensor::item() const {
    if (numel != 1)
        throw TensorError("a Tensor with " + std::to_string(numel) + " elements cannot be converted to Scalar");
    return to_host()[0];
}

// ---- autograd (src/tensor.rs:2881-3341) --------------------------------------------

namespace {

using GradKey = std::pair<const AutogradMeta *, int64_t>;

struct Grad {
    StoragePtr st;  // contiguous logical-order values of the node's output
    Dims shape;
};


Grad new_grad(Device dev, const Dims &shape) {
    Grad g;
    g.shape = shape;
    g.st = Storage::allocate(dev, layout::numel_of(shape));
    return g;
}

// add_gradient (src/tensor.rs:3302-3317): the first contribution is stored,
// later ones are added elementwise.
void add_gradient(std::map<GradKey, Grad> &grads, const MetaPtr &meta, int64_t nr, Grad g) {
    const GradKey key{meta.get(), nr};
    auto it = grads.find(key);
    if (it == grads.end()) {
        grads.emplace(key, std::move(g));
        return;
    }
    const int64_t n = layout::numel_of(g.shape);
    if (n > 0) check(trs_accumulate_f32(it->second.st->dptr, g.st->dptr, (size_t)n));
}

trs_layout saved_layout(const SavedTensor &s) { return abi_layout_of(s.shape, s.strides, s.offset); }

const char *kGraphFreed =
    "Trying to backward through the graph a second time (or directly access saved tensors after they have already "
    "been freed). Saved intermediate values of the graph are freed when you call .backward() or autograd.grad(). "
    "Specify retain_graph=True if you need to backward through the graph a second time or if you need to access "
    "saved tensors after calling backward.";

// validate_saved_values (src/tensor.rs:134-156).
void validate(const GradFn &fn) {
    switch (fn.kind) {
    case GradKind::Multiply:
    case GradKind::Matmul: {
        const SavedTensor &l = fn.inputs[0], &r = fn.inputs[1];
        if ((l.autograd && !r.values) || (r.autograd && !l.values)) throw TensorError(kGraphFreed);
        break;
    }
    case GradKind::MultiplyScalar:
        if (fn.inputs[0].autograd && !fn.scalar_live) throw TensorError(kGraphFreed);
        break;
    case GradKind::Relu:
        if (!fn.inputs[0].values) throw TensorError(kGraphFreed);
        break;
    case GradKind::Exp:
        if (!fn.output.values) throw TensorError(kGraphFreed);
        break;
    case GradKind::MaskApply:
        if (!fn.mask) throw TensorError(kGraphFreed);
        break;
    case GradKind::Fused:
        for (int a : fn.fused.args) {
            if (a < 0) continue;
            const bool bytes = (size_t)a < fn.fused_bytes.size() && fn.fused_bytes[a];
            if (!bytes && !fn.inputs[a].values) throw TensorError(kGraphFreed);
        }
        break;
    default:
        break;
    }
}

// consume_saved_values (src/tensor.rs:158-174).
void consume(GradFn &fn) {
    validate(fn);
    switch (fn.kind) {
    case GradKind::Multiply:
    case GradKind::Matmul:
        fn.inputs[0].values.reset();
        fn.inputs[1].values.reset();
        break;
    case GradKind::MultiplyScalar: fn.scalar_live = false; break;
    case GradKind::Relu: fn.inputs[0].values.reset(); break;
    case GradKind::Exp: fn.output.values.reset(); break;
    case GradKind::MaskApply: fn.mask.reset(); break;
    case GradKind::Fused:
        for (auto &in : fn.inputs) in.values.reset();
        for (auto &b : fn.fused_bytes) b.reset();
        break;
    default: break;
    }
}

// Gradient of one node given its upstream (contiguous, node-output order).
// The caller hands `up` over: a VJP that passes the upstream through
// unchanged gives its storage to the input instead of copying it.  `keep`
// holds the storage until every kernel that reads it has been queued, so a
// merge in add_gradient cannot return the block to the cache early.
void apply_grad_fn(const GradFn &fn, Grad up, Device dev, std::map<GradKey, Grad> &grads) {
    const StoragePtr keep = up.st;
    const trs_layout lup = abi_layout_of(up.shape, layout::contiguous_strides(up.shape), 0);
    const int64_t nup = layout::numel_of(up.shape);
    switch (fn.kind) {
    case GradKind::Sum: {  // fill(up[0]) (src/tensor.rs:3008-3013)
        const SavedTensor &in = fn.inputs[0];
        if (!in.autograd) return;
        Grad g = new_grad(dev, in.shape);
        check(trs_fill_from_device_f32(g.st->dptr, (size_t)in.numel, up.st->dptr));
        add_gradient(grads, in.autograd, in.output_nr, std::move(g));
        return;
    }
    case GradKind::MultiplyScalar: {  // up * s (src/tensor.rs:3014-3021)
        const SavedTensor &in = fn.inputs[0];
        if (!in.autograd) return;
        Grad g = new_grad(dev, in.shape);
        const trs_layout lg = abi_layout_of(in.shape, layout::contiguous_strides(in.shape), 0);
        const trs_layout lu = abi_layout_of(in.shape, layout::contiguous_strides(in.shape), 0);
        if (in.numel) check(trs_binary_scalar_f32(TRS_S_MUL, up.st->dptr, &lu, fn.scalar, g.st->dptr, &lg));
        add_gradient(grads, in.autograd, in.output_nr, std::move(g));
        return;
    }
    case GradKind::Negate: {  // sign flip (src/tensor.rs:3022-3030)
        const SavedTensor &in = fn.inputs[0];
        if (!in.autograd) return;
        Grad g = new_grad(dev, in.shape);
        const trs_layout lg = abi_layout_of(in.shape, layout::contiguous_strides(in.shape), 0);
        if (in.numel) check(trs_unary_f32(TRS_NEG, up.st->dptr, &lg, g.st->dptr, &lg));
        add_gradient(grads, in.autograd, in.output_nr, std::move(g));
        return;
    }
    case GradKind::Relu: {  // apply_relu_vjp (src/tensor.rs:3161-3176)
        const SavedTensor &in = fn.inputs[0];
        if (!in.autograd) return;
        Grad g = new_grad(dev, in.shape);
        const trs_layout li = saved_layout(in);
        if (in.numel) check(trs_relu_backward_f32(in.values->dptr, &li, up.st->dptr, g.st->dptr));
        add_gradient(grads, in.autograd, in.output_nr, std::move(g));
        return;
    }
    case GradKind::Exp: {  // dx = up * exp(x)
        const SavedTensor &in = fn.inputs[0];
        if (!in.autograd) return;
        Grad g = new_grad(dev, in.shape);
        const trs_layout lo = saved_layout(fn.output);
        const trs_layout lg = abi_layout_of(in.shape, layout::contiguous_strides(in.shape), 0);
        if (in.numel) check(trs_binary_f32(TRS_MUL, up.st->dptr, &lg, fn.output.values->dptr, &lo, g.st->dptr, &lg));
        add_gradient(grads, in.autograd, in.output_nr, std::move(g));
        return;
    }
    case GradKind::Fused: {  // every input gradient in one kernel over the output shape, then unbroadcast
        const FusedBackward &bwd = fn.fused;
        std::vector<const void *> ptrs;
        std::vector<trs_layout> lays;
        for (int a : bwd.args) {
            if (a < 0) {
                ptrs.push_back(up.st->dptr);
                lays.push_back(lup);
            } else {
                const SavedTensor &sv = fn.inputs[a];
                const bool bytes = (size_t)a < fn.fused_bytes.size() && fn.fused_bytes[a];
                ptrs.push_back(bytes ? (const void *)fn.fused_bytes[a]->dptr : (const void *)sv.values->dptr);
                lays.push_back(saved_layout(sv));
            }
        }
        std::vector<std::shared_ptr<Storage>> full;
        std::vector<float *> outs;
        for (size_t o = 0; o < bwd.targets.size(); o++) {
            full.push_back(new_grad(dev, up.shape).st);
            outs.push_back(full.back()->dptr);
        }
        if (layout::numel_of(up.shape) > 0)
            check(trs_fusion_launch_multi(bwd.program, (int)ptrs.size(), ptrs.data(), lays.data(), (int)outs.size(),
                                          outs.data(), &lup));
        for (size_t o = 0; o < bwd.targets.size(); o++) {
            const SavedTensor &in = fn.inputs[bwd.targets[o]];
            if (!in.autograd) continue;
            if (in.shape == up.shape) {
                add_gradient(grads, in.autograd, in.output_nr, Grad{full[o], up.shape});
                continue;
            }
            // A broadcast input: the reference's accumulation (from +0.0 in
            // output row-major order), as the eager VJPs reduce.
            Grad g = new_grad(dev, in.shape);
            const trs_layout lin = abi_layout_of(in.shape, layout::contiguous_strides(in.shape), 0);
            check(trs_reduce_to_shape_f32(full[o]->dptr, &lup, &lin, g.st->dptr));
            add_gradient(grads, in.autograd, in.output_nr, std::move(g));
        }
        return;
    }
    case GradKind::MaskApply: {  // (up * scale) * mask: the reverse of mul then mul_scalar
        const SavedTensor &in = fn.inputs[0];
        if (!in.autograd) return;
        Grad g = new_grad(dev, in.shape);
        const trs_layout lg = abi_layout_of(in.shape, layout::contiguous_strides(in.shape), 0);
        if (in.numel) check(trs_mask_backward_f32(up.st->dptr, &lg, fn.mask->dptr, &lg, fn.scalar, g.st->dptr, &lg));
        add_gradient(grads, in.autograd, in.output_nr, std::move(g));
        return;
    }
    case GradKind::Multiply: {  // src/tensor.rs:3031-3097
        const SavedTensor &l = fn.inputs[0], &r = fn.inputs[1];
        for (int side = 0; side < 2; side++) {
            const SavedTensor &self = side ? r : l, &other = side ? l : r;
            if (!self.autograd) continue;
            Grad g = new_grad(dev, self.shape);
            const trs_layout lo = saved_layout(other);
            const trs_layout ls = abi_layout_of(self.shape, layout::contiguous_strides(self.shape), 0);
            if (self.numel) check(trs_mul_backward_f32(up.st->dptr, &lup, other.values->dptr, &lo, &ls, g.st->dptr));
            add_gradient(grads, self.autograd, self.output_nr, std::move(g));
        }
        return;
    }
    case GradKind::AddTensor:
    case GradKind::SubTensor: {  // db = sum over broadcast dims of up
        bool up_given = false;
        for (int side = 0; side < 2; side++) {
            const SavedTensor &self = fn.inputs[side];
            if (!self.autograd) continue;
            const bool negate = side == 1 && fn.kind == GradKind::SubTensor;
            if (!negate && !up_given && self.numel == nup) {
                // Not broadcast: the gradient is the upstream itself.
                add_gradient(grads, self.autograd, self.output_nr, Grad{up.st, self.shape});
                up_given = true;
                continue;
            }
            Grad g = new_grad(dev, self.shape);
            const trs_layout ls = abi_layout_of(self.shape, layout::contiguous_strides(self.shape), 0);
            if (self.numel) {
                check(trs_reduce_to_shape_f32(up.st->dptr, &lup, &ls, g.st->dptr));
                if (side == 1 && fn.kind == GradKind::SubTensor)
                    check(trs_unary_f32(TRS_NEG, g.st->dptr, &ls, g.st->dptr, &ls));
            }
            add_gradient(grads, self.autograd, self.output_nr, std::move(g));
        }
        return;
    }
    case GradKind::Matmul: {  // dA = dC @ B^T, dB = A^T @ dC
        const SavedTensor &a = fn.inputs[0], &b = fn.inputs[1];
        const size_t rk = a.shape.size();
        auto transposed = [&](const SavedTensor &s) {
            trs_layout t = saved_layout(s);
            std::swap(t.shape[rk - 2], t.shape[rk - 1]);
            std::swap(t.stride[rk - 2], t.stride[rk - 1]);
            return t;
        };
        if (a.autograd) {
            Grad g = new_grad(dev, a.shape);
            const trs_layout lbt = transposed(b);
            const trs_layout lg = abi_layout_of(a.shape, layout::contiguous_strides(a.shape), 0);
            if (a.numel) check(trs_matmul_f32(up.st->dptr, &lup, b.values->dptr, &lbt, g.st->dptr, &lg));
            add_gradient(grads, a.autograd, a.output_nr, std::move(g));
        }
        if (b.autograd) {
            Grad g = new_grad(dev, b.shape);
            const trs_layout lat = transposed(a);
            const trs_layout lg = abi_layout_of(b.shape, layout::contiguous_strides(b.shape), 0);
            if (b.numel) check(trs_matmul_f32(a.values->dptr, &lat, up.st->dptr, &lup, g.st->dptr, &lg));
            add_gradient(grads, b.autograd, b.output_nr, std::move(g));
        }
        return;
    }
    case GradKind::Transfer:
        throw TensorError("backward through a device transfer is not supported: create the leaf tensor on the device "
                          "(device=\"cuda\") so its gradient stays in HBM");
    case GradKind::Identity: {  // TransformMapping::Identity: the same values in logical order
        const SavedTensor &in = fn.inputs[0];
        if (!in.autograd) return;
        add_gradient(grads, in.autograd, in.output_nr, Grad{up.st, in.shape});
        return;
    }
    case GradKind::Permute: {  // transform_backward Permute (src/tensor.rs:3246-3298)
        const SavedTensor &in = fn.inputs[0];
        if (!in.autograd) return;
        Grad g = new_grad(dev, in.shape);
        // up is contiguous over the permuted shape; read it as the input's
        // shape: input axis dims[p] has the stride of output axis p.
        const Dims ust = layout::contiguous_strides(up.shape);
        Dims rs(in.shape.size(), 0);
        for (size_t p = 0; p < fn.dims.size(); p++) rs[fn.dims[p]] = ust[p];
        const trs_layout lu = abi_layout_of(in.shape, rs, 0);
        const trs_layout lg = abi_layout_of(in.shape, layout::contiguous_strides(in.shape), 0);
        if (in.numel) check(trs_unary_f32(TRS_COPY, up.st->dptr, &lu, g.st->dptr, &lg));
        add_gradient(grads, in.autograd, in.output_nr, std::move(g));
        return;
    }
    case GradKind::Index: {  // TransformMapping::Index (src/tensor.rs:3237-3245)
        const SavedTensor &in = fn.inputs[0];
        if (!in.autograd) return;
        Grad g = new_grad(dev, in.shape);
        if (in.numel) check(trs_memset_zero(g.st->dptr, (size_t)in.numel * sizeof(float)));
        if (nup)
            check(trs_memcpy_d2d(g.st->dptr + fn.index_start, up.st->dptr, (size_t)nup * sizeof(float)));
        add_gradient(grads, in.autograd, in.output_nr, std::move(g));
        return;
    }
    }
}

struct TopoEntry {
    MetaPtr meta;
    GradFn *fn;  // null for leaves
};

// collect_topology (src/tensor.rs:2945-2994): iterative DFS, post-order,
// right operand pushed first so the left subtree is visited first.
std::vector<TopoEntry> collect_topology(const MetaPtr &root) {
    std::vector<TopoEntry> topo;
    std::map<const AutogradMeta *, bool> seen;
    struct Frame {
        MetaPtr meta;
        bool exit;
    };
    std::vector<Frame> stack{{root, false}};
    while (!stack.empty()) {
        Frame f = std::move(stack.back());
        stack.pop_back();
        if (f.exit) {
            topo.push_back({f.meta, f.meta->leaf ? nullptr : f.meta->fn.get()});
            continue;
        }
        if (seen.count(f.meta.get())) continue;
        seen[f.meta.get()] = true;
        if (!f.meta->leaf) {
            if (!f.meta->fn) throw TensorError(kGraphFreed);
            validate(*f.meta->fn);
        }
        stack.push_back({f.meta, true});
        if (!f.meta->leaf) {
            const auto &ins = f.meta->fn->inputs;
            for (auto it = ins.rbegin(); it != ins.rend(); ++it)
                if (it->autograd) stack.push_back({it->autograd, false});
        }
    }
    return topo;
}

}  // namespace

// Tensor::backward and run_backward (src/tensor.rs:884-898, 2881-2938).
void Tensor::backward() const {
    if (!requires_grad() || !autograd)
        throw TensorError("element 0 of tensors does not require grad and does not have a grad_fn");
    if (numel != 1) throw TensorError("grad can be implicitly created only for scalar outputs");
    require_cuda("backward");
    std::lock_guard<std::mutex> lock(g_backward_mu);
    const Device dev = device();
    std::vector<TopoEntry> topo = collect_topology(autograd);
    std::map<GradKey, Grad> grads;
    {
        Grad seed = new_grad(dev, shape);
        check(trs_fill_f32(seed.st->dptr, 1, 1.0f));
        grads.emplace(GradKey{autograd.get(), output_nr}, std::move(seed));
    }
    std::vector<std::pair<MetaPtr, Grad>> leaf_grads;
    for (auto it = topo.rbegin(); it != topo.rend(); ++it) {
        auto g = grads.find(GradKey{it->meta.get(), 0});
        if (g == grads.end()) continue;
        Grad up = std::move(g->second);
        grads.erase(g);
        if (!it->fn) {
            leaf_grads.emplace_back(it->meta, std::move(up));
            continue;
        }
        apply_grad_fn(*it->fn, std::move(up), dev, grads);
    }
    // Free value-dependent saved state only after every gradient succeeded.
    for (auto &e : topo)
        if (e.fn) consume(*e.fn);
    // accumulate_leaf_gradient (src/tensor.rs:3319-3341).
    for (auto &lg : leaf_grads) {
        AutogradMeta &m = *lg.first;
        std::lock_guard<std::mutex> gl(m.grad_mu);
        const int64_t n = layout::numel_of(lg.second.shape);
        if (m.grad) {
            if (n) check(trs_accumulate_f32(m.grad->dptr, lg.second.st->dptr, (size_t)n));
        } else {
            m.grad = lg.second.st;
            m.grad->shared_gradient = true;
        }
    }
}

bool Tensor::has_grad() const {
    if (!autograd || !autograd->leaf) return false;
    std::lock_guard<std::mutex> gl(autograd->grad_mu);
    return autograd->grad != nullptr;
}

// Tensor::grad (src/tensor.rs:808-832): a detached contiguous copy.
Tensor Tensor::grad() const {
    if (!autograd || !autograd->leaf) throw TensorError("tensor has no gradient");
    std::lock_guard<std::mutex> gl(autograd->grad_mu);
    if (!autograd->grad) throw TensorError("tensor has no gradient");
    const Dims &shp = autograd->leaf_shape;
    const int64_t n = layout::numel_of(shp);
    Tensor out = make_tensor(Storage::allocate(autograd->grad->device, n), shp, layout::contiguous_strides(shp), 0);
    if (n) {
        select_device(autograd->grad->device);
        check(trs_memcpy_d2d(out.storage->dptr, autograd->grad->dptr, (size_t)n * sizeof(float)));
    }
    return out;
}

// Tensor::live_grad (src/tensor.rs:835-861): the leaf's gradient storage
// itself, contiguous, with no graph history.  Later backward passes
// accumulate into that storage in place, so the alias sees them.
Tensor Tensor::live_grad() const {
    if (!autograd || !autograd->leaf) throw TensorError("tensor has no gradient");
    std::lock_guard<std::mutex> gl(autograd->grad_mu);
    if (!autograd->grad) throw TensorError("tensor has no gradient");
    const Dims &shp = autograd->leaf_shape;
    return make_tensor(autograd->grad, shp, layout::contiguous_strides(shp), 0);
}

// ---- byte buffers (dropout masks) ----------------------------------------------------

ByteBuffer::~ByteBuffer() {
    if (dptr) {
        select_device_quietly(device);
        (void)trs_free(dptr);
    }
}

std::shared_ptr<ByteBuffer> ByteBuffer::from_host(const uint8_t *data, const Dims &shape, Device device) {
    if (!device.is_cuda()) throw TensorError("byte buffers live on the device");
    select_device(device);
    auto b = std::make_shared<ByteBuffer>();
    b->device = device;
    b->shape = shape;
    b->numel = layout::numel_of(shape);
    if (b->numel > 0) {
        void *p = nullptr;
        int rc = trs_alloc((size_t)b->numel, &p);
        if (rc != TRS_OK) throw TensorError("failed to allocate storage for " + std::to_string(b->numel) + " elements");
        b->dptr = (uint8_t *)p;
        check(trs_memcpy_h2d(b->dptr, data, (size_t)b->numel));
    }
    return b;
}

// ---- fusion ------------------------------------------------------------------------------

FusedProgram FusedProgram::compile(const std::string &ir, int nin) {
    FusedProgram p;
    check(trs_fusion_compile(ir.data(), ir.size(), &p.id));
    p.nin = nin;
    return p;
}

namespace {

Device fused_arg_device(const FusedArg &a) { return a.bytes ? a.bytes->device : a.tensor.device(); }

trs_layout fused_arg_layout(const FusedArg &a) {
    if (!a.bytes) return a.tensor.abi_layout();
    return abi_layout_of(a.bytes->shape, layout::contiguous_strides(a.bytes->shape), 0);
}

const void *fused_arg_ptr(const FusedArg &a) {
    return a.bytes ? (const void *)a.bytes->dptr : (const void *)a.tensor.storage->dptr;
}

}  // namespace

Tensor FusedProgram::launch(const std::vector<FusedArg> &inputs, const Dims &out_shape, const Dims &out_strides) const {
    if ((int)inputs.size() != nin)
        throw TensorError("fused program takes " + std::to_string(nin) + " inputs, got " + std::to_string(inputs.size()));
    if (inputs.empty()) throw TensorError("fused program has no inputs");
    const Device dev = fused_arg_device(inputs[0]);
    for (auto &a : inputs) {
        if (a.bytes) {
            if (!a.bytes->device.is_cuda()) throw TensorError("fused program: byte buffer is not on a device");
        } else {
            a.tensor.require_cuda("fused program");
        }
        if (!(fused_arg_device(a) == dev)) throw TensorError("fused program inputs are on different devices");
    }
    Tensor out = empty_like_layout(dev, out_shape, out_strides);
    if (out.numel == 0) return out;
    std::vector<trs_layout> lays;
    std::vector<const void *> ptrs;
    for (auto &a : inputs) {
        lays.push_back(fused_arg_layout(a));
        ptrs.push_back(fused_arg_ptr(a));
    }
    const trs_layout lo = out.abi_layout();
    check(trs_fusion_launch(id, nin, ptrs.data(), lays.data(), out.storage->dptr, &lo));
    return out;
}

Tensor FusedProgram::launch_with_grad(const std::vector<FusedArg> &inputs, const Dims &out_shape,
                                      const Dims &out_strides, const FusedBackward &bwd) const {
    for (int a : bwd.args)
        if (a < -1 || a >= (int)inputs.size()) throw TensorError("fused gradient program argument out of range");
    std::vector<bool> seen(inputs.size(), false);
    for (int t : bwd.targets) {
        if (t < 0 || t >= (int)inputs.size() || seen[t] || inputs[t].bytes)
            throw TensorError("fused gradient program target invalid");
        seen[t] = true;
    }
    int nout = 0;
    check(trs_fusion_outputs(bwd.program, &nout));
    if (nout != (int)bwd.targets.size())
        throw TensorError("fused gradient program has " + std::to_string(nout) + " outputs for " +
                          std::to_string(bwd.targets.size()) + " targets");
    Tensor out = launch(inputs, out_shape, out_strides);
    bool any = false;
    for (int t : bwd.targets) any = any || inputs[t].tensor.requires_grad();
    if (!any || !is_grad_enabled()) return out;
    auto fn = std::make_unique<GradFn>();
    fn->kind = GradKind::Fused;
    fn->node = Node::Fused;
    for (const auto &a : inputs) {
        if (a.bytes) {
            SavedTensor sv;
            sv.shape = a.bytes->shape;
            sv.strides = layout::contiguous_strides(a.bytes->shape);
            sv.numel = a.bytes->numel;
            fn->inputs.push_back(sv);
        } else {
            fn->inputs.push_back(save(a.tensor, true));
        }
        fn->fused_bytes.push_back(a.bytes);
    }
    fn->fused = bwd;
    attach(out, std::move(fn));
    return out;
}

}  // namespace trs_engine
