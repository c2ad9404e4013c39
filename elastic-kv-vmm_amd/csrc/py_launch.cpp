// Python-facing launch helpers for the kernel entry points of the library:
// the resident lookup (ekv_resolve_resident*), the row gather
// (ekv_gather_rows), the plane gather / scatter / move (ekv_gather_kv,
// ekv_scatter_kv, ekv_move_kv), the batch-token swap-in (ekv_swap_in*), the
// per-layer SGLang-convention swap-in (ekv_hisparse_swap_in) and the one-call
// decode step (ekv_decode_step). Their GPU work can be a few microseconds at
// small shapes, so
// describing the tensors for the C ABI from Python (attribute reads and
// struct packing, about 1 us per tensor) set the call rate. Here the
// descriptors are read straight from the tensors, the device and stream come
// from torch's current HIP stream, and the entry point, passed in by address
// from the loaded libelastic_vmm.so, is called with the GIL released.
// Validation of shapes and types stays in the entry points; this file only
// builds descriptors, with the same device and dtype errors as the ctypes
// path (elastic_kv/_native.py).
#include <Python.h>

#include <c10/hip/HIPFunctions.h>
#include <c10/hip/HIPStream.h>
#include <torch/csrc/autograd/python_variable.h>

#include "../../include/ekv_kernels.h"

#include <set>
#include <string>

#ifndef EKV_SOURCE_HASH
#define EKV_SOURCE_HASH unknown
#endif
#define EKV_STRINGIFY_(x) #x
#define EKV_STRINGIFY(x) EKV_STRINGIFY_(x)

namespace {

int dtype_code(c10::ScalarType type) {
    switch (type) {
        case c10::ScalarType::Int: return EKV_INT32;
        case c10::ScalarType::Long: return EKV_INT64;
        case c10::ScalarType::Byte: return EKV_UINT8;
        case c10::ScalarType::Char: return EKV_INT8;
        case c10::ScalarType::Short: return EKV_INT16;
        case c10::ScalarType::BFloat16: return EKV_BFLOAT16;
        case c10::ScalarType::Half: return EKV_FLOAT16;
        case c10::ScalarType::Float: return EKV_FLOAT32;
        default: return 0;
    }
}

// One optional tensor argument: its Python object, name and descriptor.
struct Arg {
    PyObject* object;
    const char* name;
    bool described = true;   // false: only its device is checked (a K/V row buffer of any dtype)
    ekv_tensor view{};
    const at::Tensor* tensor = nullptr;
    const ekv_tensor* pointer() const { return object == Py_None ? nullptr : &view; }
};

// Fills every present argument's descriptor; returns the device index, or -1
// with a Python exception set. The device checks run over all arguments
// before any descriptor is built, as elastic_kv._native.device_of does.
template <size_t N>
int describe_all(Arg (&args)[N]) {
    const at::Tensor* tensors[N] = {};
    for (size_t i = 0; i < N; ++i) {
        if (args[i].object == Py_None) {
            continue;
        }
        if (!THPVariable_Check(args[i].object)) {
            PyErr_Format(PyExc_TypeError, "%s must be a tensor", args[i].name);
            return -1;
        }
        tensors[i] = args[i].tensor = &THPVariable_Unpack(args[i].object);
    }
    std::set<std::string> devices;
    c10::Device device(c10::DeviceType::CPU);
    for (size_t i = 0; i < N; ++i) {
        if (tensors[i] != nullptr) {
            device = tensors[i]->device();
            devices.insert(device.str());
        }
    }
    if (devices.size() != 1) {
        std::string listed = "[";
        for (const std::string& one : devices) {
            listed += (listed.size() > 1 ? ", '" : "'") + one + "'";
        }
        PyErr_Format(PyExc_ValueError, "tensors must share one device, got %s]", listed.c_str());
        return -1;
    }
    if (!device.is_cuda()) {
        PyErr_SetString(PyExc_ValueError, "hot-path kernels need GPU tensors (no CPU fallback exists)");
        return -1;
    }
    for (size_t i = 0; i < N; ++i) {
        const at::Tensor* t = tensors[i];
        if (t == nullptr || !args[i].described) {
            continue;
        }
        const int64_t ndim = t->dim();
        if (ndim > 4) {
            PyErr_Format(PyExc_ValueError, "%s has more than 4 dimensions", args[i].name);
            return -1;
        }
        const int code = dtype_code(t->scalar_type());
        if (code == 0) {
            PyErr_Format(PyExc_TypeError, "%s has unsupported dtype %s", args[i].name,
                         c10::toString(t->scalar_type()));
            return -1;
        }
        ekv_tensor& view = args[i].view;
        view.data = t->data_ptr();
        view.dtype = code;
        view.ndim = static_cast<int32_t>(ndim);
        for (int64_t d = 0; d < ndim; ++d) {
            view.shape[d] = t->size(d);
            view.stride[d] = t->stride(d);
        }
    }
    return device.has_index() ? device.index() : c10::hip::current_device();
}

// Makes `device` current for the call and restores the caller's device.
class CurrentDevice {
public:
    explicit CurrentDevice(int device) : previous_(c10::hip::current_device()) {
        if (previous_ != device) {
            c10::hip::set_device(static_cast<c10::DeviceIndex>(device));
        }
        device_ = device;
    }
    ~CurrentDevice() {
        if (previous_ != device_) {
            try {
                c10::hip::set_device(previous_);
            } catch (...) {
                // A destructor must not throw; the launch's own status is what the caller needs.
            }
        }
    }

private:
    c10::DeviceIndex previous_;
    int device_ = 0;
};

bool read_int(PyObject* object, const char* name, int64_t& value) {
    value = PyLong_AsLongLong(object);
    if (value == -1 && PyErr_Occurred()) {
        PyErr_Format(PyExc_TypeError, "%s must be an int", name);
        return false;
    }
    return true;
}

// resolve(form, entry, topk, table, mapping, slot_base, resident_bits,
//         bits_shift, rows, lengths, selected, output, misses, miss_count,
//         block_size) -> status of the entry point
// form 0: ekv_resolve_resident (mapping may be None)
// form 1: ekv_resolve_resident_bits
// form 2: ekv_resolve_resident_local
PyObject* resolve(PyObject*, PyObject* const* argv, Py_ssize_t argc) {
    if (argc != 15) {
        PyErr_SetString(PyExc_TypeError, "resolve takes 15 arguments");
        return nullptr;
    }
    int64_t form = 0, entry = 0, bits_shift = 0, block_size = 0;
    if (!read_int(argv[0], "form", form) || !read_int(argv[1], "entry", entry) ||
        !read_int(argv[7], "bits_shift", bits_shift) || !read_int(argv[14], "block_size", block_size)) {
        return nullptr;
    }
    Arg args[] = {{argv[2], "topk"},      {argv[3], "table"},       {argv[4], "mapping"},
                  {argv[5], "slot_base"}, {argv[6], "bits"},        {argv[8], "rows"},
                  {argv[9], "lengths"},   {argv[10], "selected"},   {argv[11], "output"},
                  {argv[12], "misses"},   {argv[13], "miss_count"}};
    try {
        const int device = describe_all(args);
        if (device < 0) {
            return nullptr;
        }
        CurrentDevice current(device);
        void* stream = c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(device)).stream();
        const ekv_tensor* t[11];
        for (int i = 0; i < 11; ++i) {
            t[i] = args[i].pointer();
        }
        int status = 0;
        Py_BEGIN_ALLOW_THREADS
        if (form == 2) {
            status = reinterpret_cast<decltype(&ekv_resolve_resident_local)>(entry)(
                t[0], t[1], t[3], t[4], bits_shift, t[5], t[6], t[7], t[8], t[9], t[10], block_size, stream);
        } else if (form == 1) {
            status = reinterpret_cast<decltype(&ekv_resolve_resident_bits)>(entry)(
                t[0], t[1], t[4], bits_shift, t[5], t[6], t[7], t[8], t[9], t[10], block_size, stream);
        } else {
            status = reinterpret_cast<decltype(&ekv_resolve_resident)>(entry)(
                t[0], t[1], t[2], t[5], t[6], t[7], t[8], t[9], t[10], block_size, stream);
        }
        Py_END_ALLOW_THREADS
        return PyLong_FromLong(status);
    } catch (const std::exception& error) {
        PyErr_SetString(PyExc_RuntimeError, error.what());
        return nullptr;
    }
}

// gather_rows(entry, raw, positions, request_ids, lengths, request_table,
//             slot_offsets, output, request_stride, sink_elements, indirect)
// -> status of ekv_gather_rows
PyObject* gather_rows(PyObject*, PyObject* const* argv, Py_ssize_t argc) {
    if (argc != 11) {
        PyErr_SetString(PyExc_TypeError, "gather_rows takes 11 arguments");
        return nullptr;
    }
    int64_t entry = 0, request_stride = 0, sink_elements = 0, indirect = 0;
    if (!read_int(argv[0], "entry", entry) || !read_int(argv[8], "request_stride", request_stride) ||
        !read_int(argv[9], "sink_elements", sink_elements) || !read_int(argv[10], "indirect", indirect)) {
        return nullptr;
    }
    Arg args[] = {{argv[1], "raw"},           {argv[2], "positions"},    {argv[3], "request_ids"},
                  {argv[4], "lengths"},       {argv[5], "request_table"}, {argv[6], "slot_offsets"},
                  {argv[7], "output"}};
    try {
        const int device = describe_all(args);
        if (device < 0) {
            return nullptr;
        }
        CurrentDevice current(device);
        void* stream = c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(device)).stream();
        int status = 0;
        Py_BEGIN_ALLOW_THREADS
        status = reinterpret_cast<decltype(&ekv_gather_rows)>(entry)(
            args[0].pointer(), args[1].pointer(), args[2].pointer(), args[3].pointer(), args[4].pointer(),
            args[5].pointer(), args[6].pointer(), request_stride, sink_elements, indirect ? 1 : 0, stream);
        Py_END_ALLOW_THREADS
        return PyLong_FromLong(status);
    } catch (const std::exception& error) {
        PyErr_SetString(PyExc_RuntimeError, error.what());
        return nullptr;
    }
}

// Row layout of a K/V tensor pair (adaptive_sparse.hisparse_swap._row_layout):
// row bytes, row stride and K -> V offset in bytes, rows. False with a Python
// exception set.
bool row_layout(const at::Tensor& first, const at::Tensor& second, const char* name, ekv_planes& planes) {
    if (first.sizes() != second.sizes() || first.scalar_type() != second.scalar_type() ||
        first.strides() != second.strides()) {
        PyErr_Format(PyExc_ValueError, "%s K and V must share shape, dtype and strides", name);
        return false;
    }
    if (first.dim() < 1 || first.size(0) == 0) {
        PyErr_Format(PyExc_ValueError, "%s needs at least one row", name);
        return false;
    }
    const int64_t item = static_cast<int64_t>(first.element_size());
    int64_t expect = 1;
    for (int64_t d = first.dim() - 1; d >= 1; --d) {
        if (first.size(d) > 1 && first.stride(d) != expect) {
            PyErr_Format(PyExc_ValueError, "%s rows must be contiguous", name);
            return false;
        }
        expect *= first.size(d);
    }
    planes.layers = 1;
    planes.kv = 2;
    planes.layer_stride = 0;
    planes.kv_stride = static_cast<int64_t>(reinterpret_cast<uintptr_t>(second.data_ptr()) -
                                            reinterpret_cast<uintptr_t>(first.data_ptr()));
    planes.row_stride = first.stride(0) * item;
    planes.row_bytes = expect * item;
    planes.rows = first.size(0);
    return true;
}

// hisparse(entry, pointer_entry, top_k_blocks, device_buffer_tokens,
//          host_cache_locs, device_buffer_locs, host_cache_k, host_cache_v,
//          device_buffer_k, device_buffer_v, top_k_device_locs,
//          req_pool_indices, seq_lens, lru_slots, item_size_bytes,
//          hot_buffer_size, sparse_block_size, num_real_reqs)
// -> status of ekv_hisparse_swap_in (or of ekv_host_device_pointer)
// The checks and their order are those of
// adaptive_sparse.hisparse_swap.load_blocks_to_device_buffer_mha.
PyObject* hisparse(PyObject*, PyObject* const* argv, Py_ssize_t argc) {
    if (argc != 18) {
        PyErr_SetString(PyExc_TypeError, "hisparse takes 18 arguments");
        return nullptr;
    }
    int64_t entry = 0, pointer_entry = 0, item_size = 0, hot = 0, block_size = 0;
    if (!read_int(argv[0], "entry", entry) || !read_int(argv[1], "pointer_entry", pointer_entry) ||
        !read_int(argv[14], "item_size_bytes", item_size) || !read_int(argv[15], "hot_buffer_size", hot) ||
        !read_int(argv[16], "sparse_block_size", block_size)) {
        return nullptr;
    }
    Arg args[] = {{argv[2], "top_k_blocks"},        {argv[3], "device_buffer_tokens"},
                  {argv[4], "host_cache_locs"},     {argv[5], "device_buffer_locs"},
                  {argv[10], "top_k_device_locs"},  {argv[11], "req_pool_indices"},
                  {argv[12], "seq_lens"},           {argv[13], "lru_slots"},
                  {argv[17], "num_real_reqs"},      {argv[8], "device_buffer_k", false},
                  {argv[9], "device_buffer_v", false}};
    if (argv[8] == Py_None || argv[9] == Py_None) {
        PyErr_SetString(PyExc_TypeError, "device_buffer_k and device_buffer_v are required");
        return nullptr;
    }
    for (PyObject* host : {argv[6], argv[7]}) {
        if (!THPVariable_Check(host)) {
            PyErr_SetString(PyExc_TypeError, "host_cache_k and host_cache_v must be tensors");
            return nullptr;
        }
    }
    try {
        const int device = describe_all(args);
        if (device < 0) {
            return nullptr;
        }
        const at::Tensor& host_k = THPVariable_Unpack(argv[6]);
        const at::Tensor& host_v = THPVariable_Unpack(argv[7]);
        ekv_planes host{}, dev{};
        if (!row_layout(host_k, host_v, "host cache", host) ||
            !row_layout(*args[9].tensor, *args[10].tensor, "device buffer", dev)) {
            return nullptr;
        }
        if (host.row_bytes != dev.row_bytes || host.row_bytes != item_size) {
            PyErr_Format(PyExc_ValueError, "rows hold %lld (host) and %lld (device) bytes, item_size_bytes is %lld",
                         static_cast<long long>(host.row_bytes), static_cast<long long>(dev.row_bytes),
                         static_cast<long long>(item_size));
            return nullptr;
        }
        for (const at::Tensor* t : {&host_k, &host_v}) {
            if (!t->device().is_cpu() || !t->is_pinned()) {
                PyErr_SetString(PyExc_ValueError, "the host cache must be pinned CPU memory (pin_memory)");
                return nullptr;
            }
        }
        const auto device_pointer = reinterpret_cast<decltype(&ekv_host_device_pointer)>(pointer_entry);
        void* host_k_device = nullptr;
        void* host_v_device = nullptr;
        int status = device_pointer(host_k.data_ptr(), &host_k_device);
        if (status == 0) {
            status = device_pointer(host_v.data_ptr(), &host_v_device);
        }
        if (status != 0) {
            return PyLong_FromLong(status);
        }
        host.base = host_k_device;
        host.kv_stride = static_cast<int64_t>(reinterpret_cast<uintptr_t>(host_v_device) -
                                              reinterpret_cast<uintptr_t>(host_k_device));
        dev.base = args[9].tensor->data_ptr();
        CurrentDevice current(device);
        void* stream = c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(device)).stream();
        Py_BEGIN_ALLOW_THREADS
        status = reinterpret_cast<decltype(&ekv_hisparse_swap_in)>(entry)(
            args[0].pointer(), args[1].pointer(), args[2].pointer(), args[3].pointer(), &host, &dev,
            args[4].pointer(), args[5].pointer(), args[6].pointer(), args[7].pointer(), hot, block_size,
            args[8].pointer(), stream);
        Py_END_ALLOW_THREADS
        return PyLong_FromLong(status);
    } catch (const std::exception& error) {
        PyErr_SetString(PyExc_RuntimeError, error.what());
        return nullptr;
    }
}

// The fields of a KVPlanes object (adaptive_sparse.kv_pool.KVPlanes). False
// with a Python exception set.
bool read_planes(PyObject* object, ekv_planes& planes) {
    static const char* const names[] = {"base", "layers", "kv", "layer_stride", "kv_stride", "row_stride",
                                        "row_bytes", "rows"};
    int64_t values[8];
    for (int i = 0; i < 8; ++i) {
        PyObject* value = PyObject_GetAttrString(object, names[i]);
        if (value == nullptr) {
            return false;
        }
        values[i] = PyLong_AsLongLong(value);
        Py_DECREF(value);
        if (values[i] == -1 && PyErr_Occurred()) {
            return false;
        }
    }
    planes.base = reinterpret_cast<void*>(static_cast<uintptr_t>(values[0]));
    planes.layers = values[1];
    planes.kv = values[2];
    planes.layer_stride = values[3];
    planes.kv_stride = values[4];
    planes.row_stride = values[5];
    planes.row_bytes = values[6];
    planes.rows = values[7];
    return true;
}

// The dense (B, L, KV, K, *row) rows of `tensor` for slots [L, B, K] of
// `planes` (adaptive_sparse.sparse_read._dense_struct). False with a Python
// exception set.
bool dense_rows(const at::Tensor& tensor, const ekv_planes& planes, const at::Tensor& slots, const char* name,
                ekv_kv_rows& rows) {
    if (tensor.dim() < 4) {
        PyErr_Format(PyExc_ValueError, "%s must be shaped (B, L, KV, K, ...)", name);
        return false;
    }
    if (slots.dim() != 3) {
        PyErr_SetString(PyExc_ValueError, "slots must be shaped [L, B, K]");
        return false;
    }
    const int64_t expected[4] = {slots.size(1), slots.size(0), planes.kv, slots.size(2)};
    for (int d = 0; d < 4; ++d) {
        if (tensor.size(d) != expected[d]) {
            PyErr_Format(PyExc_ValueError, "%s leading shape (%lld, %lld, %lld, %lld) != (%lld, %lld, %lld, %lld)",
                         name, static_cast<long long>(tensor.size(0)), static_cast<long long>(tensor.size(1)),
                         static_cast<long long>(tensor.size(2)), static_cast<long long>(tensor.size(3)),
                         static_cast<long long>(expected[0]), static_cast<long long>(expected[1]),
                         static_cast<long long>(expected[2]), static_cast<long long>(expected[3]));
            return false;
        }
    }
    const int64_t item = static_cast<int64_t>(tensor.element_size());
    int64_t expect = 1;
    for (int64_t d = tensor.dim() - 1; d >= 4; --d) {
        expect *= tensor.size(d);
    }
    if (expect * item != planes.row_bytes) {
        PyErr_Format(PyExc_ValueError, "%s rows hold %lld bytes, pool rows %lld", name,
                     static_cast<long long>(expect * item), static_cast<long long>(planes.row_bytes));
        return false;
    }
    expect = 1;
    for (int64_t d = tensor.dim() - 1; d >= 4; --d) {
        if (tensor.size(d) > 1 && tensor.stride(d) != expect) {
            PyErr_Format(PyExc_ValueError, "%s rows must be contiguous", name);
            return false;
        }
        expect *= tensor.size(d);
    }
    rows.data = tensor.data_ptr();
    rows.layer_stride = tensor.stride(1) * item;
    rows.batch_stride = tensor.stride(0) * item;
    rows.kv_stride = tensor.stride(2) * item;
    rows.lane_stride = tensor.stride(3) * item;
    return true;
}

// decode_step(entry, topk, rows, lengths, selected, table, resident_bits,
//             bits_shift, resident_counts, slot_base, slot_token, stamps,
//             step, step_counter, status, host_table, host_planes,
//             pool_planes, slots, output, block_size, workspace)
// -> status of ekv_decode_step (the planes are KVPlanes objects; the
// workspace is a device tensor of at least ekv_decode_step_workspace_bytes)
PyObject* decode_step(PyObject*, PyObject* const* argv, Py_ssize_t argc) {
    if (argc != 22) {
        PyErr_SetString(PyExc_TypeError, "decode_step takes 22 arguments");
        return nullptr;
    }
    int64_t entry = 0, bits_shift = 0, step = 0, block_size = 0;
    if (!read_int(argv[0], "entry", entry) || !read_int(argv[7], "bits_shift", bits_shift) ||
        !read_int(argv[12], "step", step) || !read_int(argv[20], "block_size", block_size)) {
        return nullptr;
    }
    Arg args[] = {{argv[1], "topk"},         {argv[2], "rows"},           {argv[3], "lengths"},
                  {argv[4], "selected"},     {argv[5], "table"},          {argv[6], "resident_bits"},
                  {argv[8], "resident_counts"}, {argv[9], "slot_base"},   {argv[10], "slot_token"},
                  {argv[11], "stamps"},      {argv[13], "step_counter"},  {argv[14], "status"},
                  {argv[15], "host_table"},  {argv[18], "slots"},         {argv[19], "output", false},
                  {argv[21], "workspace", false}};
    for (const int required : {1, 2, 3, 4, 5, 9, 10, 11, 15, 18, 19, 21}) {
        if (argv[required] == Py_None) {
            PyErr_SetString(PyExc_TypeError, "decode_step: a required tensor is None");
            return nullptr;
        }
    }
    try {
        const int device = describe_all(args);
        if (device < 0) {
            return nullptr;
        }
        ekv_planes host{}, pool{};
        ekv_kv_rows out{};
        if (!read_planes(argv[16], host) || !read_planes(argv[17], pool) ||
            !dense_rows(*args[14].tensor, pool, *args[13].tensor, "output", out)) {
            return nullptr;
        }
        const at::Tensor& workspace = *args[15].tensor;
        ekv_step_args step_args{};
        step_args.topk = args[0].pointer();
        step_args.block_size = block_size;
        step_args.rows = args[1].pointer();
        step_args.lengths = args[2].pointer();
        step_args.selected = args[3].pointer();
        step_args.table = args[4].pointer();
        step_args.resident_bits = args[5].pointer();
        step_args.bits_shift = bits_shift;
        step_args.resident_counts = args[6].pointer();
        step_args.slot_base = args[7].pointer();
        step_args.slot_token = args[8].pointer();
        step_args.stamps = args[9].pointer();
        step_args.step = step;
        step_args.step_counter = args[10].pointer();
        step_args.status = args[11].pointer();
        step_args.host_table = args[12].pointer();
        step_args.host = &host;
        step_args.pool = &pool;
        step_args.slots = args[13].pointer();
        step_args.out = &out;
        void* workspace_data = workspace.data_ptr();
        const uint64_t workspace_bytes = static_cast<uint64_t>(workspace.numel()) * workspace.element_size();
        CurrentDevice current(device);
        void* stream = c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(device)).stream();
        int status = 0;
        Py_BEGIN_ALLOW_THREADS
        status = reinterpret_cast<decltype(&ekv_decode_step)>(entry)(&step_args, workspace_data, workspace_bytes,
                                                                     stream);
        Py_END_ALLOW_THREADS
        return PyLong_FromLong(status);
    } catch (const std::exception& error) {
        PyErr_SetString(PyExc_RuntimeError, error.what());
        return nullptr;
    }
}

// kv(entry, planes, slots, dense, zero_below, dense_name)
// -> status of ekv_gather_kv or ekv_scatter_kv (same signature): slots
// [L, B, K] of `planes` (a KVPlanes object on the slots' device) and the
// dense (B, L, KV, K, *row) rows `dense`.
PyObject* kv(PyObject*, PyObject* const* argv, Py_ssize_t argc) {
    if (argc != 6) {
        PyErr_SetString(PyExc_TypeError, "kv takes 6 arguments");
        return nullptr;
    }
    int64_t entry = 0, zero_below = 0;
    if (!read_int(argv[0], "entry", entry) || !read_int(argv[4], "zero_below", zero_below)) {
        return nullptr;
    }
    const char* name = PyUnicode_AsUTF8(argv[5]);
    if (name == nullptr) {
        return nullptr;
    }
    if (argv[2] == Py_None || argv[3] == Py_None) {
        PyErr_SetString(PyExc_TypeError, "slots and the dense rows are required");
        return nullptr;
    }
    Arg args[] = {{argv[2], "slots"}, {argv[3], name, false}};
    try {
        const int device = describe_all(args);
        if (device < 0) {
            return nullptr;
        }
        ekv_planes planes{};
        if (!read_planes(argv[1], planes)) {
            return nullptr;
        }
        PyObject* planes_device = PyObject_GetAttrString(argv[1], "device");
        if (planes_device == nullptr) {
            return nullptr;
        }
        const long long pool_device = PyLong_AsLongLong(planes_device);
        Py_DECREF(planes_device);
        if (pool_device == -1 && PyErr_Occurred()) {
            return nullptr;
        }
        if (pool_device != device) {
            PyErr_SetString(PyExc_ValueError, "slots and pool live on different devices");
            return nullptr;
        }
        ekv_kv_rows rows{};
        if (!dense_rows(*args[1].tensor, planes, *args[0].tensor, name, rows)) {
            return nullptr;
        }
        CurrentDevice current(device);
        void* stream = c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(device)).stream();
        int status = 0;
        Py_BEGIN_ALLOW_THREADS
        status = reinterpret_cast<decltype(&ekv_gather_kv)>(entry)(&planes, args[0].pointer(), &rows, zero_below,
                                                                   stream);
        Py_END_ALLOW_THREADS
        return PyLong_FromLong(status);
    } catch (const std::exception& error) {
        PyErr_SetString(PyExc_RuntimeError, error.what());
        return nullptr;
    }
}

// move(entry, src_planes, src_rows, dst_planes, dst_rows, counts, zero_below)
// -> status of ekv_move_kv (the planes are KVPlanes objects).
PyObject* move(PyObject*, PyObject* const* argv, Py_ssize_t argc) {
    if (argc != 7) {
        PyErr_SetString(PyExc_TypeError, "move takes 7 arguments");
        return nullptr;
    }
    int64_t entry = 0, zero_below = 0;
    if (!read_int(argv[0], "entry", entry) || !read_int(argv[6], "zero_below", zero_below)) {
        return nullptr;
    }
    for (const int required : {2, 4, 5}) {
        if (argv[required] == Py_None) {
            PyErr_SetString(PyExc_TypeError, "move: the row lists and counts are required");
            return nullptr;
        }
    }
    Arg args[] = {{argv[2], "src_rows"}, {argv[4], "dst_rows"}, {argv[5], "counts"}};
    try {
        const int device = describe_all(args);
        if (device < 0) {
            return nullptr;
        }
        ekv_planes src{}, dst{};
        if (!read_planes(argv[1], src) || !read_planes(argv[3], dst)) {
            return nullptr;
        }
        CurrentDevice current(device);
        void* stream = c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(device)).stream();
        int status = 0;
        Py_BEGIN_ALLOW_THREADS
        status = reinterpret_cast<decltype(&ekv_move_kv)>(entry)(&src, args[0].pointer(), &dst, args[1].pointer(),
                                                                 args[2].pointer(), zero_below, stream);
        Py_END_ALLOW_THREADS
        return PyLong_FromLong(status);
    } catch (const std::exception& error) {
        PyErr_SetString(PyExc_RuntimeError, error.what());
        return nullptr;
    }
}

// swap_in(entry, counted, topk, block_size, rows, selected, slots, misses,
//         miss_count, table, resident_bits, bits_shift, resident_counts,
//         slot_token, stamps, slot_base, host_table, promote_src,
//         promote_dst, step, step_counter, status)
// -> status of ekv_swap_in (counted = 0) or ekv_swap_in_counted (1)
PyObject* swap_in(PyObject*, PyObject* const* argv, Py_ssize_t argc) {
    if (argc != 22) {
        PyErr_SetString(PyExc_TypeError, "swap_in takes 22 arguments");
        return nullptr;
    }
    int64_t entry = 0, counted = 0, block_size = 0, bits_shift = 0, step = 0;
    if (!read_int(argv[0], "entry", entry) || !read_int(argv[1], "counted", counted) ||
        !read_int(argv[3], "block_size", block_size) || !read_int(argv[11], "bits_shift", bits_shift) ||
        !read_int(argv[19], "step", step)) {
        return nullptr;
    }
    Arg args[] = {{argv[2], "topk"},          {argv[4], "rows"},          {argv[5], "selected"},
                  {argv[6], "slots"},         {argv[7], "misses"},        {argv[8], "miss_count"},
                  {argv[9], "table"},         {argv[10], "resident_bits"}, {argv[12], "resident_counts"},
                  {argv[13], "slot_token"},   {argv[14], "stamps"},       {argv[15], "slot_base"},
                  {argv[16], "host_table"},   {argv[17], "promote_src"},  {argv[18], "promote_dst"},
                  {argv[20], "step_counter"}, {argv[21], "status"}};
    try {
        const int device = describe_all(args);
        if (device < 0) {
            return nullptr;
        }
        const ekv_tensor* t[17];
        for (int i = 0; i < 17; ++i) {
            t[i] = args[i].pointer();
        }
        CurrentDevice current(device);
        void* stream = c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(device)).stream();
        int status = 0;
        Py_BEGIN_ALLOW_THREADS
        if (counted) {
            status = reinterpret_cast<decltype(&ekv_swap_in_counted)>(entry)(
                t[0], block_size, t[1], t[2], t[3], t[4], t[5], t[6], t[7], bits_shift, t[8], t[9], t[10], t[11],
                t[12], t[13], t[14], t[15], t[16], stream);
        } else {
            status = reinterpret_cast<decltype(&ekv_swap_in)>(entry)(
                t[0], block_size, t[1], t[2], t[3], t[4], t[5], t[6], t[7], bits_shift, t[8], t[9], t[10], t[11],
                t[12], t[13], t[14], step, t[16], stream);
        }
        Py_END_ALLOW_THREADS
        return PyLong_FromLong(status);
    } catch (const std::exception& error) {
        PyErr_SetString(PyExc_RuntimeError, error.what());
        return nullptr;
    }
}

PyObject* abi_version(PyObject*, PyObject*) { return PyLong_FromLong(EKV_ABI_VERSION); }

PyObject* source_hash(PyObject*, PyObject*) { return PyUnicode_FromString(EKV_STRINGIFY(EKV_SOURCE_HASH)); }

PyMethodDef methods[] = {
    {"resolve", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(resolve)), METH_FASTCALL,
     "Describe the lookup's tensors and call an ekv_resolve_resident* entry point."},
    {"gather_rows", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(gather_rows)), METH_FASTCALL,
     "Describe the row gather's tensors and call ekv_gather_rows."},
    {"hisparse", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(hisparse)), METH_FASTCALL,
     "Check and describe the SGLang-convention swap-in's arguments and call ekv_hisparse_swap_in."},
    {"decode_step", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(decode_step)), METH_FASTCALL,
     "Describe a decode step's tensors, planes and output rows and call ekv_decode_step."},
    {"kv", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(kv)), METH_FASTCALL,
     "Describe a plane gather or scatter and call ekv_gather_kv / ekv_scatter_kv."},
    {"move", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(move)), METH_FASTCALL,
     "Describe a row move between two plane sets and call ekv_move_kv."},
    {"swap_in", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(swap_in)), METH_FASTCALL,
     "Describe the batch-token LRU swap-in's tensors and call ekv_swap_in / ekv_swap_in_counted."},
    {"abi_version", abi_version, METH_NOARGS, "EKV_ABI_VERSION this module was built against."},
    {"source_hash", source_hash, METH_NOARGS, "Fingerprint of the native sources this module was built from."},
    {nullptr, nullptr, 0, nullptr}};

PyModuleDef module = {PyModuleDef_HEAD_INIT, "_ekv_launch", "Launch helpers for the launch-bound entry points.",
                      -1, methods};

}  // namespace

PyMODINIT_FUNC PyInit__ekv_launch(void) { return PyModule_Create(&module); }
