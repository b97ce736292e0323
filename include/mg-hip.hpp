// mg-hip.hpp — MI355X (gfx950) backend: execute an mg::Graph on the GPU.
//
// Public interface of the reference's OpenCLRuntime (include/mg-opencl.hpp:23-58) so it can
// stand in for it: construct, compute(Graph&), device_name(), invalidate(Tensor*),
// import_host_region(), per-op profiling. compute() walks the topologically sorted nodes,
// uploads leaves once (cached by host address and size; quantized weights are rewritten on
// upload into the device-native packed layout), runs one libmgh kernel per node, writes the
// final node back to its host data and returns when the device is done (like the reference,
// mg-opencl.cpp:1354-1656). Errors throw std::runtime_error.
//
// mg-hip.hpp and the reference's mg-opencl.hpp are alternatives (both define OpProfile).
#pragma once
#include "mg-tensor.hpp"

#include <memory>
#include <string>
#include <vector>

struct mgh_ctx;

namespace mg {

struct OpProfile {
    std::string op;     // op-type name; MulMat split into "MulMat(q)" / "MulMat(f32)"
    int count;          // dispatches of this type
    double ms;          // accumulated device time (each node timed on its own)
};

class HipRuntime {
public:
    HipRuntime();                      // device 0
    explicit HipRuntime(int device);
    ~HipRuntime();
    HipRuntime(const HipRuntime&) = delete;
    HipRuntime& operator=(const HipRuntime&) = delete;

    void compute(Graph& g);
    const std::string& device_name() const;

    // Forget the device copy of a leaf whose host contents changed at the same address
    // (the reference's contract, mg-opencl.cpp:1283-1286).
    void invalidate(Tensor* t);

    // Zero-copy import of host memory is a Mali-specific path in the reference; weights are
    // copied to HBM once here, so this returns false and changes nothing.
    bool import_host_region(void* base, size_t size);

    void profile_enable(bool on);
    void profile_reset();
    std::vector<OpProfile> profile_report() const;

    // Algorithm for quantized FC weights: 2 = dequantized weights x fp16 activations (the
    // default: the reference's dequant-fused path, which it takes on every device without
    // cl_arm_integer_dot_product, mg-opencl.cpp:1237-1238, 1400-1423), 1 = int8-dot (its Mali
    // int8 path, :1381-1398).
    void set_quant_algo(int algo);

    // ---- device-resident decoding: additions with no counterpart in OpenCLRuntime ----
    // For the next compute only, leaf `t` reads caller-owned device memory `d` (for example
    // token ids that an on-device decode step rewrites between forwards) instead of its host
    // data.
    void bind_device(const Tensor* t, void* d);
    // compute() without the final readback: returns the device address of the final node's
    // result, which stays valid until the next compute call. Kernels are only enqueued.
    const void* compute_device(Graph& g);
    // the libmgh context whose stream runs the graph (work enqueued on it is ordered after
    // the graph's kernels)
    mgh_ctx* context() const;

private:
    const void* run(Graph& g, bool readback);

    struct Impl;
    std::unique_ptr<Impl> p_;
};

}  // namespace mg
