// MatMulNBitsKernel.hpp -- C++ host mirror of the reference's Java operator
// interface for int4 MatMulNBits, implemented over the C ABI of libmnb_hip.so.
//
// Mirrors (paths relative to the reference repository root):
//   MatMulNBitsKernel            directml-windows-bindings/src/main/java/com/aresstack/windirectml/windows/MatMulNBitsKernel.java
//     ctor (N, K, qWeight, scales, zeroPoints, blockSize)  :940-970
//     matvec(x, out) / matvec(x)                            :1847-1914 / :1674-1678  (overwrite)
//     matmulBatch(xBatch, outBatch, M)                      :2145-2263               (overwrite)
//     supportsBatch() / maxBatchRows()                      :2128 / :2361
//     dequantizeInt4(q, scales, zp, N, K, blockSize)        :2674-2705
//     getN() / getK() / close()                             :2803-2812 / :2740
//   QuantizedWeightMatrix        directml-inference/.../qwen/Qwen2Weights.java:289-319  (y += semantics)
//   DenseProjection              directml-inference/.../decoderonly/DecoderOnlyDenseProjection.java:9-59
//
// Error behaviour follows the reference: std::invalid_argument where Java
// throws IllegalArgumentException, std::logic_error for IllegalStateException
// ("Kernel not prepared"), std::runtime_error("MatMulNBitsKernel.<op> failed:
// ...") for native failures.
#pragma once

#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "mnb.h"

namespace mnb {

inline void check(int32_t rc, const char *op) {
    if (rc == MNB_OK) return;
    std::string msg = mnb_last_error();
    if (rc == MNB_ERR_INVALID_ARGUMENT) throw std::invalid_argument(msg);
    if (rc == MNB_ERR_INVALID_STATE) throw std::logic_error(msg);
    throw std::runtime_error(std::string("MatMulNBitsKernel.") + op + " failed: " + msg);
}

// The device binding shared by all kernels (the reference's WindowsBindings).
class Bindings {
public:
    explicit Bindings(int device = 0) { check(mnb_context_create(device, &ctx_), "init"); }
    ~Bindings() { if (ctx_) mnb_context_destroy(ctx_); }
    Bindings(const Bindings &) = delete;
    Bindings &operator=(const Bindings &) = delete;
    mnb_context *context() const { return ctx_; }
    mnb_device_info info() const {
        mnb_device_info i{};
        check(mnb_context_info(ctx_, &i), "info");
        return i;
    }

private:
    mnb_context *ctx_ = nullptr;
};

class MatMulNBitsKernel {
public:
    // scales are per-block fp32 [N * K/blockSize], zeroPoints the flat packed
    // uint4 stream ((N*K/blockSize + 1)/2 bytes), as the reference takes them.
    MatMulNBitsKernel(Bindings &wb, int N, int K, const std::vector<uint8_t> &qWeight,
                      const std::vector<float> &scales, const std::vector<uint8_t> &zeroPoints, int blockSize)
        : ctx_(wb.context()), N_(N), K_(K) {
        check(mnb_weight_create(ctx_, N, K, blockSize, 4, qWeight.data(), (int64_t)qWeight.size(), scales.data(),
                                MNB_F32, (int64_t)scales.size(), zeroPoints.empty() ? nullptr : zeroPoints.data(),
                                (int64_t)zeroPoints.size(), zeroPoints.empty() ? MNB_ZP_NONE : MNB_ZP_FLAT, 0, &w_),
              "prepare");
    }
    ~MatMulNBitsKernel() { close(); }
    MatMulNBitsKernel(const MatMulNBitsKernel &) = delete;
    MatMulNBitsKernel &operator=(const MatMulNBitsKernel &) = delete;

    // out = x @ W^T (overwrite); x.size() must equal K, out.size() >= N
    void matvec(const std::vector<float> &x, std::vector<float> &out) {
        ensurePrepared();
        if ((int64_t)x.size() != K_)
            throw std::invalid_argument("Input length " + std::to_string(x.size()) + " != K=" + std::to_string(K_));
        check(mnb_matmul(ctx_, w_, 1, x.data(), MNB_F32, (int64_t)x.size(), out.data(), MNB_F32,
                         (int64_t)out.size(), MNB_HOST_MEMORY, nullptr),
              "matvec");
    }

    std::vector<float> matvec(const std::vector<float> &x) {
        std::vector<float> result((size_t)N_);
        matvec(x, result);
        return result;
    }

    // outBatch[M, N] = xBatch[M, K] @ W^T (overwrite), any M >= 1
    void matmulBatch(const std::vector<float> &xBatch, std::vector<float> &outBatch, int M) {
        ensurePrepared();
        if (M < 1) throw std::invalid_argument("M out of range [1, " + std::to_string(maxBatchRows()) + "]: " + std::to_string(M));
        check(mnb_matmul(ctx_, w_, M, xBatch.data(), MNB_F32, (int64_t)xBatch.size(), outBatch.data(), MNB_F32,
                         (int64_t)outBatch.size(), MNB_HOST_MEMORY, nullptr),
              "matmulBatch");
    }

    // y += x @ W^T, the QuantizedWeight.matvec/matmul semantic
    void matmulAccumulate(const std::vector<float> &x, std::vector<float> &y, int seqLen) {
        ensurePrepared();
        check(mnb_matmul(ctx_, w_, seqLen, x.data(), MNB_F32, (int64_t)x.size(), y.data(), MNB_F32, (int64_t)y.size(),
                         MNB_HOST_MEMORY | MNB_ACCUMULATE, nullptr),
              seqLen == 1 ? "matvec" : "matmul");
    }

    bool supportsBatch() const { return w_ != nullptr && mnb_supports_batch(w_) != 0; }
    static int maxBatchRows() { return mnb_max_batch_rows(); }
    int getN() const { return N_; }
    int getK() const { return K_; }

    // dequantized weight [N * K] fp32, bit-identical to the reference's dequantizeInt4
    std::vector<float> dequantize() {
        ensurePrepared();
        std::vector<float> out((size_t)N_ * K_);
        check(mnb_dequantize(ctx_, w_, out.data(), MNB_F32, (int64_t)out.size(), MNB_HOST_MEMORY, nullptr),
              "dequantizeInt4");
        return out;
    }

    static std::vector<float> dequantizeInt4(Bindings &wb, const std::vector<uint8_t> &qWeight,
                                             const std::vector<float> &scales,
                                             const std::vector<uint8_t> &zeroPoints, int N, int K, int blockSize) {
        MatMulNBitsKernel k(wb, N, K, qWeight, scales, zeroPoints, blockSize);
        return k.dequantize();
    }

    void close() {
        if (w_) {
            mnb_weight_destroy(w_);
            w_ = nullptr;
        }
    }

    const mnb_weight *handle() const { return w_; }

private:
    void ensurePrepared() const {
        if (!w_) throw std::logic_error("Kernel not prepared");
    }
    mnb_context *ctx_;
    mnb_weight *w_ = nullptr;
    int N_, K_;
};

// Qwen2Weights.WeightMatrix over the GPU kernel: accumulate semantics (y += x W^T).
class QuantizedWeightMatrix {
public:
    explicit QuantizedWeightMatrix(std::shared_ptr<MatMulNBitsKernel> k) : k_(std::move(k)) {}
    void matvec(const std::vector<float> &x, std::vector<float> &y) { k_->matmulAccumulate(x, y, 1); }
    void matmul(const std::vector<float> &x, std::vector<float> &y, int seqLen) { k_->matmulAccumulate(x, y, seqLen); }
    int N() const { return k_->getN(); }
    int K() const { return k_->getK(); }

private:
    std::shared_ptr<MatMulNBitsKernel> k_;
};

// DecoderOnlyDenseProjection over the GPU kernel (projectInto overwrites).
class DenseProjection {
public:
    DenseProjection(std::string name, std::shared_ptr<MatMulNBitsKernel> k) : name_(std::move(name)), k_(std::move(k)) {}
    const std::string &name() const { return name_; }
    int inputSize() const { return k_->getK(); }
    int outputSize() const { return k_->getN(); }
    std::vector<float> project(const std::vector<float> &input) { return k_->matvec(input); }
    void projectInto(const std::vector<float> &input, std::vector<float> &output) {
        if ((int)output.size() < outputSize())
            throw std::invalid_argument("output buffer too small for " + name_);
        k_->matvec(input, output);
    }
    std::vector<float> projectSequence(const std::vector<float> &input, int sequenceLength) {
        if (sequenceLength < 1) throw std::invalid_argument("sequenceLength must be positive: " + std::to_string(sequenceLength));
        if ((int64_t)input.size() != (int64_t)sequenceLength * inputSize())
            throw std::invalid_argument("Sequence input length mismatch for " + name_);
        std::vector<float> out((size_t)sequenceLength * outputSize());
        k_->matmulBatch(input, out, sequenceLength);
        return out;
    }
    void close() { k_->close(); }

private:
    std::string name_;
    std::shared_ptr<MatMulNBitsKernel> k_;
};

}  // namespace mnb
