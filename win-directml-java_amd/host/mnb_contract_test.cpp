// mnb_contract_test.cpp -- the reference's QuantizedWeightMatvecTest cases
// (directml-inference/src/test/java/com/aresstack/windirectml/inference/qwen/
// QuantizedWeightMatvecTest.java:86-195), run against the C++ mirror of
// MatMulNBitsKernel on the GPU, plus the operator's error contract
// (MatMulNBitsKernel.java:1849-1850, 2147-2152 and "Kernel not prepared").
//
// Exit status 0 when every case passes; each case prints one line.
#include <cmath>
#include <cstdio>
#include <functional>
#include <string>
#include <vector>

#include "MatMulNBitsKernel.hpp"

using namespace mnb;

static int g_failed = 0;

static void expect(bool cond, const std::string &name, const std::string &detail = "") {
    std::printf("%s %s %s\n", cond ? "PASS" : "FAIL", name.c_str(), detail.c_str());
    std::fflush(stdout);
    if (!cond) ++g_failed;
}

static constexpr int BS = 128;

struct Uniform {
    std::vector<uint8_t> q;
    std::vector<float> s;
    std::vector<uint8_t> zp;
};

// QuantizedWeightMatvecTest.java:31-50 uniformWeight: K = 128, every nibble,
// zero point and scale equal.
static Uniform uniformWeight(int N, int nibble, int zp, float scale) {
    Uniform u;
    u.q.assign((size_t)N * BS / 2, (uint8_t)((nibble & 0xF) | ((nibble & 0xF) << 4)));
    u.s.assign((size_t)N, scale);
    u.zp.assign((size_t)(N + 1) / 2, (uint8_t)((zp & 0xF) | ((zp & 0xF) << 4)));
    return u;
}

static bool near(float a, float b, float tol) { return std::fabs(a - b) <= tol; }

int main() {
    Bindings wb(0);

    {   // allOnesNibbleZpZero: y = 128
        Uniform u = uniformWeight(4, 1, 0, 1.0f);
        MatMulNBitsKernel k(wb, 4, BS, u.q, u.s, u.zp, BS);
        std::vector<float> x(BS, 1.0f), y(4, 0.0f);
        k.matvec(x, y);
        bool ok = true;
        for (float v : y) ok = ok && near(v, 128.0f, 1e-3f);
        expect(ok, "matvecAllOnesNibbleZpZero");
    }
    {   // nibble8Zp8ScaleOneGivesZero: y = 0
        Uniform u = uniformWeight(4, 8, 8, 1.0f);
        MatMulNBitsKernel k(wb, 4, BS, u.q, u.s, u.zp, BS);
        std::vector<float> x(BS, 5.0f), y(4, 7.0f);
        k.matvec(x, y);   // overwrite semantics: the 7s must be replaced
        bool ok = true;
        for (float v : y) ok = ok && near(v, 0.0f, 1e-6f);
        expect(ok, "matvecNibble8Zp8ScaleOneGivesZero");
    }
    {   // scalePropagates: nibble 2, scale 0.5 -> 128
        Uniform u = uniformWeight(2, 2, 0, 0.5f);
        MatMulNBitsKernel k(wb, 2, BS, u.q, u.s, u.zp, BS);
        std::vector<float> y = k.matvec(std::vector<float>(BS, 1.0f));
        expect(near(y[0], 128.0f, 1e-3f) && near(y[1], 128.0f, 1e-3f), "matvecScalePropagates");
    }
    {   // accumulatesIntoExistingY through the WeightMatrix (y +=) adapter
        Uniform u = uniformWeight(2, 1, 0, 1.0f);
        auto k = std::make_shared<MatMulNBitsKernel>(wb, 2, BS, u.q, u.s, u.zp, BS);
        QuantizedWeightMatrix m(k);
        std::vector<float> x(BS, 1.0f), y = {10.0f, 20.0f};
        m.matvec(x, y);
        expect(near(y[0], 138.0f, 1e-3f) && near(y[1], 148.0f, 1e-3f), "matvecAccumulatesIntoExistingY");
    }
    {   // matvecMatchesReferenceForLargerN: nibble 3, zp 1, scale 2 -> 4 * sum(x)
        Uniform u = uniformWeight(16, 3, 1, 2.0f);
        MatMulNBitsKernel k(wb, 16, BS, u.q, u.s, u.zp, BS);
        std::vector<float> x(BS);
        double ref = 0;
        for (int i = 0; i < BS; ++i) {
            x[i] = (float)std::sin(i * 0.1);
            ref += 4.0 * x[i];
        }
        std::vector<float> y = k.matvec(x);
        // x is rounded to fp16 on the device: |err| <= 1e-3*sqrt(K)*max|x|*max|w|
        const float tol = 1e-3f * std::sqrt((float)BS) * 1.0f * 4.0f;
        bool ok = true;
        for (float v : y) ok = ok && near(v, (float)ref, tol);
        expect(ok, "matvecMatchesReferenceForLargerN", "ref=" + std::to_string(ref) + " got=" + std::to_string(y[0]));
    }
    {   // matmulMatchesRepeatedMatvecCalls
        Uniform u = uniformWeight(8, 5, 2, 0.25f);
        MatMulNBitsKernel k(wb, 8, BS, u.q, u.s, u.zp, BS);
        std::vector<float> x0(BS), x1(BS);
        for (int i = 0; i < BS; ++i) {
            x0[i] = (float)std::cos(i * 0.05);
            x1[i] = (float)std::sin(i * 0.07 + 1.0);
        }
        std::vector<float> xb(x0);
        xb.insert(xb.end(), x1.begin(), x1.end());
        std::vector<float> yb(16);
        k.matmulBatch(xb, yb, 2);
        std::vector<float> r0 = k.matvec(x0), r1 = k.matvec(x1);
        bool ok = true;
        for (int n = 0; n < 8; ++n)
            ok = ok && near(yb[n], r0[n], std::fabs(r0[n]) * 1e-4f + 1e-4f) &&
                 near(yb[8 + n], r1[n], std::fabs(r1[n]) * 1e-4f + 1e-4f);
        expect(ok, "matmulMatchesRepeatedMatvecCalls");
    }
    {   // dequantizeInt4 closed form: (3 - 1) * 2 = 4 everywhere
        Uniform u = uniformWeight(3, 3, 1, 2.0f);
        std::vector<float> w = MatMulNBitsKernel::dequantizeInt4(wb, u.q, u.s, u.zp, 3, BS, BS);
        bool ok = w.size() == (size_t)3 * BS;
        for (float v : w) ok = ok && v == 4.0f;
        expect(ok, "dequantizeInt4ClosedForm");
    }
    {   // error contract
        Uniform u = uniformWeight(4, 1, 0, 1.0f);
        MatMulNBitsKernel k(wb, 4, BS, u.q, u.s, u.zp, BS);
        bool threw = false;
        try {
            std::vector<float> y(4);
            k.matvec(std::vector<float>(BS - 1, 1.0f), y);
        } catch (const std::invalid_argument &e) {
            threw = std::string(e.what()).find("Input length 127 != K=128") != std::string::npos;
        }
        expect(threw, "matvecRejectsWrongInputLength");
        threw = false;
        try {
            std::vector<float> xb(BS), yb(3);
            k.matmulBatch(xb, yb, 1);
        } catch (const std::invalid_argument &) {
            threw = true;
        }
        expect(threw, "matmulBatchRejectsShortOutput");
        threw = false;
        try {
            std::vector<float> xb(BS), yb(4);
            k.matmulBatch(xb, yb, 0);
        } catch (const std::invalid_argument &) {
            threw = true;
        }
        expect(threw, "matmulBatchRejectsNonPositiveM");
        expect(k.supportsBatch() && MatMulNBitsKernel::maxBatchRows() >= 1 << 20, "supportsBatchAnyM");
        k.close();
        threw = false;
        try {
            k.matvec(std::vector<float>(BS, 1.0f));
        } catch (const std::logic_error &e) {
            threw = std::string(e.what()) == "Kernel not prepared";
        }
        expect(threw, "closedKernelIsNotPrepared");
    }
    {   // DecoderOnlyDenseProjection adapter: projectSequence == per-row project
        Uniform u = uniformWeight(5, 9, 8, 0.5f);
        auto k = std::make_shared<MatMulNBitsKernel>(wb, 5, BS, u.q, u.s, u.zp, BS);
        DenseProjection proj("test.proj", k);
        std::vector<float> seq(3 * BS);
        for (int i = 0; i < 3 * BS; ++i) seq[i] = (float)((i % 7) - 3);
        std::vector<float> out = proj.projectSequence(seq, 3);
        bool ok = proj.inputSize() == BS && proj.outputSize() == 5;
        for (int t = 0; t < 3; ++t) {
            std::vector<float> row(seq.begin() + t * BS, seq.begin() + (t + 1) * BS);
            std::vector<float> r = proj.project(row);
            for (int n = 0; n < 5; ++n) ok = ok && near(out[t * 5 + n], r[n], 1e-4f);
        }
        expect(ok, "denseProjectionSequenceMatchesRows");
    }
    std::printf("%s: %d failed\n", g_failed ? "FAILED" : "OK", g_failed);
    return g_failed ? 1 : 0;
}
