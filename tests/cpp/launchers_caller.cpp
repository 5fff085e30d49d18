// Test program: a C++ caller written against the reference's launcher signatures
// (src/kernels/dequantize.h:25-132), linked to libqmm_gfx950.so through include/qmm_launchers.hpp.
//
// usage: launchers_caller IN OUT
//   IN:  int32 ggml_type, M, N, K; fp16 A [M, K]; packed weights W [N, K]
//   OUT: fp16 C from launch_matmul_<t> (host buffers) [M, N]; fp16 C from launch_matmul_<t>_device
//        (device buffers, null stream) [M, N]; fp16 launch_dequantize_<t>(W) [N * K]; int32 1 if a
//        K the block format cannot represent threw std::invalid_argument, as the reference does.
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <fstream>
#include <iostream>
#include <stdexcept>
#include <vector>

#include "qmm_launchers.hpp"

namespace {

void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

struct Launchers {
    void (*host)(const void*, const void*, void*, int, int, int);
    void (*device)(const void*, const void*, void*, int, int, int);
    void (*dequant)(const void*, void*, int);
    int qk;
};

Launchers launchers(int t) {
    switch (t) {
        case QMM_TYPE_Q4_0: return {launch_matmul_q4_0, launch_matmul_q4_0_device, launch_dequantize_q4_0, QK4_0};
        case QMM_TYPE_Q8_0: return {launch_matmul_q8_0, launch_matmul_q8_0_device, launch_dequantize_q8_0, QK8_0};
        case QMM_TYPE_Q4_K: return {launch_matmul_q4_k, launch_matmul_q4_k_device, launch_dequantize_q4_k, QK_K};
        case QMM_TYPE_Q6_K: return {launch_matmul_q6_k, launch_matmul_q6_k_device, launch_dequantize_q6_k, QK_K};
        default: throw std::invalid_argument("unsupported ggml_type");
    }
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 3) {
        std::cerr << "usage: launchers_caller IN OUT\n";
        return 2;
    }
    try {
        std::ifstream in(argv[1], std::ios::binary);
        int32_t hdr[4];
        if (!in.read(reinterpret_cast<char*>(hdr), sizeof(hdr))) throw std::runtime_error("short input header");
        const int t = hdr[0], M = hdr[1], N = hdr[2], K = hdr[3];
        const size_t wbytes = qmm_weight_bytes(t, N, K);
        if (M <= 0 || N <= 0 || wbytes == 0) throw std::runtime_error("bad input header");
        std::vector<uint16_t> A(static_cast<size_t>(M) * K);
        std::vector<uint8_t> W(wbytes);
        if (!in.read(reinterpret_cast<char*>(A.data()), A.size() * 2) || !in.read(reinterpret_cast<char*>(W.data()), wbytes))
            throw std::runtime_error("short input");
        const Launchers L = launchers(t);

        std::vector<uint16_t> c_host(static_cast<size_t>(M) * N), c_dev(c_host.size()), deq(static_cast<size_t>(N) * K);
        L.host(A.data(), W.data(), c_host.data(), M, N, K);

        void *dA = nullptr, *dW = nullptr, *dC = nullptr;
        check_hip(hipMalloc(&dA, A.size() * 2), "hipMalloc A");
        check_hip(hipMalloc(&dW, wbytes), "hipMalloc W");
        check_hip(hipMalloc(&dC, c_dev.size() * 2), "hipMalloc C");
        check_hip(hipMemcpy(dA, A.data(), A.size() * 2, hipMemcpyHostToDevice), "copy A");
        check_hip(hipMemcpy(dW, W.data(), wbytes, hipMemcpyHostToDevice), "copy W");
        L.device(dA, dW, dC, M, N, K);
        check_hip(hipDeviceSynchronize(), "synchronize");
        check_hip(hipMemcpy(c_dev.data(), dC, c_dev.size() * 2, hipMemcpyDeviceToHost), "copy C");
        check_hip(hipFree(dA), "free A");
        check_hip(hipFree(dW), "free W");
        check_hip(hipFree(dC), "free C");

        L.dequant(W.data(), deq.data(), N * K);

        int32_t threw = 0;
        try {
            L.host(A.data(), W.data(), c_host.data() /* not written: rejected first */, M, N, K + 1);
        } catch (const std::invalid_argument&) {
            threw = 1;
        }
        // the rejected call above must not have touched the first output; recompute to be sure
        std::vector<uint16_t> c_again(c_host.size());
        L.host(A.data(), W.data(), c_again.data(), M, N, K);

        std::ofstream out(argv[2], std::ios::binary);
        out.write(reinterpret_cast<const char*>(c_again.data()), c_again.size() * 2);
        out.write(reinterpret_cast<const char*>(c_dev.data()), c_dev.size() * 2);
        out.write(reinterpret_cast<const char*>(deq.data()), deq.size() * 2);
        out.write(reinterpret_cast<const char*>(&threw), sizeof(threw));
        if (!out) throw std::runtime_error("write failed");
    } catch (const std::exception& e) {
        std::cerr << "launchers_caller: " << e.what() << "\n";
        return 1;
    }
    return 0;
}
