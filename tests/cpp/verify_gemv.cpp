// verify_gemv.cpp -- the reference's --verify-gemv check (src/main.rs:2629-2675)
// as a C++ host over include/quartz_hip.hpp.  Test infrastructure: the CPU side
// is the oracle's o_gemv (oracle/liboracle.so), the GPU side the product library.
//
//   verify_gemv FILE.gguf
//
// For the first 2-D tensor of each ggml type (in_dim % 32 == 0, both dims > 0):
// x = verify_input(in_dim), cpu = o_gemv, gpu = verify_gemv_hip, one line in the
// reference's format.  Each 3-D tensor [in, out, n_experts] is also checked
// expert by expert through gpu_expert_slice + GpuScratch::gemv_slice (the MoE
// host path, src/cuda.rs:250-281).  Exit status 1 if any line mismatches.
#include <cstdio>
#include <set>
#include <vector>

#include "quartz_hip.hpp"

extern "C" int o_gemv(uint32_t ggml_type, const float* x, const uint8_t* data, int in_dim, int out_dim, float* y);

namespace qh = quartz_hip;

static bool report(uint32_t type, const char* name, int in_dim, int out_dim, const std::vector<float>& cpu,
                   const std::vector<float>& gpu) {
    const qh::VerifyResult r = qh::verify_ok(cpu, gpu);
    std::printf("type %3u  %-40s  in=%6d out=%6d  maxdiff=%.5f  rel=%.5f  %s\n", type, name, in_dim, out_dim,
                r.maxdiff, r.rel, r.ok ? "OK" : "*** MISMATCH ***");
    std::fflush(stdout);
    return r.ok;
}

int main(int argc, char** argv) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: %s FILE.gguf\n", argv[0]);
        return 2;
    }
    qh_gguf* f = nullptr;
    if (hip_gguf_open(argv[1], &f) != QH_OK) {
        std::fprintf(stderr, "cannot open %s: %s\n", argv[1], hip_last_error());
        return 2;
    }
    bool all_ok = true;
    int checked = 0;
    try {
        std::set<uint32_t> seen;
        const int64_t nt = hip_gguf_tensor_count(f);
        for (int64_t i = 0; i < nt; i++) {
            const char* name = nullptr;
            uint32_t nd = 0, type = 0;
            uint64_t dims[8] = {}, off = 0;
            qh::check("hip_gguf_tensor_info", hip_gguf_tensor_info(f, i, &name, &nd, dims, &type, &off));
            if (nd < 2 || nd > 3) continue;
            const int in_dim = (int)dims[0], out_dim = (int)dims[1];
            if (in_dim % 32 != 0 || in_dim == 0 || out_dim == 0) continue;
            size_t bytes = 0;
            const uint8_t* data = static_cast<const uint8_t*>(hip_gguf_tensor_data(f, i, &bytes));
            const std::vector<float> x = qh::verify_input((size_t)in_dim);
            std::vector<float> cpu((size_t)out_dim);
            if (nd == 2) {
                if (!seen.insert(type).second) continue;
                if (o_gemv(type, x.data(), data, in_dim, out_dim, cpu.data()) != 0) {
                    std::printf("type %3u  %-40s  oracle has no kernel for this type, skipped\n", type, name);
                    continue;
                }
                const std::vector<float> gpu = qh::verify_gemv_hip(x.data(), x.size(), data, bytes, type, in_dim, out_dim);
                all_ok = report(type, name, in_dim, out_dim, cpu, gpu) && all_ok;
                checked++;
            } else {
                const size_t per = (size_t)in_dim * (size_t)out_dim, eb = hip_type_size(type, per);
                const qh::GpuBuf buf = qh::GpuBuf::upload(data, bytes);
                const qh::GpuScratch sc((size_t)in_dim, (size_t)out_dim);
                for (uint64_t e = 0; e < dims[2]; e++) {
                    if (o_gemv(type, x.data(), data + e * eb, in_dim, out_dim, cpu.data()) != 0) break;
                    const qh::GpuSlice s = qh::gpu_expert_slice(buf, type, (size_t)e, per);
                    const std::vector<float> gpu = sc.gemv_slice(x.data(), x.size(), s, in_dim, out_dim);
                    char label[96];
                    std::snprintf(label, sizeof label, "%s[%llu]", name, (unsigned long long)e);
                    all_ok = report(type, label, in_dim, out_dim, cpu, gpu) && all_ok;
                    checked++;
                }
                // one past the last expert must be refused, not read out of bounds
                bool refused = false;
                try {
                    (void)qh::gpu_expert_slice(buf, type, (size_t)dims[2], per);
                } catch (const qh::Error& err) {
                    refused = err.status() == QH_ERR_RANGE;
                }
                if (!refused) {
                    std::printf("%s: expert %llu past the tensor was not refused\n", name,
                                (unsigned long long)dims[2]);
                    all_ok = false;
                }
            }
        }
    } catch (const qh::Error& err) {
        std::fprintf(stderr, "error: %s\n", err.what());
        hip_gguf_close(f);
        return 1;
    }
    hip_gguf_close(f);
    std::printf("%d checks, %s\n", checked, all_ok ? "all OK" : "MISMATCH");
    return all_ok && checked > 0 ? 0 : 1;
}
