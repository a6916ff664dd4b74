// A C++ host of the C ABI with no Python and no torch: device buffers from
// the HIP runtime, one plan over three leaves (a bf16 leaf of whole
// 2048-element blocks, a bf16 leaf with a partial last block, an f32 leaf
// below min_size with f32 fallback moments), two fused adamw8 steps with the
// IEEE direction (RF_EXACT), the second over new gradient buffers through
// rf_adam8_plan_run_leaves.  These are the calls an XLA FFI handler makes
// over the buffers XLA hands it.  The scalars are derived as the reference
// derives them (adam8.py:322-339; optax add_decayed_weights and
// scale_by_learning_rate inside adamw8, adam8.py:394-443).
//
// rf_c_host_step_run(out_dir) writes raw little-endian arrays (built as a
// shared library for the test, which loads it in its own process; with
// -DRF_C_HOST_MAIN, main(argc, argv) makes it a program taking <out_dir>):
// hp_step{1,2}.bin (b1, 1-b1, b2, 1-b2, bc1, bc2, eps, eps_root, wd, -lr as
// f32), and per leaf i: p0_i, g1_i, g2_i, p_i (params, then grads of the two
// steps, then the params after them) and mu_i, mus_i, nu_i, nus_i (codes and
// scales, or the f32 fallback moments).  Returns 0 on success.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "rfadam8.h"

#define CK_HIP(x)                                                                          \
    do {                                                                                   \
        hipError_t e_ = (x);                                                               \
        if (e_ != hipSuccess) {                                                            \
            std::fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
            return 2;                                                                      \
        }                                                                                  \
    } while (0)
#define CK_RF(x)                                                                           \
    do {                                                                                   \
        rf_status s_ = (x);                                                                \
        if (s_ != RF_OK) {                                                                 \
            std::fprintf(stderr, "rf error %d at line %d: %s\n", s_, __LINE__, rf_last_error()); \
            return 3;                                                                      \
        }                                                                                  \
    } while (0)

namespace {

uint64_t g_state = 0x9E3779B97F4A7C15ull;
float uniform_pm1()  // xorshift64*: uniform in [-1, 1)
{
    g_state ^= g_state >> 12;
    g_state ^= g_state << 25;
    g_state ^= g_state >> 27;
    const uint64_t r = g_state * 0x2545F4914F6CDD1Dull;
    return (float)((double)(r >> 11) * (1.0 / 9007199254740992.0) * 2.0 - 1.0);
}

uint16_t to_bf16(float x)  // round to nearest even (finite inputs)
{
    uint32_t u;
    std::memcpy(&u, &x, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

bool write_file(const std::string& path, const void* data, size_t bytes)
{
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) return false;
    const bool ok = std::fwrite(data, 1, bytes, f) == bytes;
    return std::fclose(f) == 0 && ok;
}

struct Leaf {
    int64_t size;
    int32_t pdtype;  // RF_BF16 or RF_F32 (grads of the same dtype)
    bool quantized;
    int64_t nblocks() const { return (size + 2047) / 2048; }
    size_t pbytes() const { return (size_t)size * (pdtype == RF_BF16 ? 2 : 4); }
};

std::vector<uint8_t> random_array(const Leaf& L, float scale)
{
    std::vector<uint8_t> out(L.pbytes());
    for (int64_t i = 0; i < L.size; ++i) {
        const float x = uniform_pm1() * scale;
        if (L.pdtype == RF_BF16) {
            const uint16_t h = to_bf16(x);
            std::memcpy(out.data() + 2 * i, &h, 2);
        } else {
            std::memcpy(out.data() + 4 * i, &x, 4);
        }
    }
    return out;
}

rf_adam8_hparams hparams(int count)
{
    const double b1 = 0.9, b2 = 0.999, eps = 1e-8, wd = 0.01, lr = 1e-3;
    rf_adam8_hparams hp;
    std::memset(&hp, 0, sizeof hp);
    const float t = (float)count;
    hp.b1 = (float)b1;
    hp.one_minus_b1 = (float)(1.0 - b1);
    hp.b2 = (float)b2;
    hp.one_minus_b2 = (float)(1.0 - b2);
    hp.bc1 = 1.0f - std::pow(hp.b1, t);
    hp.bc2 = 1.0f - std::pow(hp.b2, t);
    hp.bc1_next = 1.0f - std::pow(hp.b1, (float)(count + 1));
    hp.eps = (float)eps;
    hp.eps_root = 0.0f;
    hp.weight_decay = (float)wd;
    hp.neg_lr = (float)(-lr);
    hp.nesterov_one_minus_b1 = hp.one_minus_b1;
    hp.flags = RF_DECAY_WEAK | RF_LR | RF_EXACT;
    return hp;
}

}  // namespace

extern "C" __attribute__((visibility("default"))) int rf_c_host_step_run(const char* out_dir)
{
    if (!out_dir) return 1;
    const std::string out = out_dir;
    const std::vector<Leaf> leaves = {{3 * 2048, RF_BF16, true}, {5000, RF_BF16, true}, {1000, RF_F32, false}};
    const int n = (int)leaves.size();
    hipStream_t stream;
    CK_HIP(hipStreamCreate(&stream));

    std::vector<rf_adam8_leaf> table(n);
    std::vector<void*> dp(n), dg1(n), dg2(n), dmu(n), dnu(n);
    std::vector<float*> dmus(n, nullptr), dnus(n, nullptr);
    std::vector<std::vector<uint8_t>> p0(n), g1(n), g2(n);
    for (int i = 0; i < n; ++i) {
        const Leaf& L = leaves[i];
        p0[i] = random_array(L, 0.05f);
        g1[i] = random_array(L, 1e-3f);
        g2[i] = random_array(L, 1e-3f);
        CK_HIP(hipMalloc(&dp[i], L.pbytes()));
        CK_HIP(hipMalloc(&dg1[i], L.pbytes()));
        CK_HIP(hipMalloc(&dg2[i], L.pbytes()));
        CK_HIP(hipMemcpy(dp[i], p0[i].data(), L.pbytes(), hipMemcpyHostToDevice));
        CK_HIP(hipMemcpy(dg1[i], g1[i].data(), L.pbytes(), hipMemcpyHostToDevice));
        CK_HIP(hipMemcpy(dg2[i], g2[i].data(), L.pbytes(), hipMemcpyHostToDevice));
        rf_adam8_leaf& t = table[i];
        std::memset(&t, 0, sizeof t);
        t.param = dp[i];
        t.grad = dg1[i];
        t.size = L.size;
        t.param_dtype = L.pdtype;
        t.grad_dtype = L.pdtype;
        t.state_index = i;
        t.param_index = i;
        t.flags = RF_LEAF_DECAY;
        if (L.quantized) {
            // the zero state of _init_moment_leaf (adam8.py:605-630):
            // quantize_blocks of zeros gives codes 127 / 0 and scale 1
            const size_t nc = (size_t)L.nblocks() * 2048;
            CK_HIP(hipMalloc(&dmu[i], nc));
            CK_HIP(hipMalloc(&dnu[i], nc));
            CK_HIP(hipMemset(dmu[i], 127, nc));
            CK_HIP(hipMemset(dnu[i], 0, nc));
            std::vector<float> ones((size_t)L.nblocks(), 1.0f);
            CK_HIP(hipMalloc((void**)&dmus[i], ones.size() * 4));
            CK_HIP(hipMalloc((void**)&dnus[i], ones.size() * 4));
            CK_HIP(hipMemcpy(dmus[i], ones.data(), ones.size() * 4, hipMemcpyHostToDevice));
            CK_HIP(hipMemcpy(dnus[i], ones.data(), ones.size() * 4, hipMemcpyHostToDevice));
            t.block_size = 2048;
            t.moment_kind = RF_MOMENT_QUANTIZED;
            t.mu_scales = dmus[i];
            t.nu_scales = dnus[i];
        } else {
            CK_HIP(hipMalloc(&dmu[i], (size_t)L.size * 4));
            CK_HIP(hipMalloc(&dnu[i], (size_t)L.size * 4));
            CK_HIP(hipMemset(dmu[i], 0, (size_t)L.size * 4));
            CK_HIP(hipMemset(dnu[i], 0, (size_t)L.size * 4));
            t.block_size = 2048;
            t.moment_kind = RF_MOMENT_F32;
        }
        t.mu = dmu[i];
        t.nu = dnu[i];
    }
    CK_HIP(hipDeviceSynchronize());

    rf_adam8_plan* plan = nullptr;
    CK_RF(rf_adam8_plan_create(table.data(), n, 1, &plan));
    const rf_adam8_hparams hp1 = hparams(1), hp2 = hparams(2);
    CK_RF(rf_adam8_plan_run(plan, &hp1, stream));
    for (int i = 0; i < n; ++i) table[i].grad = dg2[i];  // step 2: new gradient buffers
    CK_RF(rf_adam8_plan_run_leaves(plan, table.data(), n, &hp2, stream));
    CK_HIP(hipStreamSynchronize(stream));
    CK_RF(rf_adam8_plan_destroy(plan));

    const rf_adam8_hparams* hps[2] = {&hp1, &hp2};
    for (int s = 0; s < 2; ++s) {
        const float v[10] = {hps[s]->b1, hps[s]->one_minus_b1, hps[s]->b2, hps[s]->one_minus_b2, hps[s]->bc1,
                             hps[s]->bc2, hps[s]->eps, hps[s]->eps_root, hps[s]->weight_decay, hps[s]->neg_lr};
        if (!write_file(out + "/hp_step" + std::to_string(s + 1) + ".bin", v, sizeof v)) return 4;
    }
    for (int i = 0; i < n; ++i) {
        const Leaf& L = leaves[i];
        const std::string k = "_" + std::to_string(i) + ".bin";
        std::vector<uint8_t> p(L.pbytes());
        CK_HIP(hipMemcpy(p.data(), dp[i], L.pbytes(), hipMemcpyDeviceToHost));
        bool ok = write_file(out + "/p0" + k, p0[i].data(), L.pbytes()) &&
                  write_file(out + "/g1" + k, g1[i].data(), L.pbytes()) &&
                  write_file(out + "/g2" + k, g2[i].data(), L.pbytes()) && write_file(out + "/p" + k, p.data(), L.pbytes());
        const size_t mbytes = L.quantized ? (size_t)L.nblocks() * 2048 : (size_t)L.size * 4;
        std::vector<uint8_t> mu(mbytes), nu(mbytes);
        CK_HIP(hipMemcpy(mu.data(), dmu[i], mbytes, hipMemcpyDeviceToHost));
        CK_HIP(hipMemcpy(nu.data(), dnu[i], mbytes, hipMemcpyDeviceToHost));
        ok = ok && write_file(out + "/mu" + k, mu.data(), mbytes) && write_file(out + "/nu" + k, nu.data(), mbytes);
        if (L.quantized) {
            std::vector<float> ms((size_t)L.nblocks()), ns((size_t)L.nblocks());
            CK_HIP(hipMemcpy(ms.data(), dmus[i], ms.size() * 4, hipMemcpyDeviceToHost));
            CK_HIP(hipMemcpy(ns.data(), dnus[i], ns.size() * 4, hipMemcpyDeviceToHost));
            ok = ok && write_file(out + "/mus" + k, ms.data(), ms.size() * 4) &&
                 write_file(out + "/nus" + k, ns.data(), ns.size() * 4);
        }
        if (!ok) return 4;
        CK_HIP(hipFree(dp[i]));
        CK_HIP(hipFree(dg1[i]));
        CK_HIP(hipFree(dg2[i]));
        CK_HIP(hipFree(dmu[i]));
        CK_HIP(hipFree(dnu[i]));
        if (dmus[i]) CK_HIP(hipFree(dmus[i]));
        if (dnus[i]) CK_HIP(hipFree(dnus[i]));
    }
    CK_HIP(hipStreamDestroy(stream));
    std::printf("rf_c_host_step: %d leaves, 2 steps, %s\n", n, rf_version());
    return 0;
}

#ifdef RF_C_HOST_MAIN
int main(int argc, char** argv)
{
    if (argc != 2) {
        std::fprintf(stderr, "usage: %s <out_dir>\n", argv[0]);
        return 1;
    }
    return rf_c_host_step_run(argv[1]);
}
#endif
