// The oracle's composed adapter chain (oracle/chain.cpp) against its sequential merge, with the
// cases and inputs of the reference's tests/lora_compose_test.cpp:54-257: the same targets, the same
// std::mt19937 seeds and normal distributions, the same adapter specs and chains, the same error
// measure (max |merge - functional| / rms(merge) < 1e-5 per target) and the same check that two dora
// adapters do not commute. The -xs families of that test are not part of this path (lora and
// dora-rows only), so their cases are left out. Also checks that the merge of a single dora-rows
// adapter equals the training oracle's materialised W_eff. Prints "chain_test: ok".
#include "oracle.h"

#include <cmath>
#include <cstdio>
#include <random>
#include <string>
#include <vector>

namespace {

int fails = 0;
void expect(bool ok, const std::string& what) {
    if (!ok) {
        std::printf("FAIL: %s\n", what.c_str());
        ++fails;
    }
}

struct Target {
    std::string stem;
    int64_t in, out;
};
const std::vector<Target> kTargets = {{"dit.0.self.qkv", 8, 6}, {"dit.0.ff.up", 6, 10}, {"dit.1.self.out", 10, 4}};

struct Spec {
    bool dora;
    int rank;
    float alpha, strength;
    bool skip_solo;
};

// one adapter's tensors per target, drawn like make_adapter_specs (lora_compose_test.cpp:84-128)
struct AdTensors {
    std::vector<std::vector<float>> A, B, mag;   // per target; empty when the target is skipped
};

AdTensors make_adapter(const Spec& sp, uint32_t seed, const std::vector<std::vector<float>>& base) {
    AdTensors t;
    std::mt19937 r(seed);
    std::normal_distribution<float> n(0.0f, 0.4f);
    for (size_t ti = 0; ti < kTargets.size(); ++ti) {
        const Target& tg = kTargets[ti];
        t.A.emplace_back();
        t.B.emplace_back();
        t.mag.emplace_back();
        if (sp.skip_solo && tg.stem == "dit.1.self.out") continue;
        // ggml lora_A ne = [in, rank] = host A [rank][in]; lora_B ne = [rank, out] = host B [out][rank]
        t.A.back().resize((size_t)(tg.in * sp.rank));
        t.B.back().resize((size_t)(sp.rank * tg.out));
        for (float& v : t.A.back()) v = n(r);
        for (float& v : t.B.back()) v = n(r);
        if (sp.dora) {
            t.mag.back().resize((size_t)tg.out);
            for (int64_t o = 0; o < tg.out; ++o) {
                double s = 0;
                for (int64_t i = 0; i < tg.in; ++i) {
                    const float v = base[ti][(size_t)(o * tg.in + i)];
                    s += (double)v * v;
                }
                t.mag.back()[(size_t)o] = (float)std::sqrt(s) * 1.15f + 0.05f;
            }
        }
    }
    return t;
}

std::vector<orc_chain_adapter> chain_for(const std::vector<Spec>& specs, const std::vector<AdTensors>& ads, size_t ti) {
    std::vector<orc_chain_adapter> c;
    for (size_t a = 0; a < specs.size(); ++a) {
        if (ads[a].A[ti].empty()) continue;   // this adapter does not target ti
        c.push_back({specs[a].dora ? 1 : 0, specs[a].rank, specs[a].alpha, specs[a].strength, ads[a].A[ti].data(),
                     ads[a].B[ti].data(), specs[a].dora ? ads[a].mag[ti].data() : nullptr});
    }
    return c;
}

}  // namespace

int main() {
    std::mt19937 rng(20260730);
    std::normal_distribution<float> nd(0.0f, 0.5f);
    const int64_t SEQ = 5;
    std::vector<std::vector<float>> base, xs;
    for (const Target& t : kTargets) {
        base.emplace_back((size_t)(t.in * t.out));
        for (float& v : base.back()) v = nd(rng);
    }
    for (const Target& t : kTargets) {
        xs.emplace_back((size_t)(t.in * SEQ));
        for (float& v : xs.back()) v = nd(rng);
    }

    auto run_case = [&](const std::string& label, const std::vector<Spec>& specs) {
        std::vector<AdTensors> ads;
        for (size_t i = 0; i < specs.size(); ++i) ads.push_back(make_adapter(specs[i], 7000u + (uint32_t)i * 31u, base));
        for (size_t ti = 0; ti < kTargets.size(); ++ti) {
            const Target& t = kTargets[ti];
            const std::vector<orc_chain_adapter> c = chain_for(specs, ads, ti);
            std::vector<float> weff((size_t)(t.in * t.out)), ref((size_t)(SEQ * t.out)), fun(ref.size());
            orc_chain_merge(base[ti].data(), t.in, t.out, (int)c.size(), c.data(), weff.data());
            // reference output: mul_mat(W_eff, x) (x [SEQ][in] token-major)
            orc_gemm_nt(xs[ti].data(), weff.data(), ref.data(), SEQ, t.out, t.in);
            orc_chain_forward(xs[ti].data(), SEQ, base[ti].data(), t.in, t.out, (int)c.size(), c.data(), nullptr,
                              fun.data());
            double sumsq = 0.0, maxabs = 0.0;
            for (size_t k = 0; k < ref.size(); ++k) {
                sumsq += (double)ref[k] * ref[k];
                maxabs = std::fmax(maxabs, std::fabs((double)ref[k] - fun[k]));
            }
            const double err = maxabs / std::sqrt(sumsq / (double)ref.size());
            expect(err < 1e-5, label + " @ " + t.stem + " (err " + std::to_string(err) + ")");
        }
    };

    const Spec dora{true, 2, 4.0f, 1.0f, false}, dora2{true, 4, 8.0f, 1.0f, false}, plain{false, 2, 4.0f, 1.0f, false};
    const Spec doraS{true, 2, 4.0f, 0.6f, false}, plainS{false, 3, 6.0f, 1.7f, false};
    const Spec doraSolo{true, 2, 4.0f, 1.0f, true};
    run_case("1x dora-rows", {dora});
    run_case("1x lora", {plain});
    run_case("2x dora-rows", {dora, dora2});
    run_case("3x dora-rows", {dora, dora2, doraS});
    run_case("2x lora", {plain, plainS});
    run_case("lora then dora-rows", {plain, dora});
    run_case("dora-rows then lora", {dora, plain});
    run_case("dora, lora, dora", {dora, plainS, dora2});
    run_case("2x dora, strengths", {doraS, dora2});
    run_case("dora + dora(skips one)", {dora, doraSolo});
    run_case("dora(skips one) + dora", {doraSolo, dora});
    // a strength-0 adapter is the identity (skipped, as in the merge path)
    run_case("dora, zero-strength dora", {dora, Spec{true, 4, 8.0f, 0.0f, false}});

    // the chain does not commute (lora_compose_test.cpp:220-257): two different dora adapters
    {
        auto composed = [&](const std::vector<Spec>& specs) {
            std::vector<AdTensors> ads;
            for (size_t i = 0; i < specs.size(); ++i) ads.push_back(make_adapter(specs[i], 4242u + (uint32_t)i * 17u, base));
            const Target& t = kTargets[0];
            const std::vector<orc_chain_adapter> c = chain_for(specs, ads, 0);
            std::vector<float> y((size_t)(SEQ * t.out));
            orc_chain_forward(xs[0].data(), SEQ, base[0].data(), t.in, t.out, (int)c.size(), c.data(), nullptr, y.data());
            return y;
        };
        const std::vector<float> ab = composed({dora, dora2}), ba = composed({dora2, dora});
        double maxrel = 0.0;
        for (size_t k = 0; k < ab.size(); ++k)
            maxrel = std::fmax(maxrel, std::fabs((double)ab[k] - ba[k]) / (std::fabs((double)ab[k]) + 1e-4));
        expect(maxrel > 1e-3, "dora chain does not commute (order is respected)");
    }

    // one dora-rows adapter: the merge equals the training oracle's materialised W_eff
    {
        const Target& t = kTargets[1];
        const AdTensors a = make_adapter(dora, 99u, base);
        const orc_chain_adapter c{1, dora.rank, dora.alpha, 1.0f, a.A[1].data(), a.B[1].data(), a.mag[1].data()};
        std::vector<float> m((size_t)(t.in * t.out)), e(m.size());
        orc_chain_merge(base[1].data(), t.in, t.out, 1, &c, m.data());
        orc_effective_weight(base[1].data(), t.in, t.out, a.A[1].data(), a.B[1].data(), a.mag[1].data(), dora.rank,
                             dora.alpha, 1, e.data());
        double worst = 0.0;
        for (size_t k = 0; k < m.size(); ++k) worst = std::fmax(worst, std::fabs((double)m[k] - e[k]) / (std::fabs((double)e[k]) + 1e-6));
        expect(worst < 1e-6, "single dora-rows merge == materialised W_eff (" + std::to_string(worst) + ")");
    }

    if (fails) return 1;
    std::printf("chain_test: ok\n");
    return 0;
}
