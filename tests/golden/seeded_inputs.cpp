// tests/golden/seeded_inputs.cpp - writes the seeded inputs of the reference's own parity tests, drawn with the same
// generators in the same order (libstdc++'s std::mt19937 and std::normal_distribution<float>), as raw little-endian
// arrays into the directory given as argv[1]:
//   router_cases.f32      src/kernels/router_top10_parity.cpp:138-170: 4 x 64 rows of 512 logits (normal, all
//                         equal, 12-way tie, dominant), then the first 768 of its 8192 variant rows (:172-184)
//   plan_ids.i32          src/kernels/resident_plan_parity.cpp:48-56: for n = 1..80, pools 3, 12, 40, 512: n ids each
//   router256.f32         src/kernels/native_multi_parity.cpp:53-87 then :91-96: the 3 x 256 logits of its non-512
//                         router case (the draws of the multi-router cases before it are made and discarded)
// Built and run by tests/golden/make_golden.py; only the data it writes is committed.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <random>
#include <string>
#include <vector>

static void put(const std::string& path, const void* p, size_t bytes) {
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f || std::fwrite(p, 1, bytes, f) != bytes) { std::perror(path.c_str()); std::exit(1); }
    std::fclose(f);
}

int main(int argc, char** argv) {
    if (argc < 2) return 2;
    const std::string dir = argv[1];
    {   // router_top10_parity
        const int NE = 512, NT = 64;
        std::mt19937 rng(2024);
        std::normal_distribution<float> gauss(0.0f, 1.0f);
        std::vector<float> out;
        std::vector<float> a((size_t)NT * NE);
        for (auto& v : a) v = gauss(rng);
        out.insert(out.end(), a.begin(), a.end());
        std::vector<float> b((size_t)NT * NE, 0.5f);
        out.insert(out.end(), b.begin(), b.end());
        std::vector<float> c((size_t)NT * NE);
        for (int t = 0; t < NT; ++t)
            for (int e = 0; e < NE; ++e) c[(size_t)t * NE + e] = (e < 12) ? 2.0f : gauss(rng);
        out.insert(out.end(), c.begin(), c.end());
        std::vector<float> d((size_t)NT * NE, 0.0f);
        for (int t = 0; t < NT; ++t) d[(size_t)t * NE + (t % NE)] = 20.0f;
        out.insert(out.end(), d.begin(), d.end());
        const int NV = 8192, KEEP = 768;
        std::vector<float> v((size_t)NV * NE);
        std::uniform_int_distribution<int> pick(0, NE - 1);
        for (int t = 0; t < NV; ++t) {
            float* row = &v[(size_t)t * NE];
            const int kind = t % 6;
            for (int e = 0; e < NE; ++e) row[e] = kind == 1 ? 0.5f : gauss(rng) * (kind == 5 ? 8.0f : 1.0f);
            if (kind == 2)
                for (int e = 0; e < 12; ++e) row[pick(rng)] = 2.0f;
            if (kind == 3)
                for (int e = 0; e < 16; ++e) row[e] = 1.0f + (float)e * 1e-7f;
            if (kind == 4) row[t % NE] = 20.0f;
            if (t % 97 == 0) row[pick(rng)] = std::nanf("");
        }
        out.insert(out.end(), v.begin(), v.begin() + (size_t)KEEP * NE);
        put(dir + "/router_cases.f32", out.data(), out.size() * 4);
    }
    {   // resident_plan_parity
        std::mt19937 rng(783);
        std::vector<int32_t> all;
        for (int n = 1; n <= 80; ++n)
            for (int variant = 0; variant < 4; ++variant) {
                const int pool = variant == 0 ? 3 : (variant == 1 ? 12 : (variant == 2 ? 40 : 512));
                for (int i = 0; i < n; ++i) all.push_back((int32_t)((rng() % pool) * (512 / pool)));
            }
        put(dir + "/plan_ids.i32", all.data(), all.size() * 4);
    }
    {   // native_multi_parity
        std::mt19937 rng(783);
        std::normal_distribution<float> gauss(0.0f, 1.0f);
        for (int mode = 0; mode < 3; ++mode)
            for (int n = 1; n <= 19; ++n) {
                std::vector<float> lg((size_t)n * 512);
                for (auto& v : lg) v = gauss(rng) * 2.0f;
                if (mode == 2)
                    for (int t = 0; t < n; ++t) (void)(rng() % 512);
            }
        const int n = 3, NE = 256;
        std::vector<float> lg((size_t)n * NE);
        for (auto& v : lg) v = gauss(rng) * 2.0f;
        put(dir + "/router256.f32", lg.data(), lg.size() * 4);
    }
    return 0;
}
