// Positions of the reference's neighbor-list correctness cases
// (reference tests/test_neighbor_list.cu:18-27 generate_positions, :70-81 box from
// density, :264-266 the cases N = 100, 500, 1000 at density 0.05, cutoff 5.0):
// std::mt19937(42) with std::uniform_real_distribution<float>(0, box), box =
// cbrtf(N / density), x, y, z per atom in turn.  Prints JSON on stdout with every
// float as a 9-significant-digit decimal (round-trips exactly to fp32).
// Built and run by tests/golden/make_nl_fixtures.py (g++, libstdc++).
#include <cmath>
#include <cstdio>
#include <random>

int main() {
    const int cases[3] = {100, 500, 1000};
    const float density = 0.05f;
    std::printf("{\"source\": \"std::mt19937(42) + uniform_real_distribution<float>(0, box), "
                "box = cbrtf(N / 0.05f)\", \"density\": 0.05, \"cutoff\": 5.0, \"cases\": [");
    for (int c = 0; c < 3; ++c) {
        const int n = cases[c];
        const float box = cbrtf((float)n / density);
        std::mt19937 gen(42);
        std::uniform_real_distribution<float> dist(0.0f, box);
        std::printf("%s{\"N\": %d, \"box\": %.9g, \"positions\": [", c ? ", " : "", n, box);
        for (int i = 0; i < n; ++i) {
            const float x = dist(gen), y = dist(gen), z = dist(gen);
            std::printf("%s[%.9g, %.9g, %.9g]", i ? ", " : "", x, y, z);
        }
        std::printf("]}");
    }
    std::printf("]}\n");
    return 0;
}
