// TEST INFRASTRUCTURE ONLY — drives the reference's own rule core, gpu-d1/src/sim.h,
// compiled from where it lies (see oracle/Makefile), to produce golden vectors that
// pin the CPU restatement in oracle/d1_oracle.c. Writes one JSON document to stdout.
//
//   simref <fixture.bin>
//
// Sections:
//   mix   splitmix64 finaliser on fixed inputs                   (sim.h:15-20)
//   rng   PCG32 op streams: next / r(b) / avg(n) / round(n,d)     (sim.h:21-60)
//   wait  the monster-wait workload of gpu-d1/src/bench.cu:151-184 on map 1057:
//         per-step world digests for scan and heap scheduling    (sim.h:93-122,130-295)
#include "sim.h"
#include <cstdio>
#include <cstring>
#include <fstream>
#include <string>
#include <vector>
using namespace sim;

static uint32_t fmix32(uint32_t h) {
    h ^= h >> 16; h *= 0x85ebca6bu; h ^= h >> 13; h *= 0xc2b2ae35u; h ^= h >> 16;
    return h;
}
static uint32_t term(uint32_t w, uint32_t i) { return fmix32(w ^ (i * 0x9E3779B9u)); }

struct Fixture {
    Config c{};
    std::vector<uint8_t> floor;
    std::vector<uint16_t> dist;
    std::vector<uint32_t> los;
    std::vector<int16_t> starts;
    explicit Fixture(const char *path) {
        std::ifstream f(path, std::ios::binary);
        uint32_t magic = 0;
        int header[8];
        f.read((char *)&magic, 4);
        f.read((char *)header, sizeof header);
        c.player = header[0]; c.hp = header[1]; c.ac100 = header[2]; c.ev100 = header[3];
        c.sh100 = header[4]; c.shield_limit = header[5]; c.regen = header[6]; c.repair = 1;
        for (int j = 0; j < 2; j++) {
            int ac = c.ac100 / 100 + j, g = 0;
            while ((g + 1) * (g + 1) * (g + 1) * (g + 1) <= 65536 * ac) g++;
            c.gdr[j] = g;
        }
        f.read((char *)c.kinds, sizeof c.kinds);
        floor.resize(N); dist.resize(N); los.resize(N * 10); starts.resize(2 * MAX);
        f.read((char *)floor.data(), N);
        f.read((char *)dist.data(), N * 2);
        f.read((char *)los.data(), N * 40);
        f.read((char *)starts.data(), MAX * 4);
        if (!f || magic != 0x44314750) { fprintf(stderr, "bad fixture\n"); std::exit(1); }
    }
};

static uint64_t lcg(uint64_t &x) { x = x * 6364136223846793005ULL + 1442695040888963407ULL; return x >> 33; }

int main(int argc, char **argv) {
    if (argc < 2) { fprintf(stderr, "usage: simref fixture.bin\n"); return 2; }
    Fixture fx(argv[1]);
    printf("{\n\"mix\": [");
    const uint64_t xs[] = {0, 1, 2, 91, 123, 1057, 0xffffffffffffffffULL, 0x123456789abcdefULL};
    for (int i = 0; i < 8; i++) printf("%s[\"%llu\", \"%llu\"]", i ? ", " : "", (unsigned long long)xs[i], (unsigned long long)mix(xs[i]));
    printf("],\n\"rng\": [");
    uint64_t q = 7;
    for (int s = 0; s < 6; s++) {
        uint64_t seed = s < 3 ? mix(91 + s) : lcg(q) << 20 ^ lcg(q), seq = s + 1;
        RNG g;
        g.seed(seed, seq);
        printf("%s\n{\"seed\": \"%llu\", \"seq\": %llu, \"ops\": [", s ? "," : "", (unsigned long long)seed, (unsigned long long)seq);
        std::vector<int> ops, args, res;
        for (int k = 0; k < 400; k++) {
            int op = (int)(lcg(q) % 4), arg;
            if (op == 0) arg = 0;
            else if (op == 1) { int kind = (int)(lcg(q) % 4); arg = kind == 0 ? (int)(lcg(q) % 3) : kind == 1 ? 2 + (int)(lcg(q) % 30) : kind == 2 ? 100 + (int)(lcg(q) % 2000) : (int)(lcg(q) % 0x7fffffff); }
            else if (op == 2) arg = 1 + (int)(lcg(q) % 40);
            else { int n = (int)(lcg(q) % 1200), d = 1 + (int)(lcg(q) % 120); arg = n << 8 | d; }
            int r;
            if (op == 0) r = (int)g.next();
            else if (op == 1) r = g.r(arg);
            else if (op == 2) r = g.avg(arg);
            else r = g.round(arg >> 8, arg & 255);
            ops.push_back(op); args.push_back(arg); res.push_back(r);
        }
        for (size_t k = 0; k < ops.size(); k++) printf("%s%d", k ? "," : "", ops[k]);
        printf("], \"args\": [");
        for (size_t k = 0; k < args.size(); k++) printf("%s%d", k ? "," : "", args[k]);
        printf("], \"results\": [");
        for (size_t k = 0; k < res.size(); k++) printf("%s%d", k ? "," : "", res[k]);
        printf("], \"final_state\": \"%llu\"}", (unsigned long long)g.state);
    }
    printf("],\n\"config\": [%d,%d,%d,%d,%d,%d,%d,%d,%d,%d,%d], \"kinds\": [", 0, fx.c.player, fx.c.hp,
           fx.c.ac100, fx.c.ev100, fx.c.sh100, fx.c.shield_limit, fx.c.regen, fx.c.repair, fx.c.gdr[0], fx.c.gdr[1]);
    for (int k = 0; k < 6; k++)
        printf("%s%d,%d,%d,%d", k ? "," : "", fx.c.kinds[k].speed, fx.c.kinds[k].damage, fx.c.kinds[k].tohit, fx.c.kinds[k].bypass);
    printf("],\n\"wait\": [");
    Map m{fx.floor.data(), fx.dist.data(), fx.los.data(), fx.starts.data()};
    bool firstcase = true;
    const int counts[] = {1, 8, 32, 64};
    for (int count : counts)
        for (int scenario = 0; scenario < 3; scenario++)
            for (int heap = 0; heap < 2; heap++)
                for (int world = 0; world < 3; world++) {
                    uint64_t seed = 91;
                    int steps = 257;
                    Config c = fx.c;
                    c.count = count;
                    std::vector<int16_t> pos(count), energy(count), occ(N, -1);
                    Access a{pos.data(), energy.data(), occ.data(), 0, 1, count, true};
                    World w{};
                    w.rng.seed(mix(seed + world), world + 1);
                    w.fixture = scenario == 1 ? 1 : scenario == 2 ? world % 2 : 0;
                    reset(w, a, c, m, true);
                    int prewarm = scenario == 2 ? (world * 7) % 32 : 0;
                    for (int k = 0; k < prewarm; k++) step<false>(w, a, c, m);
                    printf("%s\n{\"count\": %d, \"scenario\": %d, \"fixture\": %d, \"heap\": %d, \"world\": %d, \"seed\": %llu, \"prewarm\": %d, \"trace\": [",
                           firstcase ? "" : ",", count, scenario, w.fixture, heap, world, (unsigned long long)seed, prewarm);
                    firstcase = false;
                    for (int k = 0; k < steps; k++) {
                        if (heap) step<true>(w, a, c, m); else step<false>(w, a, c, m);
                        uint32_t h = term((uint32_t)w.hp, 0) + term((uint32_t)w.regen, 1) + term((uint32_t)w.blocks, 2) +
                                     term((uint32_t)w.episode, 3) + term((uint32_t)w.rng.state, 4) +
                                     term((uint32_t)(w.rng.state >> 32), 5);
                        for (int i = 0; i < count; i++)
                            h += term((uint16_t)a.pos(i) | (uint32_t)(uint16_t)a.energy(i) << 16, 100 + i);
                        printf("%s%d", k ? "," : "", (int32_t)h);
                    }
                    printf("]}");
                }
    printf("\n]\n}\n");
    return 0;
}
