/* TEST INFRASTRUCTURE ONLY — host sanitizer run of the CPU restatements (the reference ran
 * ASan/UBSan on its host path, gpu-d1/RESULTS.md:92). Built by `make -C oracle asan` with
 * -fsanitize=address,undefined together with d1_oracle.c and learn_oracle.c; reads the raw
 * inputs oracle/asan_inputs.py wrote and runs every env rule set (BASELINE generated levels,
 * the 40-monster stress roster, the stairs task on map 1057 with 24 and 8 monsters, v1
 * kill-all) for 300 steps, the learning task (both clump modes, three maps) for 300 steps,
 * and the wait workload, with random and controller actions. Any sanitizer report stops the
 * run with a non-zero status. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "d1_oracle.h"
#include "../include/d1learn.h"

static void *slurp(const char *dir, const char *name, size_t *len) {
    char path[1024];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE *f = fopen(path, "rb");
    if (!f) { fprintf(stderr, "missing %s\n", path); exit(2); }
    fseek(f, 0, SEEK_END);
    long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    void *buf = malloc(n > 0 ? (size_t)n : 1);
    if (fread(buf, 1, (size_t)n, f) != (size_t)n) { fprintf(stderr, "short read %s\n", path); exit(2); }
    fclose(f);
    if (len) *len = (size_t)n;
    return buf;
}

static uint64_t lcg = 0x9E3779B97F4A7C15ULL;
static int draw(int bound) {
    lcg = lcg * 6364136223846793005ULL + 1442695040888963407ULL;
    return (int)((lcg >> 33) % (uint64_t)bound);
}

int main(int argc, char **argv) {
    const char *dir = argc > 1 ? argv[1] : ".";
    size_t n_ends, n_cfg;
    uint8_t *floor = slurp(dir, "floor.bin", NULL), *cells = slurp(dir, "cells.bin", NULL);
    int8_t *ends = slurp(dir, "ray_ends.bin", &n_ends);
    uint64_t *masks = slurp(dir, "ray_masks.bin", NULL);
    o_set_rays((int)(n_ends / 2), ends, masks);
    D1Config *cfgs = slurp(dir, "configs.bin", &n_cfg);
    const int ncfg = (int)(n_cfg / sizeof(D1Config)), n = 24, steps = 300;

    OState *st = calloc(n, sizeof(OState));
    uint8_t *obs = malloc((size_t)n * 1800);
    float *out = malloc((size_t)n * 8 * sizeof(float));
    uint32_t *hash = malloc((size_t)n * 4);
    int64_t *act = malloc((size_t)n * 8);
    uint8_t *active = malloc((size_t)n);
    for (int k = 0; k < ncfg; k++) {
        o_init(st, n, &cfgs[k], floor, cells, 17 + k, obs, hash, 1);
        long dones = 0;
        for (int t = 0; t < steps; t++) {
            for (int i = 0; i < n; i++) {
                act[i] = t % 3 ? draw(21) - 1 : o_heuristic(&st[i], &cfgs[k]);
                active[i] = (uint8_t)(draw(8) != 0);
            }
            o_step(st, n, &cfgs[k], act, obs, out, hash, t % 5 ? NULL : active, 1);
            for (int i = 0; i < n; i++) dones += out[i * 8 + 1] != 0.f;
        }
        printf("env config %d: %d worlds x %d steps, %ld episode ends\n", k, n, steps, dones);
    }

    /* the learning task on three maps, both placement modes */
    size_t nfloor, nncells;
    D1LTables t;
    t.floor = slurp(dir, "learn_floor.bin", &nfloor);
    t.cells = slurp(dir, "learn_cells.bin", NULL);
    t.index = slurp(dir, "learn_index.bin", NULL);
    t.distance = slurp(dir, "learn_distance.bin", NULL);
    t.map_ncells = slurp(dir, "learn_ncells.bin", &nncells);
    t.distance_offsets = slurp(dir, "learn_offsets.bin", NULL);
    t.los = slurp(dir, "learn_los.bin", NULL);
    t.n_maps = (int32_t)(nncells / 4);
    t.ncells = t.map_ncells[0];
    t.map_filter = -2;
    D1LConfig *lc = slurp(dir, "learn_config.bin", NULL);
    LState *ls = calloc(n, sizeof(LState));
    float *lobs = malloc((size_t)n * D1L_OBS * sizeof(float)), *lmask = malloc((size_t)n * D1L_ACTIONS * sizeof(float));
    float *lout = malloc((size_t)n * D1L_OUT * sizeof(float));
    for (int clump = 0; clump < 2; clump++) {
        lo_init(ls, n, lc, &t, 5 + clump, lobs, lmask, clump, 1);
        long dones = 0;
        for (int s = 0; s < steps; s++) {
            if (s % 2) for (int i = 0; i < n; i++) act[i] = draw(21) - 1;
            else lo_heuristic(ls, n, lc, &t, act, 1);
            for (int i = 0; i < n; i++) active[i] = (uint8_t)(draw(8) != 0);
            lo_step(ls, n, lc, &t, act, 2048, lobs, lmask, lout, s % 7 ? NULL : active, clump, 1);
            for (int i = 0; i < n; i++) dones += lout[i * D1L_OUT + 1] != 0.f;
        }
        printf("learning task clump %d: %d worlds x %d steps on %d maps, %ld episode ends\n", clump, n, steps,
               t.n_maps, dones);
    }

    /* the wait workload on map 1057 (stationary player at 3631, BFS distances from it) */
    uint16_t *dist = malloc(5600 * 2);
    int16_t starts[128];
    for (int p = 0; p < 5600; p++) dist[p] = 65535;
    {
        int16_t queue[5600];
        int head = 0, tail = 1;
        queue[0] = 3631;
        dist[3631] = 0;
        static const int DX[8] = {0, 1, 0, -1, 1, 1, -1, -1}, DY[8] = {-1, 0, 1, 0, -1, 1, 1, -1};
        while (head < tail) {
            int p = queue[head++];
            for (int d = 0; d < 8; d++) {
                int x = p % 80 + DX[d], y = p / 80 + DY[d], q = y * 80 + x;
                if (x < 0 || x >= 80 || y < 0 || y >= 70 || !floor[q] || dist[q] != 65535) continue;
                dist[q] = (uint16_t)(dist[p] + 1);
                queue[tail++] = (int16_t)q;
            }
        }
        int m = 0;
        for (int p = 0; p < 5600 && m < 128; p++)
            if (floor[p] && p != 3631 && dist[p] < 65535) starts[m++] = (int16_t)p;
    }
    const int32_t *cfg11 = (const int32_t *)lc;   /* sim::Config: count, player, hp, ..., gdr[2] */
    int32_t c11[11];
    memcpy(c11, cfg11, sizeof c11);
    c11[1] = 3631;
    int32_t *trace = malloc(257 * 4);
    for (int count = 1; count <= 64; count *= 4)
        for (int fixture = 0; fixture < 2; fixture++)
            o_wait_run(count, 257, 0, fixture, 7, (uint32_t)count, floor, dist, starts, c11, cfg11 + 11, 3, trace);
    printf("wait workload: 1-64 monsters x 257 steps\n");

    free(trace); free(dist); free(lout); free(lmask); free(lobs); free(ls); free(lc);
    free((void *)t.los); free((void *)t.distance_offsets); free((void *)t.map_ncells); free((void *)t.distance);
    free((void *)t.index); free((void *)t.cells); free((void *)t.floor);
    free(active); free(act); free(hash); free(out); free(obs); free(st); free(cfgs); free(masks); free(ends);
    free(cells); free(floor);
    puts("sanitizer run clean");
    return 0;
}
