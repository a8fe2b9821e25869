// d1hip: map-compiler kernels for MI355X (gfx950).
//
//   k_dist_rows — the all-pairs distance rows of a map file (gpu-d1/scripts/compile_corpus.py
//                 :30-52): BFS over 8-connected floor from each source cell, the distance of
//                 every cell as u16, 65535 where unreached. One wave per source; lane l owns
//                 map rows l and 64 + l as 80-bit bit rows, a layer is a dilation of the
//                 frontier rows (vertical neighbours by lane shuffles) masked by floor and not
//                 yet reached, and each newly reached cell's layer is stored.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/d1hip.h"
#include "d1_core.h"

namespace d1m {

using namespace d1;

__global__ __launch_bounds__(64) void k_dist_rows(const uint8_t *__restrict__ floor, const int16_t *__restrict__ sources,
                                                  int n, uint16_t *__restrict__ dist) {
    const int i = blockIdx.x, lane = threadIdx.x;
    if (i >= n) return;
    uint16_t *out = dist + (size_t)i * N;
    const bool has1 = lane < H - 64;
    // this lane's floor rows as bit rows
    auto row_bits = [&](int y) {
        uint32_t w[3] = {0, 0, 0};
        for (int x = 0; x < W; x++) w[x >> 5] |= (uint32_t)(floor[y * W + x] != 0) << (x & 31);
        return Row{w[0], w[1], w[2]};
    };
    const Row zero{0, 0, 0};
    const Row fl0 = row_bits(lane), fl1 = has1 ? row_bits(64 + lane) : zero;
    for (int x = 0; x < W; x++) {
        out[lane * W + x] = 65535;
        if (has1) out[(64 + lane) * W + x] = 65535;
    }
    const int src = sources[i];
    if (src < 0 || src >= N) return;   // no start cell: the whole row stays unreached
    const int sy = src / W, sx = src % W;
    const Row sbit = row_range(sx, sx);
    Row f0 = lane == sy ? sbit : zero, f1 = has1 && 64 + lane == sy ? sbit : zero;
    Row r0 = f0, r1 = f1;
    if (lane == sy) out[src] = 0;
    if (has1 && 64 + lane == sy) out[src] = 0;
    auto scatter = [&](int y, Row nw, int layer) {
        const uint32_t w[3] = {nw.a, nw.b, nw.c};
        for (int j = 0; j < 3; j++)
            for (uint32_t b = w[j]; b; b &= b - 1) out[y * W + 32 * j + __ffs(b) - 1] = (uint16_t)layer;
    };
    for (int layer = 1; layer < N; layer++) {
        const Row f1_0 = row_lane(f1, 0), f0_63 = row_lane(f0, 63);
        const Row u0 = row_sel(lane == 0, zero, row_up(f0)), d0 = row_sel(lane == 63, f1_0, row_dn(f0));
        const Row u1 = row_sel(lane == 0, f0_63, row_up(f1)), d1r = row_sel(lane >= H - 65, zero, row_dn(f1));
        const Row n0 = row_andn(row_and(dilate(f0, u0, d0), fl0), r0);
        const Row n1 = has1 ? row_andn(row_and(dilate(f1, u1, d1r), fl1), r1) : zero;
        r0 = row_or(r0, n0);
        r1 = row_or(r1, n1);
        f0 = n0;
        f1 = n1;
        scatter(lane, n0, layer);
        if (has1) scatter(64 + lane, n1, layer);
        if (!ballot(row_any(n0) || row_any(n1))) break;
    }
}

}  // namespace d1m

extern "C" int d1_distance_rows(const uint8_t *floor, const int16_t *sources, int n, uint16_t *dist, void *stream) {
    if (n < 0 || (n && (!floor || !sources || !dist))) return D1_E_ARG;
    if (n == 0) return 0;
    hipLaunchKernelGGL(d1m::k_dist_rows, dim3(n), dim3(64), 0, (hipStream_t)stream, floor, sources, n, dist);
    return (int)hipGetLastError();
}
