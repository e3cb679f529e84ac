// Wave64 / workgroup primitives for gfx950 (CDNA4): ballot-based digit matching
// and prefix scans.
#pragma once

#include "gs_common.h"

namespace gs {

__device__ __forceinline__ uint64_t lanemask_lt() {
    const unsigned lane = __lane_id();
    return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// Mask of the lanes in `active` whose `digit` (nbits wide) equals this lane's.
// nbits ballots; every lane of the wave must execute it.
__device__ __forceinline__ uint64_t match_digit(uint32_t digit, int nbits, uint64_t active) {
    uint64_t peers = active;
    for (int b = 0; b < nbits; ++b) {
        const bool bit = (digit >> b) & 1u;
        const uint64_t m = __ballot(bit);
        peers &= bit ? m : ~m;
    }
    return peers;
}

template <typename T>
__device__ __forceinline__ T wave_inclusive_scan(T x) {
    const int lane = __lane_id();
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const T t = __shfl_up(x, o, kWave);
        if (lane >= o) x += t;
    }
    return x;
}

// Exclusive scan across a workgroup of NT threads (NT multiple of 64, <= 1024).
// `tmp` must hold NT/64 + 1 elements of LDS.  Returns the exclusive prefix and
// writes the workgroup total to `total`.  Contains __syncthreads().
template <typename T, int NT>
__device__ __forceinline__ T block_exclusive_scan(T x, T *tmp, T &total) {
    constexpr int kWaves = NT / kWave;
    const int lane = __lane_id();
    const int wave = threadIdx.x / kWave;
    const T incl = wave_inclusive_scan(x);
    if (lane == kWave - 1) tmp[wave] = incl;
    __syncthreads();
    if (threadIdx.x == 0) {
        T run = 0;
        for (int w = 0; w < kWaves; ++w) {
            const T t = tmp[w];
            tmp[w] = run;
            run += t;
        }
        tmp[kWaves] = run;
    }
    __syncthreads();
    total = tmp[kWaves];
    const T res = tmp[wave] + incl - x;
    __syncthreads();
    return res;
}

}  // namespace gs
