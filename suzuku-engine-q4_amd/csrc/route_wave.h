// One wave's softmax + top-k over a token's router logits: shared by the
// routing kernels (route.hip) and the decode layer's gate/up blocks, which
// rank the logits themselves when the layer is given logits instead of
// device lists, so that both give the same picks and weights bit for bit.
// Ranking follows q4_topk (src/q4_quant.c:728-750).
#pragma once
#include <math.h>
#include <stdint.h>

#include "q4mi_common.h"

namespace q4mi {

// float -> uint key with the same order (negatives included)
__device__ inline uint32_t f2key(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// inverse of f2key
__device__ inline float key2f(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Wave maximum of an unsigned value (DPP row shifts, then the row
// broadcasts; the total lands in lane 63), returned to every lane.
__device__ inline uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, true));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, true));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, true));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, true));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, true));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, true));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// One wave's softmax + top-k of one token's logits (NJ logits per lane, so
// up to 64 * NJ experts): picks in rank order land in s_id[0..tk), their
// probabilities in s_p; returns tk = min(topk, n_exp).
template <int NJ>
__device__ inline uint32_t route_wave(const float *__restrict__ lg, uint32_t n_exp, uint32_t topk,
                                      uint32_t lane, int32_t *s_id, float *s_p) {
    float v[NJ];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const uint32_t i = lane + 64u * j;
        v[j] = i < n_exp ? lg[i] : -INFINITY;
        mx = fmaxf(mx, v[j]);
    }
    mx = key2f(wave_max_u32(f2key(mx)));   // DPP tree, no LDS round trips
    float e[NJ], s = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        e[j] = (lane + 64u * j) < n_exp ? expf(v[j] - mx) : 0.f;
        s += e[j];
    }
    s = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, q4mi_rsum<64>(s)), 63));
    const float inv = s > 0.f ? __fdiv_rn(1.f, s) : 0.f;
    uint32_t alive = 0;
#pragma unroll
    for (int j = 0; j < NJ; j++)
        if ((lane + 64u * j) < n_exp) alive |= 1u << j;
    const uint32_t tk = topk < n_exp ? topk : n_exp;
    // p >= 0, so its key is its bit pattern with the top bit set (a live
    // zero still outranks a dead entry's key 0)
    uint32_t pk[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) pk[j] = __float_as_uint(e[j] * inv) | 0x80000000u;
    for (uint32_t k = 0; k < tk; k++) {
        // this lane's best alive entry: largest key, smallest index on ties
        uint32_t bk = 0, bj = 0;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const uint32_t key = (alive & (1u << j)) ? pk[j] : 0u;
            if (key > bk) {
                bk = key;
                bj = (uint32_t)j;
            }
        }
        // wave max of the keys, then the smallest index holding it (two DPP
        // reductions; the min runs as a max of complements)
        const uint32_t m = wave_max_u32(bk);
        const uint32_t wi = ~wave_max_u32(bk == m && bk ? ~(lane + 64u * bj) : 0u);
        if ((wi & 63u) == lane) {
            const uint32_t j = wi >> 6;
            alive &= ~(1u << j);
            float pe = 0.f;
#pragma unroll
            for (int jj = 0; jj < NJ; jj++)
                if ((uint32_t)jj == j) pe = e[jj];
            s_id[k] = (int32_t)wi;
            s_p[k] = pe * inv;
        }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    return tk;
}

// Renormalized weight of pick k: p_k * (1 / sum of the tk picked p, summed
// in rank order), as q4_topk(renorm) computes it.
__device__ inline float route_inv_sum(const float *s_p, uint32_t tk) {
    float sk = 0.f;
    for (uint32_t k = 0; k < tk; k++) sk += s_p[k];
    return sk > 0.f ? __fdiv_rn(1.f, sk) : 0.f;
}

}  // namespace q4mi
