/* Synthetic MoE layer contents, defined by a counter-based hash so that the
 * host (C, for the CPU checker and the CPU baseline) and the device (HIP, for
 * HBM-resident stacks that never cross PCIe) materialise identical bytes.
 *
 * Every value is a pure function of (seed, layer, expert, tensor, index):
 *   - packed int4 / int3 code bytes and int8 shared-expert bytes are uniform
 *     random bytes (uniform random bytes are uniform random nibbles and
 *     uniform random 3-bit codes of the packed bitstream);
 *   - scales and fp32 tensors use an Irwin-Hall(12) normal built from twelve
 *     16-bit uniforms whose sum is exact in integers and converted to float
 *     once, so host and device agree bit for bit.
 *
 * The distributions follow the workload definitions: router ~N(0,0.02),
 * shared-expert gate row ~N(0,0.02), group scales |N(0,0.01)|, int8 row scales
 * |N(0,0.01)|, activations ~N(0,1).
 *
 * Plain C99 for gcc; the same text compiles as HIP host+device code. */
#ifndef SW_SYNTH_H
#define SW_SYNTH_H

#include <stdint.h>

#if defined(__HIPCC__)
#define SW_HD __host__ __device__ static inline
#else
#define SW_HD static inline
#endif

enum {
    SW_T_ROUTER = 1,      /* f32 [E x H] */
    SW_T_SHARED_GATE = 2, /* f32 [1 x H], the shared-expert sigmoid gate row */
    SW_T_SH_GATE_Q = 3,   /* int8 [I_sh x H] */
    SW_T_SH_GATE_S = 4,   /* f32 [I_sh] */
    SW_T_SH_UP_Q = 5,
    SW_T_SH_UP_S = 6,
    SW_T_SH_DOWN_Q = 7,   /* int8 [H x I_sh] */
    SW_T_SH_DOWN_S = 8,   /* f32 [H] */
    SW_T_GATE_Q = 9,      /* packed codes [I x rb_h] */
    SW_T_GATE_S = 10,     /* f32 [I x ng_h] */
    SW_T_UP_Q = 11,
    SW_T_UP_S = 12,
    SW_T_DOWN_Q = 13,     /* packed codes [H x rb_i] */
    SW_T_DOWN_S = 14,     /* f32 [H x ng_i] */
    SW_T_X = 15           /* f32 activations */
};

#define SW_GOLDEN 0x9e3779b97f4a7c15ULL

/* splitmix64 output function */
SW_HD uint64_t sw_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

SW_HD uint64_t sw_key(uint64_t seed, uint32_t layer, uint32_t expert,
                      uint32_t tensor) {
    uint64_t k = sw_mix64(seed + SW_GOLDEN);
    k = sw_mix64(k ^ (((uint64_t)layer << 32) | (uint64_t)expert));
    return sw_mix64(k + (uint64_t)tensor * SW_GOLDEN);
}

SW_HD uint64_t sw_word(uint64_t key, uint64_t i) {
    return sw_mix64(key + (i + 1) * SW_GOLDEN);
}

SW_HD uint8_t sw_byte(uint64_t key, uint64_t i) {
    return (uint8_t)(sw_word(key, i >> 3) >> (8 * (unsigned)(i & 7)));
}

/* int8 in [-127, 127] */
SW_HD int8_t sw_i8(uint64_t key, uint64_t i) {
    return (int8_t)((int)(sw_byte(key, i) % 255u) - 127);
}

/* Irwin-Hall(12) standard normal: the integer sum is exact and
 * |sum - mean| < 2^24, so the conversion and the power-of-two scale are
 * exact and the result is identical on every IEEE-754 machine. */
SW_HD float sw_normal(uint64_t key, uint64_t i) {
    int64_t s = 0;
    for (int w = 0; w < 3; w++) {
        uint64_t h = sw_word(key, 3 * i + (uint64_t)w);
        s += (int64_t)(h & 0xffff) + (int64_t)((h >> 16) & 0xffff) +
             (int64_t)((h >> 32) & 0xffff) + (int64_t)(h >> 48);
    }
    return (float)(s - 393210) * (1.0f / 65536.0f);
}

SW_HD float sw_normal_sigma(uint64_t key, uint64_t i, float sigma) {
    return sw_normal(key, i) * sigma;
}

SW_HD float sw_abs_normal_sigma(uint64_t key, uint64_t i, float sigma) {
    float v = sw_normal(key, i) * sigma;
    return v < 0.0f ? -v : v;
}

#endif
