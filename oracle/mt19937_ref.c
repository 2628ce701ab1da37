/*
 * Textbook MT19937 (M. Matsumoto, T. Nishimura, "Mersenne Twister: a
 * 623-dimensionally equidistributed uniform pseudorandom number generator",
 * ACM TOMACS 8(1), 1998), 32-bit variant with the standard integer seeding
 * x[0] = seed, x[i] = 1812433253 * (x[i-1] ^ (x[i-1] >> 30)) + i.
 *
 * TEST INFRASTRUCTURE ONLY (part of oracle/).  It pins the QJL G matrix the
 * reference draws with torch.randint(0, 2, (64, 128), generator=g) on a CPU
 * torch.Generator seeded with (user_id % 1024) ^ head
 * (reference omnistack_rs/kernels/quantize.py:410-414, :293-295): bit k of
 * that draw is the low bit of the k-th MT19937 output.
 */
#include <stdint.h>
#include <stddef.h>

#define MT_N 624
#define MT_M 397

typedef struct {
    uint32_t s[MT_N];
    int i;
} mt_state;

static void mt_seed(mt_state *m, uint32_t seed) {
    m->s[0] = seed;
    for (int k = 1; k < MT_N; ++k)
        m->s[k] = 1812433253u * (m->s[k - 1] ^ (m->s[k - 1] >> 30)) + (uint32_t)k;
    m->i = MT_N;
}

static uint32_t mt_next(mt_state *m) {
    if (m->i >= MT_N) {
        for (int k = 0; k < MT_N; ++k) {
            uint32_t y = (m->s[k] & 0x80000000u) | (m->s[(k + 1) % MT_N] & 0x7fffffffu);
            uint32_t v = m->s[(k + MT_M) % MT_N] ^ (y >> 1);
            if (y & 1u) v ^= 0x9908b0dfu;
            m->s[k] = v;
        }
        m->i = 0;
    }
    uint32_t y = m->s[m->i++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}

/* Writes the first n raw 32-bit outputs for `seed`. */
void oracle_mt19937_raw(uint32_t seed, uint32_t *out, size_t n) {
    mt_state m;
    mt_seed(&m, seed);
    for (size_t k = 0; k < n; ++k) out[k] = mt_next(&m);
}

/* Writes n low bits (0/1 bytes) of the first n outputs for `seed`. */
void oracle_mt19937_bits(uint32_t seed, uint8_t *out, size_t n) {
    mt_state m;
    mt_seed(&m, seed);
    for (size_t k = 0; k < n; ++k) out[k] = (uint8_t)(mt_next(&m) & 1u);
}
