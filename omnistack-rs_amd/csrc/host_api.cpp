// Host-side pieces of the C ABI: error reporting, version, QJL G bits.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <random>

#include "omnistack_amd.h"

namespace omni {

static thread_local char g_err[512] = "";

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

}  // namespace omni

extern "C" const char *omni_last_error(void) { return omni::g_err; }

extern "C" int omni_abi_version(void) { return 1; }

// G row i, column j = +1 iff the low bit of the (D*i + j)-th std::mt19937
// output is 1 — the same draw torch.randint(0, 2, (D/2, D), generator=g)
// makes on a CPU generator seeded with `seed` (quantize.py:410-414).
extern "C" int omni_qjl_g_bits(uint32_t seed, int head_dim, uint32_t *out_words) {
    if (!(head_dim == 128 || head_dim == 32)) {
        omni::set_error("omni_qjl_g_bits: head_dim must be 128 or 32, got %d", head_dim);
        return OMNI_EINVAL;
    }
    if (!out_words) {
        omni::set_error("omni_qjl_g_bits: out_words is NULL");
        return OMNI_EINVAL;
    }
    const int rows = head_dim / 2, words = head_dim / 32;
    std::mt19937 gen(seed);
    for (int i = 0; i < rows; ++i) {
        for (int w = 0; w < words; ++w) {
            uint32_t acc = 0;
            for (int b = 0; b < 32; ++b) acc |= (uint32_t)(gen() & 1u) << b;
            out_words[i * words + w] = acc;
        }
    }
    return OMNI_OK;
}
