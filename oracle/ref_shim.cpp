// C exports over the reference's scalar host oracle (src/host_reference.hpp of
// the reference tree), compiled straight from the reference sources into
// oracle/_ref/.  Test infrastructure only: tests use it to cross-check the
// NumPy restatement; nothing in the library links it.
#include <cstdint>

#include "host_reference.hpp"  // reference src/host_reference.hpp:1-36

extern "C" {

// Reference src/host_reference.hpp:5-13: 16-bit state ending at bit (position+1)*bits.
uint16_t stx_ref_state(const uint32_t* ring_words, int bits, int position) {
    return host_state(ring_words, bits, position);
}

// Reference src/host_reference.hpp:22-36: codebook id 0 = 3inst, 1 = mcg, 2 = mul1.
uint16_t stx_ref_codebook(uint16_t state, int codebook) { return host_codebook(state, codebook); }

// All 65,536 codebook values of one codebook (FP16 bit patterns).
void stx_ref_codebook_table(int codebook, uint16_t* out) {
    for (uint32_t s = 0; s < 65536; ++s) out[s] = host_codebook(uint16_t(s), codebook);
}

// All 256 states of one tile given as 8K ring words.
void stx_ref_tile_states(const uint32_t* ring_words, int bits, uint16_t* out) {
    for (int p = 0; p < 256; ++p) out[p] = host_state(ring_words, bits, p);
}
}
