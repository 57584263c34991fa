// Driver for the reference's own scalar decoders, built into oracle/_ref by
// oracle/Makefile from the header under the reference tree
// (vendor/strata/include/strata/artifact/dequant.hpp:33-55 fp16_to_fp32,
// :68-78 dequantize_q2_0). Test infrastructure only.
//
// Usage: ref_dequant <out.bin>
// Writes, little-endian f32:
//   1. fp16_to_fp32(h) for all 65,536 patterns h;
//   2. dequantize_q2_0 of 256 blocks built by the recipe of the reference's
//      upstream known-answer test (scripts/test-upstream.mjs:20): scale
//      h = ((b%16)+8)*1024 + (b*7)%1024 + (b odd ? 0x8000 : 0), code bytes
//      (i*19 + b*73) & 255.
#include "strata/artifact/dequant.hpp"
#include <cstdio>

int main(int argc, char **argv) {
    if (argc != 2) return 2;
    FILE *f = std::fopen(argv[1], "wb");
    if (!f) return 3;
    for (unsigned h = 0; h < 65536; h++) {
        float v = strata::fp16_to_fp32((uint16_t)h);
        std::fwrite(&v, 4, 1, f);
    }
    for (int b = 0; b < 256; b++) {
        unsigned char block[18];
        unsigned h = ((b % 16) + 8) * 1024 + (b * 7) % 1024 + (b % 2 ? 32768 : 0);
        block[0] = h & 255;
        block[1] = h >> 8;
        for (int i = 0; i < 16; i++) block[2 + i] = (unsigned char)((i * 19 + b * 73) & 255);
        float values[64];
        strata::dequantize_q2_0(block, values);
        std::fwrite(values, sizeof(values), 1, f);
    }
    return std::fclose(f) == 0 ? 0 : 4;
}
