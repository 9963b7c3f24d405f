// CPU driver of the kernels' bit-level float conversions (economize_amd/csrc/fp8_codec.hpp): reads float32 values
// from stdin and writes, per value, its e4m3fn byte, its e5m2 byte and its bf16 bit pattern (little endian).
#include <cstdio>
#include <vector>

#include "../../economize_amd/csrc/fp8_codec.hpp"

int main() {
    std::vector<float> xs;
    float x;
    while (std::fread(&x, sizeof(float), 1, stdin) == 1) xs.push_back(x);
    for (float v : xs) {
        unsigned char a = eco::f32_to_fp8<1>(v);
        unsigned char b = eco::f32_to_fp8<2>(v);
        uint16_t h = eco::f32_to_bf16(v);
        std::fwrite(&a, 1, 1, stdout);
        std::fwrite(&b, 1, 1, stdout);
        std::fwrite(&h, 2, 1, stdout);
    }
    return 0;
}
