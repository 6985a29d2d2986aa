// Installed-package smoke check: the headers compile in a plain C++ consumer, the library links
// and loads, and a call that validation rejects (null Q) returns NULL_POINTER without GPU work.
#include <cstdio>

#include "cuflash/flash_attention.h"
#include "cuflash/kernels/matmul.cuh"
#include "cuflash/version.h"

int main() {
    float x = 0.0f;
    const auto err =
        cuflash::flash_attention_forward(nullptr, &x, &x, &x, &x, 1, 1, 1, 32, 1.0f, false, 0);
    if (err != cuflash::FlashAttentionError::NULL_POINTER) {
        std::fprintf(stderr, "expected NULL_POINTER, got %d\n", static_cast<int>(err));
        return 1;
    }
    const auto merr = cuflash::kernels::matmul_ABt<64, 64, 32>(nullptr, &x, &x, 1.0f, 0);
    if (merr != cuflash::FlashAttentionError::NULL_POINTER) {
        std::fprintf(stderr, "matmul_ABt: expected NULL_POINTER, got %d\n", static_cast<int>(merr));
        return 1;
    }
    std::printf("%s %s\n", cuflash::get_error_string(cuflash::FlashAttentionError::SUCCESS),
                cuflash_version());
    return 0;
}
