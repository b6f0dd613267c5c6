// Host-side check of lora_coldot's launch geometry (lora_kernels.h): for row
// counts up to the C ABI's limit (2^31 - 1), the chunks cover every row, each
// chunk is at least 16 rows, and the chunk count (grid.y) stays within
// 65535.  Built and run by tests/test_geometry.py; prints "ok <cases>".
#include <cstdio>

#include "lora_kernels.h"

int main() {
    const long long rows_list[] = {1, 15, 16, 17, 1000, 4096, 65535, 262144, 8388480, 8388481, 8388608,
                                   9000000, 100000000, 1000000000, 2147483647};
    const long long k_list[] = {1, 8, 1152, 6912, 65536};
    int cases = 0;
    for (long long rows : rows_list)
        for (long long K : k_list) {
            const long long chunk = mft::lora_coldot_chunk(rows, K);
            const long long chunks = (rows + chunk - 1) / chunk;
            if (chunk < 16 || chunks > mft::kLoraMaxGridY || chunks * chunk < rows ||
                (chunks - 1) * chunk >= rows) {
                std::printf("BAD rows=%lld K=%lld chunk=%lld chunks=%lld\n", rows, K, chunk, chunks);
                return 1;
            }
            ++cases;
        }
    std::printf("ok %d\n", cases);
    return 0;
}
