// Host check of the T16 byte maps in qk_device.h (built by the package's build.py, run by
// tests/test_layout.py): for every type, t16_dst maps the 16 rows' GGUF runs one-to-one onto the
// group's bytes and t16_src inverts it.  Prints "ok <type> <group bytes>" per type, exits 1 on error.
#include <cstdio>
#include <vector>

#include "qk_device.h"

int main() {
    const int types[] = {qk::T_Q8_0, qk::T_Q4_K, qk::T_Q5_K, qk::T_Q6_K};
    for (int type : types) {
        const int bs = qk::sb_bytes(type), gb = qk::group_bytes(type);
        std::vector<int> seen(gb, 0);
        for (int r = 0; r < 16; r++)
            for (int p = 0; p < bs; p++) {
                const int o = qk::t16_dst(type, r, p);
                if (o < 0 || o >= gb || seen[o]++) {
                    printf("type %d: row %d byte %d -> %d out of range or repeated\n", type, r, p, o);
                    return 1;
                }
                int r2 = -1, p2 = -1;
                qk::t16_src(type, o, r2, p2);
                if (r2 != r || p2 != p) {
                    printf("type %d: t16_src(%d) = (%d, %d), want (%d, %d)\n", type, o, r2, p2, r, p);
                    return 1;
                }
            }
        printf("ok %d %d\n", type, gb);
    }
    return 0;
}
