// Prints raw Philox4x32-10 blocks from rocRAND's host-callable engine
// (rocrand/rocrand_philox4x32_10.h, MIT) for (seed, subsequence, offset)
// triples.  Built and run by make_rocrand_vectors.py; its output is the
// committed fixture rocrand_philox.json, an independent library check of the
// oracle's Philox counter layout.
#include <rocrand/rocrand_philox4x32_10.h>
#include <cstdio>

int main()
{
    const unsigned long long cases[][3] = {
        {10ull, 0ull, 0ull},          {10ull, 1ull, 0ull},         {10ull, 218111ull, 0ull},
        {10ull, 0ull, 4ull},          {10ull, 8703ull, 4ull},      {42ull, 12345ull, 8ull},
        {7ull, 524287ull, 0ull},      {0x123456789abcdefull, 3ull, 400ull},
        {123ull, 0x1ffffffffull, 4ull}, {0xffffffffffffffffull, 0xffffffffffffffffull, 0xfffffffffffffffcull},
    };
    std::printf("[\n");
    const int ncases = sizeof(cases) / sizeof(cases[0]);
    for (int i = 0; i < ncases; ++i) {
        rocrand_device::philox4x32_10_engine eng(cases[i][0], cases[i][1], cases[i][2]);
        std::printf("  {\"seed\": %llu, \"subsequence\": %llu, \"offset\": %llu, \"blocks\": [",
                    cases[i][0], cases[i][1], cases[i][2]);
        for (int b = 0; b < 3; ++b) {
            unsigned int v[4];
            for (int k = 0; k < 4; ++k) v[k] = eng.next();
            std::printf("%s[%u, %u, %u, %u]", b ? ", " : "", v[0], v[1], v[2], v[3]);
        }
        std::printf("]}%s\n", i + 1 < ncases ? "," : "");
    }
    std::printf("]\n");
    return 0;
}
