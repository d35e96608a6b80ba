// Host check of gpt_attn::join_words (gpt_amd/csrc/attn_addr.h), the
// recombination the kernels apply to a buffer descriptor's base address after
// broadcasting its two 32-bit words: every address must come back unchanged,
// in particular those whose low word has bit 31 set (device allocations above
// 2 GiB offsets within a 4 GiB window). Exit status 0 and "ok" on success.
#include "../gpt_amd/csrc/attn_addr.h"

#include <stdio.h>

static int broadcast(int x) { return x; }  // readfirstlane of a uniform value

int main()
{
    const uint64_t bases[] = {0x0ull, 0x7fffffffull, 0x80000000ull, 0xffffffffull, 0x100000000ull,
                              0x7f1280000000ull, 0x7f12ffffff00ull, 0x00007ffe9a3c4000ull, 0xfffffffffffff000ull};
    int bad = 0, n = 0, bit31 = 0;
    for (uint64_t b : bases)
    {
        for (uint64_t d = 0; d < (1u << 12); d += 16)
        {
            const uint64_t a = b + d;
            const uint64_t u = gpt_attn::join_words(broadcast((int)(uint32_t)(a >> 32)), broadcast((int)(uint32_t)a));
            ++n;
            bit31 += (a >> 31) & 1;
            if (u != a)
            {
                if (bad < 5)
                    printf("mismatch: %016llx -> %016llx\n", (unsigned long long)a, (unsigned long long)u);
                ++bad;
            }
        }
    }
    printf("%s: %d addresses, %d with bit 31 set in the low word, %d mismatches\n", bad ? "FAIL" : "ok", n, bit31,
           bad);
    return bad ? 1 : 0;
}
