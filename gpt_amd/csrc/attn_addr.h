// Address arithmetic shared by the kernels and a host-side test
// (tests/test_addr.py): no HIP dependency.
#pragma once

#include <stdint.h>

#if defined(__HIP__)
#define GPT_ATTN_HD __host__ __device__ __forceinline__
#else
#define GPT_ATTN_HD inline
#endif

namespace gpt_attn {

// A 64-bit address rebuilt from its two 32-bit words after each went through
// a 32-bit signed lane broadcast (readfirstlane is int -> int). Each word is
// taken back as uint32_t, so the low word is zero-extended: converting it
// through int instead sign-extends it into the high word for every address
// whose bit 31 is set, which corrupts a buffer descriptor's base.
GPT_ATTN_HD uint64_t join_words(int hi, int lo)
{
    return ((uint64_t)(uint32_t)hi << 32) | (uint64_t)(uint32_t)lo;
}

}  // namespace gpt_attn
