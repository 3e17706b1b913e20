// IEEE binary16 and bfloat16 conversions for the loader (the semantics of
// Core/Utils/Half.cpp:8-78): round to nearest even, exact widening.
#include "host_common.h"

#include <cstring>

namespace WSP
{
std::uint16_t floatToHalf(float value)
{
    std::uint32_t x;
    std::memcpy(&x, &value, sizeof(x));
    const std::uint32_t sign = (x >> 16) & 0x8000u;
    const std::uint32_t mag = x & 0x7FFFFFFFu;
    if (mag >= 0x7F800000u)
        return (std::uint16_t) (mag == 0x7F800000u ? (sign | 0x7C00u) : (sign | 0x7E00u | ((mag >> 13) & 0x3FFu)));
    if (mag >= 0x477FF000u)
        return (std::uint16_t) (sign | 0x7C00u);
    if (mag < 0x38800000u)
    {
        if (mag < 0x33000000u)
            return (std::uint16_t) sign;
        const std::uint32_t exponent = mag >> 23;
        const std::uint32_t significand = (mag & 0x7FFFFFu) | 0x800000u;
        const std::uint32_t shift = 126u - exponent;
        std::uint32_t k = significand >> shift;
        const std::uint32_t rest = significand & ((1u << shift) - 1u);
        const std::uint32_t half = 1u << (shift - 1u);
        if (rest > half || (rest == half && (k & 1u)))
            ++k;
        return (std::uint16_t) (sign | k);
    }
    std::uint32_t h = (mag >> 13) - (112u << 10);
    const std::uint32_t rest = mag & 0x1FFFu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u)))
        ++h;
    return (std::uint16_t) (sign | h);
}

float halfToFloat(std::uint16_t bits)
{
    const std::uint32_t sign = (std::uint32_t) (bits & 0x8000u) << 16;
    const std::uint32_t exponent = (bits >> 10) & 0x1Fu;
    std::uint32_t mantissa = bits & 0x3FFu;
    std::uint32_t x;
    if (exponent == 0x1Fu)
        x = sign | 0x7F800000u | (mantissa << 13);
    else if (exponent != 0)
        x = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    else if (mantissa == 0)
        x = sign;
    else
    {
        int e = -1;
        do
        {
            ++e;
            mantissa <<= 1;
        } while ((mantissa & 0x400u) == 0);
        x = sign | ((std::uint32_t) (112 - e) << 23) | ((mantissa & 0x3FFu) << 13);
    }
    float f;
    std::memcpy(&f, &x, sizeof(f));
    return f;
}

float bfloat16ToFloat(std::uint16_t bits)
{
    const std::uint32_t x = (std::uint32_t) bits << 16;
    float f;
    std::memcpy(&f, &x, sizeof(f));
    return f;
}
} // namespace WSP
