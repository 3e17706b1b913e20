// Shared by the host translation units: status-to-exception mapping and the
// host-side fp16/bf16 conversions the loader uses.
#pragma once

#include <cstdint>
#include <string>

namespace WSP
{
// Throws the reference's exception for a C-ABI status: LOGIC ->
// std::logic_error, HIP/DEVICE -> std::runtime_error, the rest ->
// std::invalid_argument.
void throwForStatus(int status, const std::string& message);

// IEEE binary16 <-> binary32, round to nearest even (Core/Utils/Half.cpp).
std::uint16_t floatToHalf(float value);
float halfToFloat(std::uint16_t bits);
float bfloat16ToFloat(std::uint16_t bits);
} // namespace WSP
