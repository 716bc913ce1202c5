#pragma once

// How a KV cache stores its rows (reference src/quant/kv_format.h:11-35): the subset of that interface the HIP
// backend compiles against.

#include <cstdint>
#include <string_view>

namespace xs::quant {

enum class KvFormat : uint8_t { Float, I8, Turbo4, Turbo3, Turbo2 };

struct KvFormats {
    KvFormat k = KvFormat::Float;
    KvFormat v = KvFormat::Float;
    bool operator==(const KvFormats&) const = default;
};

std::string_view kv_format_name(KvFormat f);

// Bits per value of a TurboQuant format, 0 for the others.
constexpr int turbo_bits(KvFormat f) {
    return f == KvFormat::Turbo4 ? 4 : f == KvFormat::Turbo3 ? 3 : f == KvFormat::Turbo2 ? 2 : 0;
}

}  // namespace xs::quant
