#pragma once

// How a KV cache stores its rows (reference src/quant/kv_format.h:11-23). The HIP backend stores I8.

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

}  // namespace xs::quant
