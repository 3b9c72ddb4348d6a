#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

namespace tiles {
// Lower-case hex SHA-256 of a byte range.
std::string sha256_hex(const void* data, size_t size);
} // namespace tiles
