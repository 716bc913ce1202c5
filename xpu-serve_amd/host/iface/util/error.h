#pragma once

// The interface surface the HIP backend is written against, restated from the reference (src/util/error.h:10-35):
// one exception type, a variadic message builder, and the check macro. In the reference tree the backend includes
// the reference's own header of this name instead.

#include <sstream>
#include <stdexcept>
#include <string>
#include <utility>

namespace xs {

class Error : public std::runtime_error {
public:
    using std::runtime_error::runtime_error;
};

template <typename... Args>
std::string str_cat(Args&&... args) {
    std::ostringstream os;
    (os << ... << std::forward<Args>(args));
    return os.str();
}

template <typename... Args>
[[noreturn]] void fail(Args&&... args) {
    throw Error(str_cat(std::forward<Args>(args)...));
}

}  // namespace xs

#define XS_CHECK(cond, ...)                                                   \
    do {                                                                      \
        if (!(cond)) ::xs::fail("check failed: (" #cond "): ", __VA_ARGS__);  \
    } while (0)
