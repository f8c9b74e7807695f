// error.h -- error behaviour of the host layer.
//
// The reference aborts on every violated precondition (LUISA_ASSERT, e.g.
// unknown operator include/onnx/onnx.h:362, dtype/shape mismatch on bind
// src/onnx/network_instance.cpp:50-64).  Here the same checks throw
// lcml::onnx::Error carrying the same kind of message, so a caller may catch
// it; uncaught, the process still terminates.
#pragma once

#include <cstdio>
#include <stdexcept>
#include <string>

namespace lcml::onnx {

class Error : public std::runtime_error {
public:
    explicit Error(const std::string &msg) : std::runtime_error(msg) {}
};

// a message without arguments is taken verbatim (a '%' in it is not a
// conversion)
inline std::string format(const char *msg) { return msg; }

template <typename... Args>
inline std::string format(const char *fmt, Args... args) {
    int n = std::snprintf(nullptr, 0, fmt, args...);
    std::string s(n > 0 ? (size_t)n : 0, '\0');
    std::snprintf(s.data(), s.size() + 1, fmt, args...);
    return s;
}

}  // namespace lcml::onnx

#define LCML_ASSERT(cond, ...)                                                     \
    do {                                                                           \
        if (!(cond)) throw ::lcml::onnx::Error(::lcml::onnx::format(__VA_ARGS__)); \
    } while (0)
