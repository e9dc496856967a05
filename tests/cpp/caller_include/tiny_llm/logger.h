// The caller's own tiny_llm/logger.h, as the C++ drop-in test sees it.
//
// In tiny-llm this header is the spdlog-backed logger whose TLLM_* macros
// take fmt-style "{}" format strings (include/tiny_llm/logger.h:99-104).
// This directory sits after tiny-llm_amd/include on the test's include path,
// in the place the caller's include/ takes in a real integration, so the
// test proves that the library's include directory leaves tiny_llm/logger.h
// to the caller.  It is a minimal fmt-style formatter of the test's own
// ("{}" replaced by the next argument, streamed), not spdlog.
#pragma once

#include <iostream>
#include <sstream>
#include <string>

#define TINYLLM_TEST_CALLER_LOGGER 1

namespace tiny_llm {
namespace test_log {

inline void format_into(std::ostringstream &os, const char *f) { os << f; }

template <typename T, typename... Rest>
void format_into(std::ostringstream &os, const char *f, const T &v, const Rest &...rest) {
    for (; *f; ++f) {
        if (f[0] == '{' && f[1] == '}') {
            os << v;
            format_into(os, f + 2, rest...);
            return;
        }
        os << *f;
    }
}

template <typename... Args>
std::string format(const char *f, const Args &...args) {
    std::ostringstream os;
    format_into(os, f, args...);
    return os.str();
}

inline int &error_count() {
    static int n = 0;
    return n;
}

template <typename... Args>
void emit(const char *level, const char *f, const Args &...args) {
    if (level[0] == 'E') ++error_count();
    std::cerr << "[caller] [" << level << "] " << format(f, args...) << "\n";
}

} // namespace test_log
} // namespace tiny_llm

#define TLLM_INFO(...) ::tiny_llm::test_log::emit("I", __VA_ARGS__)
#define TLLM_WARN(...) ::tiny_llm::test_log::emit("W", __VA_ARGS__)
#define TLLM_ERROR(...) ::tiny_llm::test_log::emit("E", __VA_ARGS__)
