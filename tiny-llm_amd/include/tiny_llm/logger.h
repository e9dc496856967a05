// Minimal leveled stderr logger with the reference's TLLM_* macro names
// (include/tiny_llm/logger.h:99-104).  The reference routes them through
// spdlog, which is fetched from the network at build time and is not
// available here; on the KV path the macros only report, so a printf-style
// sink keeps behaviour.  Level from TLLM_LOG_LEVEL (trace..critical, off);
// default "warn".
#pragma once

#include <cstdarg>

namespace tiny_llm {

enum class LogLevel { TRACE = 0, DEBUG = 1, INFO = 2, WARN = 3, ERROR = 4, CRITICAL = 5, OFF = 6 };

class Logger {
  public:
    static void     setLevel(LogLevel level);
    static LogLevel level();
    static bool     enabled(LogLevel level) { return static_cast<int>(level) >= static_cast<int>(Logger::level()); }
    static void     log(LogLevel level, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
};

} // namespace tiny_llm

#define TLLM_LOG_AT(lvl, ...)                                                                      \
    do {                                                                                           \
        if (::tiny_llm::Logger::enabled(lvl)) ::tiny_llm::Logger::log(lvl, __VA_ARGS__);           \
    } while (0)
#define TLLM_TRACE(...) TLLM_LOG_AT(::tiny_llm::LogLevel::TRACE, __VA_ARGS__)
#define TLLM_DEBUG(...) TLLM_LOG_AT(::tiny_llm::LogLevel::DEBUG, __VA_ARGS__)
#define TLLM_INFO(...) TLLM_LOG_AT(::tiny_llm::LogLevel::INFO, __VA_ARGS__)
#define TLLM_WARN(...) TLLM_LOG_AT(::tiny_llm::LogLevel::WARN, __VA_ARGS__)
#define TLLM_ERROR(...) TLLM_LOG_AT(::tiny_llm::LogLevel::ERROR, __VA_ARGS__)
#define TLLM_CRITICAL(...) TLLM_LOG_AT(::tiny_llm::LogLevel::CRITICAL, __VA_ARGS__)
