// Leveled stderr log of this library's own host code (private header; it is
// not on the public include path, so a caller's tiny_llm/logger.h -- the
// reference's spdlog logger with fmt-style TLLM_* macros,
// include/tiny_llm/logger.h:99-104 -- is never shadowed, and no symbol here
// collides with tiny_llm::Logger).  Printf-style messages; level from the
// environment variable TLLM_LOG_LEVEL (trace, debug, info, warn, error,
// critical, off), default warn.
#pragma once

namespace tiny_llm {
namespace detail {
namespace log {

enum class Level { TRACE = 0, DEBUG = 1, INFO = 2, WARN = 3, ERROR = 4, CRITICAL = 5, OFF = 6 };

Level level();
void  set_level(Level level);
inline bool enabled(Level l) { return static_cast<int>(l) >= static_cast<int>(level()); }
void  write(Level level, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

} // namespace log
} // namespace detail
} // namespace tiny_llm

#define TL_LOG_AT(lvl, ...)                                                                        \
    do {                                                                                           \
        if (::tiny_llm::detail::log::enabled(lvl)) ::tiny_llm::detail::log::write(lvl, __VA_ARGS__); \
    } while (0)
#define TL_LOG_TRACE(...) TL_LOG_AT(::tiny_llm::detail::log::Level::TRACE, __VA_ARGS__)
#define TL_LOG_DEBUG(...) TL_LOG_AT(::tiny_llm::detail::log::Level::DEBUG, __VA_ARGS__)
#define TL_LOG_INFO(...) TL_LOG_AT(::tiny_llm::detail::log::Level::INFO, __VA_ARGS__)
#define TL_LOG_WARN(...) TL_LOG_AT(::tiny_llm::detail::log::Level::WARN, __VA_ARGS__)
#define TL_LOG_ERROR(...) TL_LOG_AT(::tiny_llm::detail::log::Level::ERROR, __VA_ARGS__)
