// Result<T>: value-or-error return type of the KV-cache API.
// Same interface as the reference's include/tiny_llm/result.h:9-111
// (ok/err factories, isOk/isErr, value() throwing on error, error() throwing
// on success, valueOr, map, flatMap, and the Result<void> specialisation), so
// callers written against tiny-llm compile unchanged.
#pragma once

#include <optional>
#include <stdexcept>
#include <string>
#include <utility>

namespace tiny_llm {

template <typename T>
class Result {
  public:
    using ValueType = T;

    static Result ok(T value) { return Result(std::move(value), std::string(), true); }
    static Result err(std::string message) { return Result(std::nullopt, std::move(message), false); }

    bool isOk() const { return ok_; }
    bool isErr() const { return !ok_; }

    T &value() {
        if (!ok_) throw std::runtime_error("Attempted to access value of error Result: " + msg_);
        return *val_;
    }
    const T &value() const {
        if (!ok_) throw std::runtime_error("Attempted to access value of error Result: " + msg_);
        return *val_;
    }
    const std::string &error() const {
        if (ok_) throw std::runtime_error("Attempted to access error of ok Result");
        return msg_;
    }
    T valueOr(T fallback) const { return ok_ ? *val_ : fallback; }

    template <typename F>
    auto map(F &&f) -> Result<decltype(f(std::declval<T>()))> {
        using U = decltype(f(std::declval<T>()));
        if (ok_) return Result<U>::ok(f(*val_));
        return Result<U>::err(msg_);
    }
    template <typename F>
    auto flatMap(F &&f) -> decltype(f(std::declval<T>())) {
        using R = decltype(f(std::declval<T>()));
        if (ok_) return f(*val_);
        return R::err(msg_);
    }

  private:
    Result(std::optional<T> v, std::string m, bool ok) : val_(std::move(v)), msg_(std::move(m)), ok_(ok) {}
    std::optional<T> val_;
    std::string      msg_;
    bool             ok_;
};

template <>
class Result<void> {
  public:
    static Result ok() { return Result(true, std::string()); }
    static Result err(std::string message) { return Result(false, std::move(message)); }

    bool isOk() const { return ok_; }
    bool isErr() const { return !ok_; }
    const std::string &error() const {
        if (ok_) throw std::runtime_error("Attempted to access error of ok Result");
        return msg_;
    }

  private:
    Result(bool ok, std::string m) : ok_(ok), msg_(std::move(m)) {}
    bool        ok_;
    std::string msg_;
};

} // namespace tiny_llm
