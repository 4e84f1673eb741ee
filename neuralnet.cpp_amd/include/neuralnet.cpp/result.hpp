#pragma once
// result.hpp — nn::Result<T>: value-or-error return type of every engine/layer call.
//
// The reference uses exstl::Result<T> = std::expected<T, Error{std::string message}> and
// builds with -fno-exceptions (docs/introduction/01-architecture.md:221-222, :250). The
// C++ standard library available to this build (libstdc++ 11) has no <expected>, so this
// header provides the small subset the path needs, with the same spelling at call sites:
// has_value(), operator bool, operator*, operator->, error().message.

#include <cstdio>
#include <cstdlib>
#include <string>
#include <type_traits>
#include <utility>

namespace nn
{

struct Error
{
    std::string message;
};

template <class T>
class [[nodiscard]] Result
{
public:
    Result(const T& v) : ok_(true), value_(v) {}
    Result(T&& v) : ok_(true), value_(std::move(v)) {}
    Result(Error e) : ok_(false), error_(std::move(e)) {}

    [[nodiscard]] bool has_value() const noexcept { return ok_; }
    explicit operator bool() const noexcept { return ok_; }
    T& operator*() & { return value_; }
    const T& operator*() const& { return value_; }
    T&& operator*() && { return std::move(value_); }
    T* operator->() { return &value_; }
    const T* operator->() const { return &value_; }
    T& value() & { return value_; }
    [[nodiscard]] const Error& error() const { return error_; }

private:
    bool ok_;
    T value_{};
    Error error_{};
};

template <>
class [[nodiscard]] Result<void>
{
public:
    Result() : ok_(true) {}
    Result(Error e) : ok_(false), error_(std::move(e)) {}
    [[nodiscard]] bool has_value() const noexcept { return ok_; }
    explicit operator bool() const noexcept { return ok_; }
    [[nodiscard]] const Error& error() const { return error_; }

private:
    bool ok_;
    Error error_{};
};

inline Error make_error(std::string msg) { return Error{std::move(msg)}; }

}  // namespace nn

namespace exstl
{
template <class T>
using Result = nn::Result<T>;
using Error = nn::Error;
}  // namespace exstl

// Error-propagation helpers with the reference's names (exstl/error_macros.hpp):
//   EX_FAIL(msg)           return an error from the current function
//   EX_TRY(var, expr)      evaluate a Result-returning expr; on error return it, else bind `var`
//   EX_TRY_CHECK(expr)     evaluate; on error return it
//   EX_UNWRAP(cond, msg)   abort the process with msg if cond is false (for void contexts)
#define EX_FAIL(msg) return ::nn::Error { std::string(msg) }
#define EX_TRY(var, expr)                                  \
    auto var = (expr);                                     \
    if (!var.has_value()) return ::nn::Error { var.error().message }
#define EX_TRY_CHECK(expr)                                              \
    do                                                                  \
    {                                                                   \
        auto ex_r_ = (expr);                                            \
        if (!ex_r_.has_value()) return ::nn::Error{ex_r_.error().message}; \
    } while (0)
#define EX_UNWRAP(cond, msg)                                            \
    do                                                                  \
    {                                                                   \
        if (!(cond))                                                    \
        {                                                               \
            std::fprintf(stderr, "fatal: %s\n", std::string(msg).c_str()); \
            std::abort();                                               \
        }                                                               \
    } while (0)
