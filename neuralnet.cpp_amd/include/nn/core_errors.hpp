// core_errors.hpp — error type and Result<T> for the HIP engine's host side.
//
// Mirrors the reference's error convention (include/neuralnet.cpp/core_errors.hpp:15-20):
// every public call returns Result<T>; nothing throws. The reference aliases
// Result<T> to std::expected<T, Error>, which libstdc++ 11 (the toolchain on
// this image) does not ship, so this header defines a small value-or-error
// type with the same member surface (has_value, operator bool, *, ->, value,
// error) and an `nn::unexpected` wrapper used exactly like std::unexpected.
#pragma once

#include <cstdlib>
#include <string>
#include <type_traits>
#include <utility>
#include <variant>

namespace nn
{

struct Error
{
    std::string message;
};

template <class E>
class unexpected
{
public:
    explicit unexpected(E e) : e_(std::move(e)) {}
    [[nodiscard]] const E& error() const& noexcept { return e_; }
    [[nodiscard]] E& error() & noexcept { return e_; }
    [[nodiscard]] E&& error() && noexcept { return std::move(e_); }

private:
    E e_;
};
template <class E>
unexpected(E) -> unexpected<E>;

// Value-or-Error. Accessing the value of an error result aborts (the
// reference's std::expected would throw bad_expected_access, which under
// -fno-exceptions is also fatal).
template <class T>
class [[nodiscard]] Result
{
public:
    Result() : v_(std::in_place_index<0>) {}
    Result(const T& v) : v_(std::in_place_index<0>, v) {}
    Result(T&& v) : v_(std::in_place_index<0>, std::move(v)) {}
    template <class U,
              class = std::enable_if_t<std::is_constructible_v<T, U&&> &&
                                       !std::is_same_v<std::decay_t<U>, Result> &&
                                       !std::is_same_v<std::decay_t<U>, unexpected<Error>>>>
    Result(U&& v) : v_(std::in_place_index<0>, T(std::forward<U>(v))) {}
    Result(const unexpected<Error>& e) : v_(std::in_place_index<1>, e.error()) {}
    Result(unexpected<Error>&& e) : v_(std::in_place_index<1>, std::move(e).error()) {}

    [[nodiscard]] bool has_value() const noexcept { return v_.index() == 0; }
    explicit operator bool() const noexcept { return has_value(); }

    T& value() &
    {
        check_();
        return std::get<0>(v_);
    }
    const T& value() const&
    {
        check_();
        return std::get<0>(v_);
    }
    T&& value() &&
    {
        check_();
        return std::get<0>(std::move(v_));
    }
    T& operator*() & { return value(); }
    const T& operator*() const& { return value(); }
    T&& operator*() && { return std::move(*this).value(); }
    T* operator->() { return &value(); }
    const T* operator->() const { return &value(); }

    [[nodiscard]] const Error& error() const& { return std::get<1>(v_); }
    [[nodiscard]] Error& error() & { return std::get<1>(v_); }

private:
    void check_() const
    {
        if (v_.index() != 0)
            std::abort();
    }
    std::variant<T, Error> v_;
};

template <>
class [[nodiscard]] Result<void>
{
public:
    Result() = default;
    Result(const unexpected<Error>& e) : ok_(false), err_(e.error()) {}
    Result(unexpected<Error>&& e) : ok_(false), err_(std::move(e).error()) {}

    [[nodiscard]] bool has_value() const noexcept { return ok_; }
    explicit operator bool() const noexcept { return ok_; }
    void value() const
    {
        if (!ok_)
            std::abort();
    }
    void operator*() const { value(); }
    [[nodiscard]] const Error& error() const& { return err_; }
    [[nodiscard]] Error& error() & { return err_; }

private:
    bool ok_ = true;
    Error err_{};
};

// Shorthand used by engine implementations.
[[nodiscard]] inline unexpected<Error> fail(std::string msg)
{
    return unexpected<Error>(Error{std::move(msg)});
}

} // namespace nn

// Early-return helpers for Result-returning functions.
#define NN_TRY(var, expr)                                                                      \
    auto var##_res_ = (expr);                                                                  \
    if (!var##_res_)                                                                           \
        return ::nn::unexpected(var##_res_.error());                                           \
    auto& var = *var##_res_

#define NN_CHECK(expr)                                                                         \
    do                                                                                         \
    {                                                                                          \
        auto nn_check_res_ = (expr);                                                           \
        if (!nn_check_res_)                                                                    \
            return ::nn::unexpected(nn_check_res_.error());                                    \
    } while (0)
