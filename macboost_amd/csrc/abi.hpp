// abi.hpp — how the exported C functions report failures: no exception
// crosses the ABI; a failing call stores a malloc'd message in *err (released
// with macboost_free_string) and returns its error value.
#pragma once
#include <cstdlib>
#include <cstring>
#include <exception>
#include <string>

namespace mb {

inline void set_err(char **err, const std::string &m) {
    if (err) *err = strdup(m.c_str());
}

template <typename Fn>
auto guarded(char **err, Fn fn, decltype(fn()) on_error) -> decltype(fn()) {
    try {
        return fn();
    } catch (const std::exception &e) {
        set_err(err, e.what());
    } catch (...) {
        set_err(err, "Internal error: unknown failure");
    }
    return on_error;
}

}  // namespace mb
