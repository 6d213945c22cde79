// status.hpp — status codes and the thread-local last-error message of the
// C ABI. Internal code throws nut::Error; every extern "C" entry point
// catches it (and std::bad_alloc) and returns the code.
#pragma once

#include <new>
#include <stdexcept>
#include <string>

#include "nutllm_hip.h"

namespace nut {

class Error : public std::runtime_error {
public:
    Error(int code, const std::string &message)
        : std::runtime_error(message), code_(code) {}
    int code() const { return code_; }

private:
    int code_;
};

[[noreturn]] inline void fail(int code, const std::string &message)
{
    throw Error(code, message);
}

inline void require(bool condition, int code, const char *message)
{
    if (!condition)
        fail(code, message);
}

void set_last_error(const char *message);

// Runs body, mapping exceptions to status codes and the last-error string.
template <typename Body> int guarded(Body &&body)
{
    try {
        body();
        set_last_error("");
        return NUT_OK;
    } catch (const Error &e) {
        set_last_error(e.what());
        return e.code();
    } catch (const std::bad_alloc &) {
        set_last_error("out of host memory");
        return NUT_ELENGTH;
    } catch (const std::exception &e) {
        set_last_error(e.what());
        return NUT_ERUNTIME;
    }
}

} // namespace nut
