// status.h — the error convention of the C-ABI, for host and device sources
// alike: exceptions carrying a dmx_status code inside, a status code and a
// per-thread message at the boundary.
#pragma once

#include <new>
#include <stdexcept>
#include <string>

namespace dmx {

// Error carrying one of the dmx_status codes of include/dmx.h.
struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string &msg) : std::runtime_error(msg), code(c) {}
};

[[noreturn]] inline void throw_error(int code, const std::string &msg) { throw Error(code, msg); }

// The calling thread's last error message (dmx_last_error).
std::string &last_error_slot();

// Runs f, turning exceptions into a dmx_status code and a message.
template <class F>
int guarded(F &&f) {
    try {
        f();
        last_error_slot().clear();
        return 0;
    } catch (const Error &e) {
        last_error_slot() = e.what();
        return e.code;
    } catch (const std::bad_alloc &) {
        last_error_slot() = "out of host memory";
        return 7;
    } catch (const std::exception &e) {
        last_error_slot() = e.what();
        return 6;
    }
}

}  // namespace dmx
