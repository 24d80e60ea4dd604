// How the C entry points of libtchip_host.so (include/tchip_host.h) report a
// failure: the body runs under `guarded`, which turns a thrown `hip::Error`,
// shape error or other exception into the status the entry point returns and
// keeps the message for `tch_last_error()` on the calling thread.
#pragma once

#include <stdexcept>
#include <string>

#include "backend.hpp"

namespace tensorcrate {
namespace hip {

inline thread_local std::string host_error;

template <typename F>
int guarded(F&& body) {
    try {
        body();
        return TC_OK;
    } catch (const Error& e) {
        host_error = e.what();
        return e.status;
    } catch (const std::invalid_argument& e) {
        host_error = e.what();
        return TC_INVALID;
    } catch (const std::exception& e) {
        host_error = e.what();
        return TC_DEVICE;
    }
}

}  // namespace hip
}  // namespace tensorcrate
