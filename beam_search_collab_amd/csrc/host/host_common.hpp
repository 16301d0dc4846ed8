// Shared helpers of the host library (error text, thread count).
#pragma once
#include <string>

namespace bsh {
extern thread_local std::string g_err;
int fail(int code, const std::string& msg);
// inside a catch handler: the error code and text for the exception in flight
int exception_code();
int n_threads(int threads);
}  // namespace bsh
