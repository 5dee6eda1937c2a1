#include "ft/error.hpp"

#include <cstdio>

namespace ftrain {

void Result::compose(FTrainStatus status, const char* text, std::va_list* args) noexcept {
    status_ = status;
    char* out = text_.data();
    out[0] = '\0';
    if (status == FTRAIN_STATUS_SUCCESS || text == nullptr) return;
    // "%s" on a literal and the caller's format on arguments go through the
    // same bounded formatter, so truncation is identical for both.
    int written = args ? std::vsnprintf(out, kMessageBytes, text, *args) : std::snprintf(out, kMessageBytes, "%s", text);
    if (written < 0) out[0] = '\0';
    out[kMessageBytes - 1] = '\0';
}

void Result::vformat(FTrainStatus status, const char* fmt, std::va_list args) noexcept {
    std::va_list copy;
    va_copy(copy, args);
    compose(status, fmt, &copy);
    va_end(copy);
}

void Result::format(FTrainStatus status, const char* fmt, ...) noexcept {
    std::va_list args;
    va_start(args, fmt);
    compose(status, fmt, &args);
    va_end(args);
}

Failure::Failure(const Result& result) noexcept : result_(result) {
    // A Failure always reports a failure: a success status here is a bug in
    // the raising code, reported as such rather than as a silent success.
    if (result_.isSuccess()) result_.set(FTRAIN_STATUS_INTERNAL_ERROR, "internal: a failure was raised with a success status");
}

void raise(FTrainStatus status, const char* fmt, ...) {
    Result r;
    std::va_list args;
    va_start(args, fmt);
    r.vformat(status, fmt, args);
    va_end(args);
    throw Failure(r);
}

}  // namespace ftrain
