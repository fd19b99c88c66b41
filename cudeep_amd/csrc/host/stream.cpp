// RAII stream / event (interface of the reference's src/stream.cu:5-65).
#include "../../../include/cudeep/stream.hpp"

namespace cudeep {

Stream::Stream() { CUDEEP_CHECK_HIP(hipStreamCreate(&stream_)); }

Stream::~Stream() {
    if (owns_ && stream_) (void)hipStreamDestroy(stream_);
}

Stream::Stream(Stream&& o) noexcept : stream_(o.stream_), owns_(o.owns_) {
    o.stream_ = nullptr;
    o.owns_ = false;
}

Stream& Stream::operator=(Stream&& o) noexcept {
    if (this != &o) {
        if (owns_ && stream_) (void)hipStreamDestroy(stream_);
        stream_ = o.stream_;
        owns_ = o.owns_;
        o.stream_ = nullptr;
        o.owns_ = false;
    }
    return *this;
}

void Stream::synchronize() { CUDEEP_CHECK_HIP(hipStreamSynchronize(stream_)); }

Stream& Stream::default_stream() {
    static Stream* s = new Stream(nullptr, false);   // the null stream, never destroyed
    return *s;
}

Event::Event() { CUDEEP_CHECK_HIP(hipEventCreate(&event_)); }

Event::~Event() {
    if (event_) (void)hipEventDestroy(event_);
}

void Event::record(hipStream_t stream) { CUDEEP_CHECK_HIP(hipEventRecord(event_, stream)); }

void Event::synchronize() { CUDEEP_CHECK_HIP(hipEventSynchronize(event_)); }

float Event::elapsed_ms(const Event& start) const {
    float ms = 0.0f;
    CUDEEP_CHECK_HIP(hipEventElapsedTime(&ms, start.event_, event_));
    return ms;
}

}  // namespace cudeep
