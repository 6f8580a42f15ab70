// Identity of the stream a call is ordered on, for the library's per-stream
// state (scratch buffers, split-merge counter slots).
//
// hipStreamPerThread is one handle value that names a different stream in
// every host thread, so calls made with it are keyed by the calling thread as
// well: two threads passing it run concurrently on different streams and must
// not share a buffer. Every other handle names one stream whatever thread
// passes it. That includes the null stream: this library is built without
// per-thread default streams, so its launches with a null handle go to the
// device's one legacy null stream.

#ifndef OFH_STREAM_KEY_H
#define OFH_STREAM_KEY_H

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <thread>
#include <tuple>

namespace ofh {

struct StreamKey {
    int device;
    uintptr_t stream;
    std::thread::id thread;  // default id unless the handle is per-thread

    bool operator<(const StreamKey& o) const {
        return std::tie(device, stream, thread) < std::tie(o.device, o.stream, o.thread);
    }
    bool operator==(const StreamKey& o) const {
        return device == o.device && stream == o.stream && thread == o.thread;
    }
};

inline bool per_thread_stream(hipStream_t s) { return s == hipStreamPerThread; }

inline StreamKey stream_key(int device, hipStream_t s) {
    return StreamKey{device, reinterpret_cast<uintptr_t>(s),
                     per_thread_stream(s) ? std::this_thread::get_id() : std::thread::id()};
}

}  // namespace ofh

#endif  // OFH_STREAM_KEY_H
