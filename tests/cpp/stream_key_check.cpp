// Checks the stream keys of the library's per-stream state
// (dnn-flash_amd/csrc/stream_key.h) on the CPU: hipStreamPerThread is keyed
// per host thread, every other handle (NULL included) names one stream
// whatever thread passes it, and devices never share a key. No HIP call is
// made. Prints "ok" and exits 0 on success.
#include <cstdio>
#include <thread>

#include "stream_key.h"

static int failures = 0;
#define CHECK(c)                                                    \
    do {                                                            \
        if (!(c)) {                                                 \
            std::printf("FAILED line %d: %s\n", __LINE__, #c);      \
            ++failures;                                             \
        }                                                           \
    } while (0)

int main() {
    hipStream_t user = reinterpret_cast<hipStream_t>(0x1234560);
    ofh::StreamKey pt_main = ofh::stream_key(0, hipStreamPerThread);
    ofh::StreamKey user_main = ofh::stream_key(0, user);
    ofh::StreamKey null_main = ofh::stream_key(0, nullptr);
    ofh::StreamKey pt_other, user_other, null_other;
    std::thread t([&] {
        pt_other = ofh::stream_key(0, hipStreamPerThread);
        user_other = ofh::stream_key(0, user);
        null_other = ofh::stream_key(0, nullptr);
    });
    t.join();
    CHECK(ofh::per_thread_stream(hipStreamPerThread));
    CHECK(!ofh::per_thread_stream(user) && !ofh::per_thread_stream(nullptr));
    CHECK(!(pt_main == pt_other));                       // two threads, two streams
    CHECK(pt_main < pt_other || pt_other < pt_main);     // distinct map keys
    CHECK(pt_main == ofh::stream_key(0, hipStreamPerThread));  // stable within a thread
    CHECK(user_main == user_other);                      // one stream whatever the thread
    CHECK(null_main == null_other);
    CHECK(!(user_main == null_main) && !(user_main == pt_main) && !(null_main == pt_main));
    CHECK(!(ofh::stream_key(1, user) == user_main));     // devices never share
    CHECK(!(ofh::stream_key(1, hipStreamPerThread) == pt_main));
    if (failures == 0) std::printf("ok\n");
    return failures == 0 ? 0 : 1;
}
