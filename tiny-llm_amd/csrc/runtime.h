// Host runtime pieces of the KV path: metadata staging, device workspace,
// the per-device context of the stateless entry points.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <mutex>
#include <vector>

namespace tiny_llm {
namespace detail {

// Ring of (pinned host, device) buffer pairs for per-step metadata.  begin()
// returns host memory to fill; commit() queues one async H2D copy on the
// stream and returns the device copy.  A slot is rewritten only after its
// previous copy has completed (event), so the host never overwrites bytes a
// pending copy still reads; kernels that read a device slot are ordered
// before its next copy by the stream.  (A copy on a separate stream, to
// overlap the previous step's kernels, ran as a blit kernel reading host
// memory next to the attention kernel and slowed it by more than it hid.)
class MetaRing {
  public:
    explicit MetaRing(int slots = 4);
    ~MetaRing();
    MetaRing(const MetaRing &) = delete;
    MetaRing &operator=(const MetaRing &) = delete;

    void *begin(size_t bytes);
    void *commit(hipStream_t stream);
    // Sizes every slot for `bytes` now, so steps up to that size never
    // allocate.
    void reserve(size_t bytes);

  private:
    struct Slot {
        void      *host = nullptr;
        void      *dev = nullptr;
        size_t     cap = 0;
        hipEvent_t ev = nullptr;
        bool       pending = false;
    };
    void              grow(Slot &s, size_t bytes);
    std::vector<Slot> slots_;
    // Buffers replaced by a larger one: kernels queued earlier may still read
    // a device buffer, so they are freed with the ring, not at growth (a free
    // would synchronise the device in the middle of a step).
    std::vector<void *> retired_dev_, retired_host_;
    int                 cur_ = -1;
    size_t              bytes_ = 0;
};

// Grow-only device buffer (split-K partials).
class Workspace {
  public:
    Workspace() = default;
    ~Workspace();
    Workspace(const Workspace &) = delete;
    Workspace &operator=(const Workspace &) = delete;
    float *get(size_t floats);
    // Grow-only ints that are zero between uses (the attention merge
    // counters: the kernels that count in them leave them zero).  A new
    // buffer is cleared on `stream`, ahead of whatever is queued there after
    // this call.
    int *counters(size_t n, hipStream_t stream);

  private:
    float              *ptr_ = nullptr;
    size_t              cap_ = 0;
    std::vector<float *> retired_; // replaced buffers, freed with the workspace
    int                *cnt_ = nullptr;
    size_t              cnt_cap_ = 0;
    std::vector<int *>  retired_cnt_;
};

// Staging + workspace of the stateless entry points, one per device.
struct DeviceContext {
    std::mutex  mu;
    MetaRing    ring;
    Workspace   ws;
    hipStream_t last_stream = nullptr;
    bool        used = false;
    // Orders this call after the previous user of the shared workspace.
    void claim(hipStream_t stream);
    static DeviceContext &get(int device);
};

int current_device();

// Event timing of the launchers (tl_profile_*); ids are KernelId values.
void profile_set(bool on);
void profile_reset();
bool profile_query(int id, double *total_ms, long long *launches);

} // namespace detail
} // namespace tiny_llm
