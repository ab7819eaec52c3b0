// Host-side bookkeeping of the serving dispatcher (serving.cpp), free of HIP
// so its rules are testable on the host.
//
// Submissions<T>: ownership of accepted serving submissions across a terminal
// device failure (the reference's Submissions<T>,
// crates/nvidia/src/submissions.rs:1-47).
//
// Pending records are keyed by submission id. A device failure poisons the
// owner for good; the records it held are retired only when the stream drain
// that followed the failure succeeded (the one evidence that no queued work
// still touches them), otherwise they stay quarantined until teardown, and
// physical release is refused while that is so.
#pragma once

#include <stdint.h>

#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace ribn_amd_dispatch {

template <class T>
class Submissions {
public:
    std::unordered_map<uint64_t, T> pending;

    // The first failure's message, or null while healthy.
    const char* fault() const { return faulted_ ? fault_.c_str() : nullptr; }
    // False while a failed drain left ownership uncertain.
    bool release_is_safe() const { return !undrained_; }
    void quarantine(T value) { quarantined_.push_back(std::move(value)); }
    size_t quarantined() const { return quarantined_.size(); }

    // Ends polling of every pending submission. Returns the records that may
    // be retired (all of them, quarantined ones included, after a successful
    // drain; none otherwise). The owner stays poisoned either way, reporting
    // the latest failure.
    std::vector<T> fail(std::string error, bool drained) {
        fault_ = std::move(error);
        faulted_ = true;
        undrained_ = !drained;
        for (auto& kv : pending) quarantined_.push_back(std::move(kv.second));
        pending.clear();
        std::vector<T> retired;
        if (drained) retired.swap(quarantined_);
        return retired;
    }

    // Everything still held, for teardown.
    std::vector<T> take_all() {
        std::vector<T> all;
        all.swap(quarantined_);
        for (auto& kv : pending) all.push_back(std::move(kv.second));
        pending.clear();
        return all;
    }

private:
    std::vector<T> quarantined_;
    std::string fault_;
    bool faulted_ = false;
    bool undrained_ = false;
};

// Row results collected while queueing one scheduler batch (QueuedRows,
// serving.rs:39-58): the leased output slot (-1: none) and queueing time per
// row in scheduler order, and the state keys the queued work touches.
struct QueuedRows {
    std::vector<int32_t> outputs;
    std::vector<uint64_t> elapsed;
    std::vector<uint64_t> state_keys;

    // scatter_group: rows that ran together as `group` return to their
    // scheduler positions `indices`.
    void scatter(const std::vector<size_t>& indices, QueuedRows&& group) {
        for (size_t i = 0; i < indices.size(); ++i) {
            outputs[indices[i]] = group.outputs[i];
            elapsed[indices[i]] = group.elapsed[i];
        }
        state_keys.insert(state_keys.end(), group.state_keys.begin(), group.state_keys.end());
    }
};

}  // namespace ribn_amd_dispatch
