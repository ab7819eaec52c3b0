// Host-only tests of the serving dispatcher's bookkeeping
// (engine_amd/csrc/serving_submissions.hpp), after the reference's
// submissions.rs tests (failed_drain_retains_all_resources_until_teardown,
// successful_drain_retires_resources_but_keeps_dispatcher_poisoned) and
// serving.rs nonadjacent_group_slots_return_to_original_positions.
// Built and run by tests/test_serving.py with g++; prints "ok" on success.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <memory>

#include "serving_submissions.hpp"

using ribn_amd_dispatch::QueuedRows;
using ribn_amd_dispatch::Submissions;

#define CHECK(c)                                                     \
    do {                                                             \
        if (!(c)) {                                                  \
            std::fprintf(stderr, "%s:%d: %s\n", __FILE__, __LINE__, #c); \
            std::exit(1);                                            \
        }                                                            \
    } while (0)

// Counts destructions, like the reference's Drop-counting Resource.
struct Resource {
    std::shared_ptr<int> drops;
    explicit Resource(std::shared_ptr<int> d) : drops(std::move(d)) {}
    Resource(Resource&& o) noexcept : drops(std::move(o.drops)) {}
    Resource& operator=(Resource&& o) noexcept {
        release();
        drops = std::move(o.drops);
        return *this;
    }
    Resource(const Resource&) = delete;
    ~Resource() { release(); }
    void release() {
        if (drops) ++*drops;
        drops.reset();
    }
};

static void failed_drain_retains_everything_until_teardown() {
    auto drops = std::make_shared<int>(0);
    {
        Submissions<Resource> s;
        s.pending.emplace(1, Resource(drops));
        s.quarantine(Resource(drops));
        std::vector<Resource> retired = s.fail("event query failed", false);
        CHECK(retired.empty());
        CHECK(s.pending.empty());
        CHECK(s.fault() != nullptr);
        CHECK(!s.release_is_safe());
        CHECK(s.quarantined() == 2);
        CHECK(*drops == 0);
    }
    CHECK(*drops == 2);  // teardown releases the quarantined records
}

static void successful_drain_retires_but_stays_poisoned() {
    Submissions<int> s;
    s.pending.emplace(1, 7);
    s.quarantine(8);
    std::vector<int> retired = s.fail("pinned read failed", true);
    std::sort(retired.begin(), retired.end());
    CHECK((retired == std::vector<int>{7, 8}));
    CHECK(s.pending.empty());
    CHECK(s.release_is_safe());
    CHECK(s.fault() != nullptr);
    CHECK(std::string(s.fault()) == "pinned read failed");
    // a later failure replaces the message and keeps the dispatcher poisoned
    s.fail("second", true);
    CHECK(std::string(s.fault()) == "second");
}

static void take_all_returns_pending_and_quarantined() {
    Submissions<int> s;
    s.pending.emplace(3, 30);
    s.quarantine(40);
    std::vector<int> all = s.take_all();
    std::sort(all.begin(), all.end());
    CHECK((all == std::vector<int>{30, 40}));
    CHECK(s.pending.empty() && s.quarantined() == 0);
    CHECK(s.fault() == nullptr && s.release_is_safe());
}

static void nonadjacent_group_slots_return_to_original_positions() {
    QueuedRows rows;
    rows.outputs.assign(3, -1);
    rows.elapsed.assign(3, 0);
    QueuedRows group;
    group.outputs = {7, 3};
    group.elapsed = {11, 19};
    group.state_keys = {5, 6};
    rows.scatter({0, 2}, std::move(group));
    CHECK((rows.outputs == std::vector<int32_t>{7, -1, 3}));
    CHECK((rows.elapsed == std::vector<uint64_t>{11, 0, 19}));
    CHECK((rows.state_keys == std::vector<uint64_t>{5, 6}));
}

int main() {
    failed_drain_retains_everything_until_teardown();
    successful_drain_retires_but_stays_poisoned();
    take_all_returns_pending_and_quarantined();
    nonadjacent_group_slots_return_to_original_positions();
    std::puts("ok");
    return 0;
}
