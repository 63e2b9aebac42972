// CPU test of the C++ layer's greedy-packet transport (Exl3GreedyPacketTransport,
// Exl3PendingGreedyPacket) in include/voidinfer_sampling.hpp: submit / finish,
// cross-lane batches split and validated per lane, stale identities, pool
// exhaustion, and dropping an unfinished packet.  The five vi_packet_* entry
// points are replaced here by a host stand-in (plain memory, copies at submit)
// so that the layer's logic runs without a GPU; the real entry points are
// exercised on the GPU by tests/test_gpu_transport.py.
#include <cstdio>
#include <cstring>
#include <vector>

#include "voidinfer_sampling.hpp"

using namespace voidinfer_amd;

// ---- host stand-in for the transport entry points (test double) ----
struct vi_packet_transport {
    struct Slot { std::vector<vi_greedy_row> rows; bool busy = false; };
    std::vector<Slot> slots;
    int max_rows = 0;
};
extern "C" {
vi_status vi_packet_transport_create(int slots, int max_rows, vi_packet_transport** out) {
    if (slots <= 0 || max_rows <= 0 || !out) return VI_ERR_INVALID;
    *out = new vi_packet_transport;
    (*out)->slots.resize(std::size_t(slots));
    (*out)->max_rows = max_rows;
    return VI_OK;
}
vi_status vi_packet_transport_destroy(vi_packet_transport* t) { delete t; return VI_OK; }
vi_status vi_packet_submit(vi_packet_transport* t, const vi_greedy_row* rows, int n, void*, int* slot) {
    if (n <= 0 || n > t->max_rows) return VI_ERR_INVALID;
    for (std::size_t i = 0; i < t->slots.size(); ++i)
        if (!t->slots[i].busy) {
            t->slots[i].rows.assign(rows, rows + n);
            t->slots[i].busy = true;
            *slot = int(i);
            return VI_OK;
        }
    return VI_ERR_WORKSPACE;
}
vi_status vi_packet_query(vi_packet_transport* t, int slot, int* ready) {
    if (slot < 0 || slot >= int(t->slots.size()) || !t->slots[std::size_t(slot)].busy) return VI_ERR_INVALID;
    *ready = 1;
    return VI_OK;
}
vi_status vi_packet_finish(vi_packet_transport* t, int slot, vi_greedy_row* out, int n) {
    auto& s = t->slots[std::size_t(slot)];
    if (!s.busy || n != int(s.rows.size())) return VI_ERR_INVALID;
    std::memcpy(out, s.rows.data(), sizeof(vi_greedy_row) * std::size_t(n));
    s.busy = false;
    return VI_OK;
}
const char* vi_status_string(vi_status) { return "status"; }
}

static int failures = 0;
#define CHECK(c) do { if (!(c)) { std::printf("FAIL %s:%d %s\n", __FILE__, __LINE__, #c); ++failures; } } while (0)
template <class E, class F> static bool throws(F&& f) {
    try { f(); } catch (const E&) { return true; } catch (...) { return false; }
    return false;
}

static std::vector<Exl3GreedyRow> rows_for(std::uint64_t serial, int n, int token0) {
    std::vector<Exl3GreedyRow> r(static_cast<std::size_t>(n));
    for (int i = 0; i < n; ++i) r[std::size_t(i)] = Exl3GreedyRow{serial, token0 + i, 0u};
    return r;
}

int main() {
    {   // one context: submit, poll, finish, validate
        Exl3GreedyPacketTransport t(2, 16);
        auto r = rows_for(7, 3, 100);
        auto p = t.submit(r.data(), 3, /*generation=*/4, /*position=*/50, /*serial=*/7, nullptr);
        CHECK(p.valid() && t.ready(p));
        const Exl3GreedyPacket g = t.finish(std::move(p), 4, 50, 7);
        CHECK(g.rows == 3 && g.decisions[2].token == 102 && g.serial == 7 && !p.valid());
    }
    {   // stale: the context moved on (serial / position / generation) before finish
        Exl3GreedyPacketTransport t(2, 16);
        auto r = rows_for(9, 1, 5);
        CHECK(throws<std::runtime_error>([&] { (void)t.finish(t.submit(r.data(), 1, 1, 10, 9, nullptr), 1, 10, 10); }));
        CHECK(throws<std::runtime_error>([&] { (void)t.finish(t.submit(r.data(), 1, 1, 10, 9, nullptr), 1, 11, 9); }));
        CHECK(throws<std::runtime_error>([&] { (void)t.finish(t.submit(r.data(), 1, 1, 10, 9, nullptr), 2, 10, 9); }));
        // the slots were freed by the failed finishes: two more submits fit
        auto a = t.submit(r.data(), 1, 1, 10, 9, nullptr);
        auto b = t.submit(r.data(), 1, 1, 10, 9, nullptr);
        CHECK(a.valid() && b.valid());
        // pool exhausted
        CHECK(throws<Exl3ResourceReservationExhausted>([&] { (void)t.submit(r.data(), 1, 1, 10, 9, nullptr); }));
        { auto drop = std::move(a); }   // dropping an unfinished packet frees its slot
        auto c = t.submit(r.data(), 1, 1, 10, 9, nullptr);
        CHECK(c.valid());
    }
    {   // a row from another serial, a non-finite row, an out-of-range token
        Exl3GreedyPacketTransport t(1, 16);
        auto r = rows_for(3, 2, 10);
        r[1].serial = 2;
        CHECK(throws<std::runtime_error>([&] { (void)t.finish(t.submit(r.data(), 2, 0, 0, 3, nullptr), 0, 0, 3); }));
        r = rows_for(3, 2, 10);
        r[0].nonfinite = 1;
        CHECK(throws<std::runtime_error>([&] { (void)t.finish(t.submit(r.data(), 2, 0, 0, 3, nullptr), 0, 0, 3); }));
        r = rows_for(3, 2, 10);
        r[1].token = 248320;
        CHECK(throws<std::runtime_error>([&] { (void)t.finish(t.submit(r.data(), 2, 0, 0, 3, nullptr), 0, 0, 3); }));
    }
    {   // a batch: three lanes' packets end to end, one copy, validated per lane
        Exl3GreedyPacketTransport t(1, 64);
        std::vector<Exl3GreedyRow> all;
        for (auto [serial, n, tok] : {std::tuple{11ull, 1, 1}, std::tuple{12ull, 16, 100}, std::tuple{13ull, 4, 900}}) {
            auto r = rows_for(serial, n, tok);
            all.insert(all.end(), r.begin(), r.end());
        }
        const std::vector<Exl3PendingGreedyPacket::Member> m{{1, 1, 5, 11}, {16, 2, 6, 12}, {4, 3, 7, 13}};
        auto p = t.submit_batch(all.data(), m, nullptr);
        CHECK(p.members().size() == 3);
        const auto g = t.finish_batch(std::move(p));
        CHECK(g.size() == 3 && g[1].rows == 16 && g[1].decisions[15].token == 115 && g[2].position == 7 &&
              g[2].decisions[0].token == 900 && g[0].generation == 1);
        // a member's rows belong to another member: that lane's validation fails
        std::swap(all[0], all[1]);
        CHECK(throws<std::runtime_error>([&] { (void)t.finish_batch(t.submit_batch(all.data(), m, nullptr)); }));
        // rows outside 1..16 or serial 0 are refused before anything is copied
        const std::vector<Exl3PendingGreedyPacket::Member> bad{{17, 1, 1, 1}};
        CHECK(throws<std::invalid_argument>([&] { (void)t.submit_batch(all.data(), bad, nullptr); }));
        const std::vector<Exl3PendingGreedyPacket::Member> zero{{1, 1, 1, 0}};
        CHECK(throws<std::invalid_argument>([&] { (void)t.submit_batch(all.data(), zero, nullptr); }));
    }
    if (failures) return 1;
    std::printf("transport host layer PASS\n");
    return 0;
}
