// GPU test of the engine-facing launchers of include/voidinfer_sampling.hpp,
// linked against libvoidinfer_sampling.so and called the way the engine calls
// them: exl3_launch_greedy_packet, Exl3GreedyPacketTransport (single packet and
// batch), exl3_presence_reset / _record / _truncate, exl3_launch_sampled_packet
// over that presence table, dflash2_topk16_for_test (with the library's own
// scratch and with a caller's), dflash_sampled_choices.  Inputs and the CPU
// oracle's outputs come from the fixture directory given as argv[1]
// (written by tests/test_gpu_launchers.py): raw little-endian arrays, one file
// each, and meta.txt with the scalar parameters.
#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstring>
#include <fstream>
#include <iostream>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "voidinfer_sampling.hpp"

using namespace voidinfer_amd;

namespace {
int failures = 0;
void need(bool ok, const std::string& what) {
    if (!ok) {
        std::cerr << "FAIL: " << what << "\n";
        ++failures;
    }
}
void hip(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        std::cerr << "HIP error " << hipGetErrorString(e) << " at " << what << "\n";
        std::exit(2);
    }
}

std::string dir;
std::map<std::string, long long> meta;

template <class T>
std::vector<T> load(const std::string& name) {
    std::ifstream f(dir + "/" + name, std::ios::binary | std::ios::ate);
    if (!f) { std::cerr << "missing fixture " << name << "\n"; std::exit(2); }
    const auto bytes = static_cast<std::size_t>(f.tellg());
    std::vector<T> v(bytes / sizeof(T));
    f.seekg(0);
    f.read(reinterpret_cast<char*>(v.data()), std::streamsize(bytes));
    return v;
}
void load_meta() {
    std::ifstream f(dir + "/meta.txt");
    std::string line;
    while (std::getline(f, line)) {
        const auto eq = line.find('=');
        if (eq != std::string::npos) meta[line.substr(0, eq)] = std::stoll(line.substr(eq + 1));
    }
}
double meta_f(const std::string& key) {   // floats are stored as their bits
    const long long b = meta.at(key);
    float f;
    const std::uint32_t u = std::uint32_t(b);
    std::memcpy(&f, &u, 4);
    return f;
}

template <class T>
T* upload(const std::vector<T>& v) {
    T* d = nullptr;
    hip(hipMalloc(reinterpret_cast<void**>(&d), std::max<std::size_t>(v.size(), 1) * sizeof(T)), "malloc");
    hip(hipMemcpy(d, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice), "upload");
    return d;
}
template <class T>
std::vector<T> download(const T* d, std::size_t n) {
    std::vector<T> v(n);
    hip(hipMemcpy(v.data(), d, n * sizeof(T), hipMemcpyDeviceToHost), "download");
    return v;
}
void* zeroed(std::size_t bytes) {
    void* d = nullptr;
    hip(hipMalloc(&d, std::max<std::size_t>(bytes, 1)), "malloc");
    hip(hipMemset(d, 0, std::max<std::size_t>(bytes, 1)), "memset");
    return d;
}

void test_greedy_and_transport(hipStream_t stream) {
    const int rows = int(meta.at("greedy_rows")), V = int(meta.at("greedy_vocab"));
    const auto bits = load<std::uint16_t>("greedy_logits.bin");
    const auto want_tok = load<std::int32_t>("greedy_tokens.bin");
    const auto want_nf = load<std::uint32_t>("greedy_nonfinite.bin");
    const std::uint64_t serial = std::uint64_t(meta.at("greedy_serial"));
    const std::uint16_t* d_bits = upload(bits);
    const std::size_t sb = Exl3GreedySplitScratch::bytes(rows, V);
    const auto scratch = Exl3GreedySplitScratch::carve(zeroed(sb), sb);
    Exl3GreedyRow* d_out = nullptr;
    hip(hipMalloc(reinterpret_cast<void**>(&d_out), sizeof(Exl3GreedyRow) * rows), "malloc");
    for (int rep = 0; rep < 2; ++rep) {   // (the scratch is reusable without clearing)
        exl3_launch_greedy_packet(false, rows, stream, d_bits, V, V, serial, d_out, scratch);
        hip(hipStreamSynchronize(stream), "greedy");
        const auto got = download(d_out, std::size_t(rows));
        for (int r = 0; r < rows; ++r) {
            need(got[r].token == want_tok[r], "greedy token row " + std::to_string(r));
            need(got[r].nonfinite == want_nf[r], "greedy nonfinite row " + std::to_string(r));
            need(got[r].serial == serial, "greedy serial row " + std::to_string(r));
        }
    }
    // readback through the transport: the clean rows as one packet, then as a
    // batch of two lanes' packets
    const int clean = int(meta.at("greedy_clean_rows"));
    Exl3GreedyPacketTransport transport(2, 16);
    auto pending = transport.submit(d_out, clean, 7, 4096, serial, stream);
    const Exl3GreedyPacket pkt = transport.finish(std::move(pending), 7, 4096, serial, V);
    for (int r = 0; r < clean; ++r) need(pkt.decisions[std::size_t(r)].token == want_tok[r], "transport row");
    std::vector<std::int64_t> path(static_cast<std::size_t>(clean));
    exl3_greedy_path(42, pkt, path);
    need(path[0] == 42 && (clean < 2 || path[1] == want_tok[0]), "greedy path from the transported packet");
    const int first = clean / 2;
    const Exl3PendingGreedyPacket::Member members[2] = {{first, 7, 100, serial}, {clean - first, 8, 200, serial}};
    auto batch = transport.submit_batch(d_out, members, stream);
    const auto packets = transport.finish_batch(std::move(batch), V);
    need(packets.size() == 2, "batch packets");
    for (int r = 0; r < clean; ++r) {
        const auto& p = packets[r < first ? 0 : 1];
        need(p.decisions[std::size_t(r < first ? r : r - first)].token == want_tok[r], "batch row");
    }
    bool stale = false;
    try {
        auto again = transport.submit(d_out, clean, 7, 4096, serial, stream);
        (void)transport.finish(std::move(again), 7, 4097, serial, V);
    } catch (const std::runtime_error&) {
        stale = true;
    }
    need(stale, "a stale packet is refused");
    hip(hipFree(d_out), "free");
}

void test_presence_and_sampled_packet(hipStream_t stream) {
    const int V = int(meta.at("packet_vocab")), rows = int(meta.at("packet_rows"));
    const auto bits = load<std::uint16_t>("packet_logits.bin");
    const auto hist = load<std::int64_t>("presence_tokens.bin");
    const auto want_table = load<std::int32_t>("presence_table.bin");
    const auto depths = load<std::int32_t>("packet_depths.bin");
    const auto inputs = load<std::int32_t>("packet_inputs.bin");
    const auto want_tok = load<std::int32_t>("packet_tokens.bin");
    std::int32_t* table = static_cast<std::int32_t*>(zeroed(sizeof(std::int32_t) * std::size_t(V)));
    const std::int64_t* d_hist = upload(hist);
    exl3_presence_reset(table, stream, V);
    exl3_presence_record(table, int(meta.at("presence_first")), d_hist, hist.size(), stream, V);
    exl3_presence_truncate(table, int(meta.at("presence_truncate")), stream, V);
    hip(hipStreamSynchronize(stream), "presence");
    need(download(table, std::size_t(V)) == want_table, "presence table after reset / record / truncate");

    Exl3DeviceSampling cfg;
    cfg.temperature = float(meta_f("packet_temperature"));
    cfg.top_k = int(meta.at("packet_top_k"));
    cfg.top_p = float(meta_f("packet_top_p"));
    cfg.min_p = float(meta_f("packet_min_p"));
    cfg.seed = std::uint64_t(meta.at("packet_seed"));
    cfg.presence_penalty = float(meta_f("packet_presence"));
    cfg.first_occurrence = table;
    const std::uint16_t* d_bits = upload(bits);
    const std::size_t sb = Exl3SampledSliceScratch::bytes(rows, V);
    const auto scratch = Exl3SampledSliceScratch::carve(zeroed(sb), sb);
    Exl3GreedyRow* d_out = nullptr;
    hip(hipMalloc(reinterpret_cast<void**>(&d_out), sizeof(Exl3GreedyRow) * rows), "malloc");
    exl3_launch_sampled_packet(rows, stream, d_bits, V, V, cfg, int(meta.at("packet_first_key")), depths, inputs,
                               5, d_out, scratch);
    hip(hipStreamSynchronize(stream), "sampled packet");
    const auto got = download(d_out, std::size_t(rows));
    const auto near = load<std::uint8_t>("packet_near.bin");   // oracle rows within rounding of a boundary
    for (int r = 0; r < rows; ++r)
        need(near[std::size_t(r)] || got[r].token == want_tok[r], "sampled packet row " + std::to_string(r));
    hip(hipFree(d_out), "free");
}

void test_topk16(hipStream_t stream) {
    const int rows = int(meta.at("topk_rows")), V = int(meta.at("topk_vocab"));
    const auto bits = load<std::uint16_t>("topk_logits.bin");
    const auto want_ids = load<std::int64_t>("topk_ids.bin");
    const auto want_vals = load<float>("topk_values.bin");
    const std::uint16_t* d_bits = upload(bits);
    std::int64_t* ids = nullptr;
    float* vals = nullptr;
    hip(hipMalloc(reinterpret_cast<void**>(&ids), sizeof(std::int64_t) * rows * 16), "malloc");
    hip(hipMalloc(reinterpret_cast<void**>(&vals), sizeof(float) * rows * 16), "malloc");
    unsigned int* flag = static_cast<unsigned int*>(zeroed(4));
    // the reference's call shape (the library's scratch), then a caller's scratch
    for (int with_scratch = 0; with_scratch < 2; ++with_scratch) {
        Exl3TopkScratch scratch;
        if (with_scratch) {
            scratch.size = vi_topk_workspace_bytes(rows, V, 16);
            scratch.base = zeroed(scratch.size);
        }
        hip(hipMemset(ids, 0xff, sizeof(std::int64_t) * rows * 16), "memset");
        dflash2_topk16_for_test(d_bits, rows, V, ids, vals, true, true, stream, flag, scratch);
        hip(hipStreamSynchronize(stream), "top-16");
        const auto gi = download(ids, std::size_t(rows) * 16);
        const auto gv = download(vals, std::size_t(rows) * 16);
        for (std::size_t i = 0; i < gi.size(); ++i) {
            need(gi[i] == want_ids[i], "top-16 id " + std::to_string(i));
            need(std::memcmp(&gv[i], &want_vals[i], 4) == 0, "top-16 value " + std::to_string(i));
        }
    }
    need(download(flag, 1)[0] == std::uint32_t(meta.at("topk_nonfinite")), "top-16 non-finite flag");
}

void test_draft_choices(hipStream_t stream) {
    const int lanes = int(meta.at("draft_lanes")), positions = int(meta.at("draft_positions"));
    const int V = int(meta.at("draft_vocab"));
    const auto scores = load<float>("draft_scores.bin");
    const auto cands = load<std::int64_t>("draft_candidates.bin");
    const auto seeds = load<std::int64_t>("draft_seed_tokens.bin");
    const auto want = load<std::int64_t>("draft_proposals.bin");
    const auto smp = load<DraftSelectSampling>("draft_sampling.bin");   // (no first-occurrence tables)
    need(smp.size() == std::size_t(lanes), "draft sampling records");
    const float* d_scores = upload(scores);
    const std::int64_t* d_cands = upload(cands);
    const std::int64_t* d_seeds = upload(seeds);
    const DraftSelectSampling* d_smp = upload(smp);
    std::int64_t* d_out = nullptr;
    hip(hipMalloc(reinterpret_cast<void**>(&d_out), sizeof(std::int64_t) * lanes * positions), "malloc");
    dflash_sampled_choices(lanes, positions, d_scores, d_cands, d_seeds, d_smp, d_out, stream, V);
    hip(hipStreamSynchronize(stream), "draft choices");
    need(download(d_out, std::size_t(lanes) * positions) == want, "draft proposals");
}
}  // namespace

int main(int argc, char** argv) {
    if (argc < 2) {
        std::cerr << "usage: test_launchers_gpu FIXTURE_DIR\n";
        return 2;
    }
    dir = argv[1];
    load_meta();
    if (vi_init() != VI_OK) {
        std::cerr << "device is not gfx950\n";
        return 2;
    }
    hipStream_t stream;
    hip(hipStreamCreate(&stream), "stream");
    test_greedy_and_transport(stream);
    test_presence_and_sampled_packet(stream);
    test_topk16(stream);
    test_draft_choices(stream);
    hip(hipStreamDestroy(stream), "stream");
    if (failures) {
        std::cerr << failures << " launcher check(s) failed\n";
        return 1;
    }
    std::cout << "launchers PASS\n";
    return 0;
}
