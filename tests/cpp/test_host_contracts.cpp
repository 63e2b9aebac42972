// Host-contract tests of include/voidinfer_sampling.hpp, written the way the
// reference tests its own contracts (tests/test_exl3_sampling_policy.cpp,
// test_exl3_request_sampling_state.cpp, test_exl3_sampling_window_transaction.cpp,
// test_exl3_sampling_control_stop_semantics.cpp, test_exl3_greedy_packet.cpp,
// test_exl3_sampling_workspace_reservation.cpp, test_exl3_sampled_authority_boundary.cpp,
// test_exl3_draft_distribution_contract.cpp, test_exl3_sampled_acceptance_reference.cpp):
// the same scenarios and expectations against this library's types.
#include "voidinfer_sampling.hpp"

#include <array>
#include <initializer_list>
#include <cstdio>
#include <cstdlib>
#include <iostream>
#include <limits>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

using namespace voidinfer_amd;

namespace {
int failures = 0;
void need(bool ok, const char* what) {
    if (!ok) {
        std::cerr << "FAIL: " << what << "\n";
        ++failures;
    }
}
template <class E = std::exception, class F>
bool refuses(F&& call) {
    try { call(); } catch (const E&) { return true; } catch (...) { return false; }
    return false;
}

void test_resolve_sampling() {
    ModelSamplingDefaults d;
    d.thinking = SamplingPreset{0.6F, 20, 0.95F, 0.0F, 0.0F, 0.0F};
    d.non_thinking = SamplingPreset{0.7F, 20, 0.8F, 0.0F, 1.5F, 0.0F};
    auto r = resolve_sampling(d, SamplingMode::Thinking, {});
    need(r.temperature == 0.6F && r.top_k == 20 && r.top_p == 0.95F && r.seed == 0, "preset fills omitted fields");
    SamplingOverrides o;
    o.temperature = 0.0F;
    o.seed = 99;
    r = resolve_sampling(d, SamplingMode::NonThinking, o);
    need(r.temperature == 0.0F && r.presence_penalty == 1.5F && r.seed == 99, "explicit zero is a real override");
    using Edit = void (*)(SamplingOverrides&);
    for (Edit bad : std::initializer_list<Edit>{[](SamplingOverrides& x) { x.temperature = 2.5F; }, [](SamplingOverrides& x) { x.top_k = -1; },
                     [](SamplingOverrides& x) { x.top_p = 1.01F; }, [](SamplingOverrides& x) { x.min_p = -0.1F; },
                     [](SamplingOverrides& x) { x.presence_penalty = 2.5F; },
                     [](SamplingOverrides& x) { x.frequency_penalty = -3.0F; },
                     [](SamplingOverrides& x) { x.top_p = std::numeric_limits<float>::quiet_NaN(); }}) {
        SamplingOverrides x;
        bad(x);
        need(refuses<std::invalid_argument>([&] { (void)resolve_sampling(d, SamplingMode::Thinking, x); }),
             "out-of-range resolved parameter admitted");
    }
}

void test_policy() {
    ResolvedSamplingParameters greedy;
    greedy.temperature = 0;
    greedy.top_k = 0;
    greedy.top_p = 0;
    greedy.min_p = 1;
    auto policy = Exl3SamplingPolicy::normalize(greedy, 7);
    need(policy.greedy && policy.effective_top_k == 7 && policy.top_p_enabled && policy.min_p_enabled &&
             !policy.occurrence_counts_required,
         "greedy special case");
    auto sampled = greedy;
    sampled.temperature = 0.7F;
    sampled.top_k = 19;
    sampled.top_p = 0.8F;
    sampled.min_p = 0.1F;
    policy = Exl3SamplingPolicy::normalize(sampled);
    need(policy.requires_sampled_distribution() && policy.effective_top_k == 19 && policy.top_p_enabled &&
             policy.min_p_enabled,
         "positive-temperature filters");
    sampled.top_k = 20;
    need(Exl3SamplingPolicy::normalize(sampled).effective_top_k == 20, "top-k menu clamp at 20");
    sampled.top_k = 500;
    need(Exl3SamplingPolicy::normalize(sampled).effective_top_k == 20, "top-k above the menu");
    auto penalized = greedy;
    penalized.presence_penalty = 0.5F;
    need(Exl3SamplingPolicy::normalize(penalized).requires_sampled_distribution(),
         "temperature-zero penalty kept as sampled");
    auto invalid = sampled;
    invalid.top_p = 1.01F;
    need(refuses<std::invalid_argument>([&] { (void)Exl3SamplingPolicy::normalize(invalid); }), "top_p > 1");
    invalid = sampled;
    invalid.temperature = std::numeric_limits<float>::quiet_NaN();
    need(refuses<std::invalid_argument>([&] { (void)Exl3SamplingPolicy::normalize(invalid); }), "NaN temperature");
    need(refuses<std::invalid_argument>([&] { (void)Exl3SamplingPolicy::normalize(sampled, 0); }), "zero vocabulary");
    policy = Exl3SamplingPolicy::normalize(sampled, 3);
    const std::array<float, 3> finite{1, 2, 3};
    policy.require_logits(finite);
    auto nonfinite = finite;
    nonfinite[1] = std::numeric_limits<float>::infinity();
    need(refuses([&] { policy.require_logits(nonfinite); }) &&
             refuses([&] { policy.require_logits(std::span<const float>(finite).first(2)); }),
         "non-finite or short logits admitted");
    // routes
    const auto dev = policy.device_sampling();
    need(dev.top_k == 3 && dev.temperature == 0.7F && dev.sampled() && dev.active(), "coupled-route config");
    const auto row = Exl3SamplingPolicy::normalize(sampled).row_params(5, 1234, 1.1F);
    need(row.top_k == 500 && row.lane == 5 && row.position == 1234 && row.repetition_penalty == 1.1F,
         "batched-route row parameters");
}

void test_request_state() {
    auto revision = std::make_shared<const int>(1);
    auto next_revision = std::make_shared<const int>(2);
    Exl3RequestSamplingState request(11, 7, 0xabc, 123);
    request.bind_acquisition(41, revision, 64);
    auto first = request.begin(64);
    const auto draw0 = request.draw(first), draw1 = request.draw(first);
    need(draw0 == exl3_splitmix64(123ULL ^ 0xabcULL ^ 7ULL ^ 0ULL) &&
             draw1 == exl3_splitmix64(123ULL ^ 0xabcULL ^ 7ULL ^ 1ULL),
         "draw i is splitmix(seed ^ fingerprint ^ generation ^ i)");
    request.rollback(first);
    auto retry = request.begin(64);
    need(request.draw(retry) == draw0 && request.draw(retry) == draw1, "rollback replays");
    request.claim_publication(retry);
    request.commit(retry, 1, 65, next_revision);
    need(request.committed_draws() == 1 && request.committed_prefix() == 65, "partial commit");
    need(refuses<std::logic_error>([&] { (void)request.begin(64); }), "stale prefix opened a transaction");
    auto suffix = request.begin(65);
    need(request.draw(suffix) == draw1, "partial commit replays the first rejected draw");
    need(refuses<std::logic_error>([&] { (void)request.begin(65); }), "second open transaction");
    request.rollback(suffix);

    Exl3RequestSamplingState independent(11, 8, 0xabc, 123);
    independent.bind_acquisition(42, revision, 64);
    auto other = independent.begin(64);
    need(independent.draw(other) != draw0, "independent request shares the stream");
    independent.rollback(other);

    Exl3RequestSamplingState reload(12, 7, 0xabc, 123);
    reload.bind_acquisition(1, revision, 64);
    auto replay = reload.begin(64);
    need(reload.draw(replay) == draw0 &&
             reload.reproducibility() == Exl3SamplingReproducibility::seeded_request_replay_across_reload,
         "seeded replay across reload");
    reload.rollback(replay);

    auto cancelled = request.begin(65);
    request.cancel();
    need(request.cancelled() && refuses([&] { (void)request.draw(cancelled); }) &&
             refuses([&] { request.commit(cancelled, 0, 65, next_revision); }),
         "cancelled transaction drew or published");
    need(refuses([&] { request.bind_acquisition(99, revision, 65); }), "cancelled request rebound");
    need(refuses<std::invalid_argument>([] { Exl3RequestSamplingState s(0, 1, 1, 1); }), "zero identity admitted");
}

void test_window_transaction() {
    auto root = std::make_shared<const int>(1), root65 = std::make_shared<const int>(2);
    Exl3RequestSamplingState state(3, 5, 7, 11);
    state.bind_acquisition(13, root, 64);

    Exl3SamplingWindowTransaction rejected(state, 64, 8);
    (void)rejected.draw_proposal();
    (void)rejected.draw_acceptance();
    (void)rejected.reject_and_draw_correction();
    need(rejected.sealed() && refuses([&] { (void)rejected.draw_proposal(); }), "first rejection seals");
    rejected.claim_publication();
    rejected.commit(1, root65);
    need(state.committed_draws() == 3 && state.committed_prefix() == 65, "correction commits three draws");

    Exl3SamplingWindowTransaction aborted(state, 65, 4);
    const auto p1 = aborted.draw_proposal();
    const auto a1 = aborted.draw_acceptance();
    aborted.accept_proposal();
    const auto p2 = aborted.draw_proposal();
    const auto a2 = aborted.draw_acceptance();
    aborted.accept_proposal();
    aborted.rollback();
    Exl3SamplingWindowTransaction again(state, 65, 4);
    need(again.draw_proposal() == p1 && again.draw_acceptance() == a1, "abort consumed first decision");
    again.accept_proposal();
    need(again.draw_proposal() == p2 && again.draw_acceptance() == a2, "abort changed later decisions");
    again.accept_proposal();
    again.rollback();

    auto root67 = std::make_shared<const int>(3);
    Exl3SamplingWindowTransaction stopped(state, 65, 4);
    (void)stopped.draw_proposal();
    (void)stopped.draw_acceptance();
    stopped.accept_proposal();
    (void)stopped.draw_proposal();
    (void)stopped.draw_acceptance();
    stopped.accept_proposal();
    const auto up = stopped.draw_proposal();
    const auto ua = stopped.draw_acceptance();
    stopped.accept_proposal();
    stopped.seal_stop_boundary();
    stopped.claim_publication();
    stopped.commit(2, root67);
    need(state.committed_draws() == 7 && state.committed_prefix() == 67, "stop-truncated publication");
    Exl3SamplingWindowTransaction after(state, 67, 1);
    need(after.draw_proposal() == up && after.draw_acceptance() == ua, "unpublished decision replays");
    after.accept_proposal();
    need(refuses<std::logic_error>([&] { (void)after.draw_proposal(); }), "window capacity exceeded");
    after.rollback();
    need(refuses([&] { stopped.commit(0, root67); }), "window published twice");

    Exl3SamplingWindowTransaction order(state, 67, 2);
    need(refuses<std::logic_error>([&] { (void)order.draw_acceptance(); }), "acceptance before proposal");
    (void)order.draw_proposal();
    need(refuses<std::logic_error>([&] { order.accept_proposal(); }), "accept without acceptance draw");
    need(refuses<std::logic_error>([&] { order.seal_stop_boundary(); }), "stop inside a decision");
    need(refuses<std::logic_error>([&] { order.claim_publication(); }), "publication inside a decision");
    order.rollback();
}

void test_control_stop() {
    auto root = std::make_shared<const int>(1), control_root = std::make_shared<const int>(2);
    Exl3RequestSamplingState state(3, 5, 7, 11);
    state.bind_acquisition(13, root, 64);
    Exl3SamplingControlStopSemantics::commit_forced_control_after_resident(state, 2, control_root);
    need(state.committed_prefix() == 66 && state.committed_draws() == 0, "forced control consumed randomness");
    auto terminal_root = std::make_shared<const int>(3);
    Exl3SamplingWindowTransaction terminal(state, 66, 4);
    (void)terminal.draw_proposal();
    (void)terminal.draw_acceptance();
    terminal.accept_proposal();
    terminal.seal_stop_boundary();
    Exl3SamplingControlStopSemantics::claim_model_publication(terminal);
    const auto hidden =
        Exl3SamplingControlStopSemantics::commit_model_after_resident(terminal, 1, true, false, terminal_root);
    need(hidden.resident_tokens == 1 && hidden.visible_tokens == 0 && hidden.terminal && !hidden.terminal_visible &&
             state.committed_prefix() == 67 && state.committed_draws() == 2,
         "hidden terminal accounting");
    Exl3SamplingWindowTransaction before(state, 67, 2);
    const auto proposed = before.draw_proposal();
    const auto acceptance = before.draw_acceptance();
    Exl3SamplingControlStopSemantics::abandon_before_correction(before);
    Exl3SamplingWindowTransaction retry(state, 67, 2);
    need(retry.draw_proposal() == proposed && retry.draw_acceptance() == acceptance, "abandon consumed draws");
    retry.accept_proposal();
    retry.rollback();
    Exl3SamplingWindowTransaction claimed(state, 67, 1);
    (void)claimed.draw_proposal();
    (void)claimed.draw_acceptance();
    claimed.accept_proposal();
    Exl3SamplingControlStopSemantics::claim_model_publication(claimed);
    state.cancel();
    const auto visible = Exl3SamplingControlStopSemantics::commit_model_after_resident(
        claimed, 1, false, false, std::make_shared<const int>(4));
    need(visible.visible_tokens == 1 && state.committed_prefix() == 68, "claimed publication survives cancel");
    need(refuses([&] { state.advance_forced_control(1, root, false); }), "uncommitted forced control");
    need(refuses<std::invalid_argument>([&] {
             Exl3RequestSamplingState s(1, 1, 1, 1);
             s.bind_acquisition(1, root, 0);
             Exl3SamplingWindowTransaction w(s, 0, 1);
             (void)w.draw_proposal();
             (void)w.draw_acceptance();
             w.accept_proposal();
             w.claim_publication();
             (void)Exl3SamplingControlStopSemantics::commit_model_after_resident(w, 1, false, true, root);
         }),
         "terminal published without a terminal token");
}

void test_greedy_packet() {
    ::setenv("VOIDINFER_EXL3_DEVICE_GREEDY", "", 1);
    need(exl3_device_greedy_enabled(), "empty flag enables device greedy");
    ::setenv("VOIDINFER_EXL3_DEVICE_GREEDY", "0", 1);
    need(!exl3_device_greedy_enabled(), "0 disables");
    ::setenv("VOIDINFER_EXL3_DEVICE_GREEDY", "1", 1);
    need(exl3_device_greedy_enabled(), "1 enables");
    ::setenv("VOIDINFER_EXL3_DEVICE_GREEDY", "invalid", 1);
    need(refuses<std::invalid_argument>([] { (void)exl3_device_greedy_enabled(); }), "invalid flag");
    ::unsetenv("VOIDINFER_EXL3_DEVICE_GREEDY");
    for (unsigned rows : {1u, 8u, 16u}) {
        Exl3GreedyPacket packet;
        packet.rows = rows;
        packet.generation = 19;
        packet.position = 1024;
        packet.serial = 7;
        packet.ready = true;
        for (unsigned i = 0; i < rows; ++i) packet.decisions[i] = {7, static_cast<int>(100 + i), 0};
        auto validate = [](const Exl3GreedyPacket& p, unsigned n) { p.validate(n, 19, 1024, 7); };
        validate(packet, rows);
        const auto greedy = Exl3SelectionAuthorityRequirement::greedy(rows, 19, 1024, 7);
        greedy.validate(packet);
        std::vector<std::int64_t> path(rows);
        exl3_greedy_path(42, packet, path);
        need(path[0] == 42, "greedy path seed");
        for (unsigned i = 1; i < rows; ++i) need(path[i] == 99 + i, "greedy path decisions");
        const auto sampled = Exl3SelectionAuthorityRequirement::sampled(rows, 19, 1024, 7);
        need(refuses<std::invalid_argument>([&] { sampled.validate(packet); }), "packet satisfied sampled");
        Exl3SampledDistributionAuthority missing;
        missing.rows = rows;
        missing.vocabulary = 248320;
        missing.row_stride = 248320;
        missing.generation = 19;
        missing.position = 1024;
        missing.serial = 7;
        missing.ready = true;
        need(refuses<std::invalid_argument>([&] { sampled.validate(missing); }), "ownerless distribution");
        std::vector<float> probabilities(static_cast<std::size_t>(rows) * 248320);
        Exl3SampledDistributionAuthority dist{std::make_shared<int>(1), probabilities.data(), rows, 248320, 248320,
                                              19, 7, 1024, true};
        sampled.validate(dist);
        need(refuses<std::invalid_argument>([&] { greedy.validate(dist); }), "distribution satisfied greedy");
        auto bad = packet;
        bad.decisions[rows - 1].nonfinite = 1;
        need(refuses<std::runtime_error>([&] { validate(bad, rows); }), "non-finite last row");
        bad = packet; bad.decisions[rows - 1].serial = 6;
        need(refuses<std::runtime_error>([&] { validate(bad, rows); }), "stale row serial");
        bad = packet; bad.decisions[0].token = 248320;
        need(refuses<std::runtime_error>([&] { validate(bad, rows); }), "token out of range");
        bad = packet; bad.ready = false;
        need(refuses<std::runtime_error>([&] { validate(bad, rows); }), "not ready");
        bad = packet; bad.abi = 2;
        need(refuses<std::runtime_error>([&] { validate(bad, rows); }), "abi");
        bad = packet; ++bad.generation;
        need(refuses<std::runtime_error>([&] { validate(bad, rows); }), "generation");
        bad = packet; ++bad.position;
        need(refuses<std::runtime_error>([&] { validate(bad, rows); }), "position");
        bad = packet; ++bad.serial;
        need(refuses<std::runtime_error>([&] { validate(bad, rows); }), "serial");
        bad = packet; bad.rows = 0;
        need(refuses<std::runtime_error>([&] { validate(bad, rows); }), "zero rows");
        bad = packet; bad.rows = 17;
        need(refuses<std::runtime_error>([&] { validate(bad, rows); }), "17 rows");
        need(refuses<std::invalid_argument>([&] { exl3_greedy_path(42, packet, {}); }), "empty path");
        std::array<std::int64_t, 17> oversized{};
        need(refuses<std::invalid_argument>([&] { exl3_greedy_path(42, packet, oversized); }), "17-row path");
    }
    need(Exl3SelectionAuthorityRequirement::request(0, 0, 0).kind() == Exl3SelectionAuthorityKind::greedy_argmax &&
             Exl3SelectionAuthorityRequirement::request(0, 0, 0.1F).needs_sampled_distribution(),
         "request authority kind");
}

// Host-logit and device-packet greedy decisions (branch_reference.h:23-31,
// exact_outer_reference.h:14-36) over a stand-in text context.
struct FakeTextContext {
    std::vector<float> root;           // logits_host
    std::vector<float> continuation;   // continuation_logits_host: rows x 248320
    Exl3GreedyPacket packet;
    int packet_calls = 0, host_calls = 0;
    bool last_continuation = false;
    Exl3GreedyPacket greedy_packet(bool continuation_rows, void*) {
        ++packet_calls;
        last_continuation = continuation_rows;
        return packet;
    }
    std::vector<float> logits_host(void*) { ++host_calls; return root; }
    std::vector<float> continuation_logits_host(void*) { ++host_calls; return continuation; }
};

void test_host_greedy_path() {
    constexpr std::size_t V = 248320;
    const unsigned rows = 5;
    FakeTextContext ctx;
    ctx.root.assign(V, -3.0f);
    ctx.root[77] = 2.5f;
    ctx.root[9000] = 2.5f;   // a tie: the first index wins
    ctx.continuation.assign(rows * V, 0.0f);
    const std::array<std::int64_t, rows> argmax{11, 248319, 0, 123456, 5};
    for (unsigned r = 0; r < rows; ++r) {
        for (std::size_t i = 0; i < V; ++i) ctx.continuation[r * V + i] = -float((i * 2654435761u + r) % 1000) / 100.0f;
        ctx.continuation[r * V + std::size_t(argmax[r])] = 40.0f;
    }
    ctx.continuation[500] = 40.0f;   // row 0: a tie after its first largest entry
    ctx.packet.rows = rows;
    ctx.packet.generation = 3;
    ctx.packet.position = 64;
    ctx.packet.serial = 9;
    ctx.packet.ready = true;
    for (unsigned r = 0; r < rows; ++r) ctx.packet.decisions[r] = {9, static_cast<std::int32_t>(argmax[r]), 0};

    // Host route.
    ::setenv("VOIDINFER_EXL3_DEVICE_GREEDY", "0", 1);
    need(exl3_branch_greedy(ctx) == 77, "host branch greedy takes the first largest entry");
    std::array<std::int64_t, rows> host_path{};
    std::int64_t host_bonus = -1;
    exl3_outer_greedy_path(ctx, 42, std::span<std::int64_t>(host_path), nullptr, &host_bonus);
    need(host_path[0] == 42, "host path seed");
    for (unsigned r = 1; r < rows; ++r) need(host_path[r] == argmax[r - 1], "host path row decisions");
    need(host_bonus == argmax[rows - 1], "host deferred bonus is the last row's decision");
    need(ctx.packet_calls == 0, "host route reads no packet");
    {
        auto bad = ctx;
        bad.continuation[3 * V + 17] = std::numeric_limits<float>::infinity();
        need(refuses<std::runtime_error>([&] { exl3_outer_greedy_path(bad, 42, std::span<std::int64_t>(host_path), nullptr); }),
             "host path refuses +Inf");
        bad = ctx;
        bad.continuation[(rows - 1) * V + 2] = std::numeric_limits<float>::quiet_NaN();
        need(refuses<std::runtime_error>([&] { exl3_outer_greedy_path(bad, 42, std::span<std::int64_t>(host_path), nullptr); }),
             "host path refuses NaN in the bonus row");
        bad = ctx;
        bad.continuation.pop_back();
        need(refuses<std::runtime_error>([&] { exl3_outer_greedy_path(bad, 42, std::span<std::int64_t>(host_path), nullptr); }),
             "host path refuses mis-sized logits");
        bad = ctx;
        bad.root[5] = -std::numeric_limits<float>::infinity();
        need(refuses<std::runtime_error>([&] { (void)exl3_branch_greedy(bad); }), "host branch refuses -Inf");
        bad.root.clear();
        need(refuses<std::runtime_error>([&] { (void)exl3_branch_greedy(bad); }), "host branch refuses an empty row");
    }

    // Device route: the same decisions from the packet.
    ::setenv("VOIDINFER_EXL3_DEVICE_GREEDY", "1", 1);
    need(exl3_branch_greedy(ctx) == argmax[0], "device branch greedy is packet row 0");
    need(!ctx.last_continuation, "branch greedy asks for the root packet");
    std::array<std::int64_t, rows> dev_path{};
    std::int64_t dev_bonus = -1;
    exl3_outer_greedy_path(ctx, 42, std::span<std::int64_t>(dev_path), nullptr, &dev_bonus);
    need(ctx.last_continuation, "outer path asks for the continuation packet");
    need(dev_path == host_path && dev_bonus == host_bonus, "device and host routes agree");
    {
        auto stale = ctx;
        stale.packet.decisions[rows - 1].nonfinite = 1;
        need(refuses<std::runtime_error>([&] { exl3_outer_greedy_path(stale, 42, std::span<std::int64_t>(dev_path), nullptr); }),
             "device path refuses a non-finite bonus row");
    }
    need(refuses<std::invalid_argument>([&] { exl3_outer_greedy_path(ctx, 42, std::span<std::int64_t>(), nullptr); }),
         "empty path");
    ::unsetenv("VOIDINFER_EXL3_DEVICE_GREEDY");
}

void test_workspace_and_admission() {
    ResolvedSamplingParameters values;
    auto policy = Exl3SamplingPolicy::normalize(values, 248320);
    const auto current = Exl3DraftDistributionAvailability::current_dflash2();
    const auto greedy = Exl3SamplingWorkspacePlan::derive(policy, current, 8, 4096);
    need(!greedy.sampled && !greedy.device_bytes &&
             !greedy.requirement().units[static_cast<unsigned>(Exl3ResourceInventory::Domain::device)],
         "greedy reserved workspace");
    values.temperature = .8F;
    policy = Exl3SamplingPolicy::normalize(values, 248320);
    need(refuses<std::invalid_argument>([&] { (void)Exl3SamplingWorkspacePlan::derive(policy, current, 8, 4096); }),
         "sampled plan without q");
    auto capable = current;
    capable.normalized_q_available = true;
    capable.complete_vocabulary_support = true;
    capable.conditioning = Exl3DraftDistributionConditioning::autoregressive_predecessor;
    const auto plan = Exl3SamplingWorkspacePlan::derive(policy, capable, 8, 4096);
    need(plan.target_probability_bytes == 8ULL * 248320 * 4 && plan.device_bytes == 3 * plan.target_probability_bytes + 4096,
         "probability workspace bytes");
    auto a = std::make_shared<int>(1), b = std::make_shared<int>(2);
    Exl3ResourceInventory::Allocation alloc_a{a, 0, Exl3ResourceInventory::Domain::device, plan.device_bytes};
    Exl3ResourceInventory::Allocation alloc_b{b, 0, Exl3ResourceInventory::Domain::device, plan.device_bytes};
    auto first = Exl3SamplingWorkspaceAuthority::from_reserved_allocation(plan, alloc_a, a.get(), 11, 13, 17);
    auto second = Exl3SamplingWorkspaceAuthority::from_reserved_allocation(plan, alloc_b, b.get(), 12, 19, 23);
    need(first.matches(plan, 11, 13, 17) && second.matches(plan, 12, 19, 23) && !first.matches(plan, 12, 19, 23) &&
             first.owner() != second.owner(),
         "workspaces aliased");
    auto wrong = alloc_b;
    wrong.units--;
    need(refuses<std::invalid_argument>([&] {
             (void)Exl3SamplingWorkspaceAuthority::from_reserved_allocation(plan, wrong, b.get(), 12, 19, 23);
         }),
         "under-reserved workspace");
    values.presence_penalty = .5F;
    policy = Exl3SamplingPolicy::normalize(values, 248320);
    const auto counted = Exl3SamplingWorkspacePlan::derive(policy, capable, 8, 0);
    need(counted.occurrence_count_bytes == 248320ULL * 4 &&
             counted.device_bytes == 3 * counted.target_probability_bytes + counted.occurrence_count_bytes,
         "occurrence table budget");
    need(refuses<std::overflow_error>([&] {
             (void)Exl3SamplingWorkspacePlan::derive(policy, capable, 8, std::numeric_limits<std::uint64_t>::max());
         }),
         "workspace size overflow");

    // admission gates, in order
    ResolvedSamplingParameters v;
    Exl3SampledAdmissionRequest req{Exl3SamplingPolicy::normalize(v, 3), Exl3DraftDistributionAvailability::current_dflash2()};
    need(Exl3SampledAuthorityBoundary::decide(req).greedy(), "greedy request");
    v.temperature = .7F;
    req.policy = Exl3SamplingPolicy::normalize(v, 3);
    need(Exl3SampledAuthorityBoundary::decide(req).disposition ==
             Exl3SampledAdmissionDisposition::draft_distribution_unavailable,
         "missing q");
    req.draft_availability = capable;
    need(Exl3SampledAuthorityBoundary::decide(req).disposition ==
             Exl3SampledAdmissionDisposition::public_sampled_disabled,
         "public scope");
    auto root = std::make_shared<const int>(1);
    Exl3RequestSamplingState state(2, 11, 17, 23);
    state.bind_acquisition(29, root, 31);
    auto owner = std::make_shared<std::array<float, 6>>();
    Exl3DraftDistributionAuthority q;
    q.method = Exl3SampledAcceptanceMethod::independent_rejection_with_residual;
    q.conditioning = Exl3DraftDistributionConditioning::autoregressive_predecessor;
    q.owner = owner; q.probabilities = owner->data(); q.rows = 2; q.vocabulary = 3; q.row_stride = 3;
    q.request_generation = 11; q.root_revision = 37; q.first_position = 31;
    q.normalized = q.complete_vocabulary_support = q.ready = true;
    Exl3SampledDistributionAuthority p{owner, owner->data(), 2, 3, 3, 11, 41, 31, true};
    req.exposure = Exl3SampledApiExposure::unqualified_source_api;
    need(Exl3SampledAuthorityBoundary::decide(req).disposition ==
             Exl3SampledAdmissionDisposition::request_state_unavailable,
         "missing request state");
    req.request_state = &state; req.rows = 2; req.vocabulary = 3; req.request_generation = 11;
    req.root_revision = 37; req.target_serial = 41; req.first_position = 31; req.acquisition = 29;
    need(Exl3SampledAuthorityBoundary::decide(req).disposition ==
             Exl3SampledAdmissionDisposition::draft_distribution_invalid,
         "missing q authority");
    req.draft_q = &q;
    need(Exl3SampledAuthorityBoundary::decide(req).disposition ==
             Exl3SampledAdmissionDisposition::target_distribution_unavailable,
         "missing p authority");
    req.target_p = &p;
    need(Exl3SampledAuthorityBoundary::decide(req).disposition ==
             Exl3SampledAdmissionDisposition::workspace_unavailable,
         "missing workspace");
    const auto wplan = Exl3SamplingWorkspacePlan::derive(req.policy, req.draft_availability, 2, 64);
    Exl3ResourceInventory::Allocation walloc{owner, 1, Exl3ResourceInventory::Domain::device, wplan.device_bytes};
    auto ws = Exl3SamplingWorkspaceAuthority::from_reserved_allocation(wplan, walloc, owner.get(), 11, 37, 29);
    req.workspace_plan = &wplan;
    req.workspace = &ws;
    const auto ready = Exl3SampledAuthorityBoundary::decide(req);
    need(ready.unqualified_source_ready() && !ready.publicly_enabled(), "source-ready stays unqualified");
    auto stale = q;
    stale.root_revision = 38;
    req.draft_q = &stale;
    need(Exl3SampledAuthorityBoundary::decide(req).disposition ==
             Exl3SampledAdmissionDisposition::draft_distribution_invalid,
         "stale q admitted");
    req.draft_q = &q;
    auto stale_p = p;
    stale_p.serial = 40;
    req.target_p = &stale_p;
    need(Exl3SampledAuthorityBoundary::decide(req).disposition ==
             Exl3SampledAdmissionDisposition::target_distribution_invalid,
         "stale p admitted");
    req.target_p = &p;
    state.cancel();
    need(Exl3SampledAuthorityBoundary::decide(req).disposition ==
             Exl3SampledAdmissionDisposition::request_state_unavailable,
         "cancelled request admitted");
    need(Exl3SampledAuthorityBoundary::message(Exl3SampledAdmissionDisposition::greedy).size() > 0, "messages");
}

void test_acceptance_and_prefix() {
    const std::array<double, 2> pa{0.6, 0.4}, qa{0.5, 0.5};
    auto r = Exl3IndependentAcceptanceReference::evaluate(pa, qa, 0, 0.999, 0.25);
    need(r.accepted && !r.correction_draw_used && r.token == 0 && r.acceptance_probability == 1 && r.residual.empty(),
         "p/q capped at one");
    const std::array<double, 2> pr{0.2, 0.8};
    r = Exl3IndependentAcceptanceReference::evaluate(pr, qa, 0, 0.5, 0.75);
    need(!r.accepted && r.correction_draw_used && r.token == 1 && std::abs(r.acceptance_probability - 0.4) < 1e-12 &&
             r.residual[0] == 0 && r.residual[1] == 1,
         "normalized residual");
    const std::array<double, 2> pg{0.25, 0.75}, qg{0, 1};
    r = Exl3IndependentAcceptanceReference::evaluate(pg, qg, 1, 0.9, 0.0);
    need(!r.accepted && r.token == 0 && r.residual[0] == 1 && r.residual[1] == 0, "target-only support");
    const std::array<double, 3> pz{0, 0.5, 0.5}, qz{0, 0.25, 0.75};
    need(refuses<std::invalid_argument>([&] { (void)Exl3IndependentAcceptanceReference::evaluate(pz, qz, 0, .5, .5); }),
         "zero-q proposal");
    const std::array<double, 2> same{0.5, 0.5};
    r = Exl3IndependentAcceptanceReference::evaluate(same, same, 1, 0.999999, 0.5);
    need(r.accepted && !r.correction_draw_used, "identical distributions");
    auto malformed = pa;
    malformed[0] = std::numeric_limits<double>::infinity();
    const std::array<double, 2> unnorm{0.4, 0.4};
    need(refuses([&] { (void)Exl3IndependentAcceptanceReference::evaluate(malformed, qa, 0, .1, .1); }) &&
             refuses([&] { (void)Exl3IndependentAcceptanceReference::evaluate(unnorm, qa, 0, .1, .1); }) &&
             refuses([&] { (void)Exl3IndependentAcceptanceReference::evaluate(pa, qa, 0, 1.0, .1); }),
         "invalid probability or draw");
    // residual of a rejection that leaves no mass: p == q except the proposal
    // cannot happen (p/q >= 1 accepts), so only round-off reaches it — refused.

    const std::array<std::int64_t, 3> t{5, 6, 7}, ok{5, 6, 7}, miss{5, 9, 7};
    auto d = decide_exl3_outer_prefix(t, ok);
    need(d.committed_tokens == std::vector<std::int64_t>{5, 6, 7} && d.accepted == 3 && !d.rejected && !d.stopped,
         "full prefix");
    d = decide_exl3_outer_prefix(t, miss);
    need(d.committed_tokens == std::vector<std::int64_t>{5, 6} && d.accepted == 1 && d.rejected, "mismatch");
    const std::array<std::int64_t, 1> term{6};
    d = decide_exl3_outer_prefix(t, ok, term);
    need(d.committed_tokens == std::vector<std::int64_t>{5, 6} && d.accepted == 2 && d.stopped, "terminal");
    need(refuses<std::invalid_argument>([&] { (void)decide_exl3_outer_prefix({}, {}); }), "empty decision");

    // sibling promotion: chain [s, a, b] with siblings at offsets {1, 1, 2}
    const std::array<std::int64_t, 6> tentative{10, 11, 12, 20, 21, 22};
    const std::array<std::int64_t, 3> chain_target{10, 21, 30};
    d = decide_exl3_outer_prefix(std::span(chain_target), std::span(tentative).first(3));
    need(d.accepted == 1 && d.rejected, "chain rejected at depth 1");
    const std::array<int, 3> offsets{1, 1, 2};
    const std::array<std::int64_t, 3> sibling_next{40, 41, 42};
    const int promoted = exl3_promote_sibling(d, tentative, 3, offsets, sibling_next);
    need(promoted == 4 && d.accepted == 2 && d.committed_tokens == std::vector<std::int64_t>{10, 21, 41},
         "sibling at the rejected depth continues");
    auto d2 = decide_exl3_outer_prefix(std::span(chain_target), std::span(tentative).first(3));
    const std::array<std::int64_t, 1> stop41{41};
    (void)exl3_promote_sibling(d2, tentative, 3, offsets, sibling_next, stop41);
    need(d2.stopped, "promoted terminal stops");
    auto d3 = decide_exl3_outer_prefix(std::span(chain_target), std::span(tentative).first(3), stop41);
    const std::array<std::int64_t, 3> other_target{10, 99, 30};
    auto d4 = decide_exl3_outer_prefix(std::span(other_target), std::span(tentative).first(3));
    need(exl3_promote_sibling(d4, tentative, 3, offsets, sibling_next) == -1 && d4.accepted == 1,
         "no sibling matches the correction");
    (void)d3;
}

void test_vericache() {
    const std::array<std::int64_t, 5> tokens{1, 2, 3, 4, 5};
    std::array<Exl3RowScore, 5> s{};
    for (int i = 0; i < 5; ++i) s[i] = {tokens[i + 1 < 5 ? i + 1 : 4], 0.0F};
    s[1].gap = 0.05F;
    auto d = exl3_vericache_decide(tokens, s, 0.0625F);
    need(d.reject == 5 && d.correction == -1 && d.tokens.size() == 5 && d.max_gap == 0.05F, "all kept within delta");
    s[2] = {77, 0.5F};
    d = exl3_vericache_decide(tokens, s, 0.0625F);
    need(d.reject == 3 && d.correction == 77 && d.tokens == std::vector<std::int64_t>{1, 2, 3, 77}, "gap refusal");
    s[2] = {77, 0.0F};
    d = exl3_vericache_decide(tokens, s, 0.0F);
    need(d.reject == 3 && d.correction == 77, "exact mode compares tokens");
    need(exl3_vericache_delta("1") == 0.0625F && exl3_vericache_delta("exact") == 0.0625F &&
             exl3_vericache_delta("tolerance") == 1.0F && exl3_vericache_delta("1", "0.25") == 0.25F,
         "delta modes");
    need(refuses<std::invalid_argument>([] { (void)exl3_vericache_delta("2"); }) &&
             refuses<std::invalid_argument>([] { (void)exl3_vericache_delta("1", "-1"); }),
         "invalid VeriCache mode");
}

}  // namespace

int main() {
    test_resolve_sampling();
    test_policy();
    test_request_state();
    test_window_transaction();
    test_control_stop();
    test_greedy_packet();
    test_host_greedy_path();
    test_workspace_and_admission();
    test_acceptance_and_prefix();
    test_vericache();
    if (failures) {
        std::cerr << failures << " host contract check(s) failed\n";
        return 1;
    }
    std::cout << "host contracts PASS\n";
    return 0;
}
