// ref_diff.cpp — differential test of this library's C++20 host layer
// (include/voidinfer_sampling.hpp) against the reference's own host-only headers,
// compiled from where they lie under /root/reference (oracle/Makefile, target
// `diff`, output oracle/_ref/ref_diff).  Test infrastructure only.
//
// Random scripts drive both implementations side by side and compare every
// observable: returned values, state accessors and the exception class of each
// refused call (invalid_argument / logic_error / overflow_error / runtime_error).
#include "exl3/greedy_packet.h"
#include "exl3/request_sampling_state.h"
#include "exl3/sampled_acceptance_reference.h"
#include "exl3/sampled_authority_boundary.h"
#include "exl3/sampling_control_stop_semantics.h"
#include "exl3/sampling_policy.h"
#include "exl3/sampling_window_transaction.h"
#include "exl3/sampling_workspace_reservation.h"
#include "exl3/verification_tree.h"
#include "runtime/contract/sampling.h"

#include "../include/voidinfer_sampling.hpp"

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <limits>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

namespace R = voidinfer::exl3;
namespace RR = voidinfer::runtime;
namespace M = voidinfer_amd;

namespace {

struct Rng {
    std::uint64_t s;
    std::uint64_t next() {
        s += 0x9e3779b97f4a7c15ULL;
        std::uint64_t z = s;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
        return z ^ (z >> 31);
    }
    int below(int n) { return int(next() % std::uint64_t(n)); }
    double unit() { return double(next() >> 11) * 0x1.0p-53; }
    bool coin(int percent = 50) { return below(100) < percent; }
};

// 0 = returned, 1 invalid_argument, 2 logic_error, 3 overflow_error, 4 runtime_error, 5 other
template <class F>
int outcome(F&& f) {
    try { f(); return 0; }
    catch (const std::invalid_argument&) { return 1; }
    catch (const std::logic_error&) { return 2; }
    catch (const std::overflow_error&) { return 3; }
    catch (const std::runtime_error&) { return 4; }
    catch (...) { return 5; }
}

int mismatches = 0;
long checks = 0;
void same(bool ok, const char* what, long index) {
    ++checks;
    if (!ok && mismatches++ < 20) std::fprintf(stderr, "MISMATCH %s (case %ld)\n", what, index);
}

float pick_float(Rng& g, std::initializer_list<float> menu) {
    const int i = g.below(int(menu.size()));
    return *(menu.begin() + i);
}

// ---------------------------------------------------------------- policy / resolve
void diff_policy(Rng& g, long n) {
    const float nan = std::numeric_limits<float>::quiet_NaN(), inf = std::numeric_limits<float>::infinity();
    for (long c = 0; c < n; ++c) {
        RR::ResolvedSamplingParameters r;
        M::ResolvedSamplingParameters m;
        r.temperature = m.temperature = pick_float(g, {0.0F, 0.3F, 0.7F, 1.2F, 2.0F, 2.01F, -0.1F, nan});
        r.top_k = m.top_k = std::vector<int>{0, 1, 5, 19, 20, 21, 100, -1}[g.below(8)];
        r.top_p = m.top_p = pick_float(g, {0.0F, 0.5F, 0.95F, 1.0F, 1.01F, -0.01F, inf});
        r.min_p = m.min_p = pick_float(g, {0.0F, 0.05F, 1.0F, 1.5F, -1.0F});
        r.presence_penalty = m.presence_penalty = pick_float(g, {0.0F, 0.5F, -2.0F, 2.0F, 2.5F, -inf});
        r.frequency_penalty = m.frequency_penalty = pick_float(g, {0.0F, -0.3F, 2.0F, -2.5F, nan});
        r.seed = m.seed = g.next();
        const std::uint32_t v = std::vector<std::uint32_t>{0, 1, 3, 7, 19, 20, 248320}[g.below(7)];
        R::Exl3NormalizedSamplingPolicy rp;
        M::Exl3NormalizedSamplingPolicy mp;
        const int ro = outcome([&] { rp = R::Exl3SamplingPolicy::normalize(r, v); });
        const int mo = outcome([&] { mp = M::Exl3SamplingPolicy::normalize(m, v); });
        same(ro == mo, "normalize outcome", c);
        if (ro == 0 && mo == 0)
            same(rp.vocabulary == mp.vocabulary && rp.effective_top_k == mp.effective_top_k &&
                     rp.greedy == mp.greedy && rp.top_p_enabled == mp.top_p_enabled &&
                     rp.min_p_enabled == mp.min_p_enabled &&
                     rp.occurrence_counts_required == mp.occurrence_counts_required &&
                     rp.requires_sampled_distribution() == mp.requires_sampled_distribution(),
                 "normalize fields", c);
        if (ro == 0 && mo == 0 && v > 0 && v < 64) {
            std::vector<float> logits(v + g.below(2));
            for (auto& x : logits) x = g.coin(95) ? float(g.unit()) : inf;
            same(outcome([&] { rp.require_logits(logits); }) == outcome([&] { mp.require_logits(logits); }),
                 "require_logits", c);
        }
        // resolve
        voidinfer::ModelSamplingDefaults rd;
        M::ModelSamplingDefaults md;
        rd.thinking = {r.temperature, r.top_k, r.top_p, r.min_p, r.presence_penalty, r.frequency_penalty};
        md.thinking = {m.temperature, m.top_k, m.top_p, m.min_p, m.presence_penalty, m.frequency_penalty};
        rd.non_thinking = {0.5F, 3, 0.9F, 0.0F, 0.0F, 0.0F};
        md.non_thinking = {0.5F, 3, 0.9F, 0.0F, 0.0F, 0.0F};
        voidinfer::SamplingOverrides ro_;
        M::SamplingOverrides mo_;
        if (g.coin()) { const float t = pick_float(g, {0.0F, 1.0F, 3.0F}); ro_.temperature = t; mo_.temperature = t; }
        if (g.coin()) { const int k = std::vector<int>{0, 7, -2}[g.below(3)]; ro_.top_k = k; mo_.top_k = k; }
        if (g.coin()) { const float p = pick_float(g, {0.8F, 1.0F, 2.0F}); ro_.top_p = p; mo_.top_p = p; }
        if (g.coin(20)) { ro_.min_p = 0.1F; mo_.min_p = 0.1F; }
        if (g.coin(20)) { ro_.presence_penalty = 0.2F; mo_.presence_penalty = 0.2F; }
        if (g.coin(20)) { ro_.frequency_penalty = -0.2F; mo_.frequency_penalty = -0.2F; }
        if (g.coin()) { const auto s = g.next(); ro_.seed = s; mo_.seed = s; }
        const bool thinking = g.coin();
        RR::ResolvedSamplingParameters rres;
        M::ResolvedSamplingParameters mres;
        const int a = outcome([&] {
            rres = RR::resolve_sampling(rd, thinking ? voidinfer::SamplingMode::Thinking
                                                     : voidinfer::SamplingMode::NonThinking, ro_);
        });
        const int b = outcome([&] {
            mres = M::resolve_sampling(md, thinking ? M::SamplingMode::Thinking : M::SamplingMode::NonThinking, mo_);
        });
        same(a == b, "resolve outcome", c);
        if (a == 0 && b == 0)
            same(rres.temperature == mres.temperature && rres.top_k == mres.top_k &&
                     rres.top_p == mres.top_p && rres.min_p == mres.min_p &&
                     rres.presence_penalty == mres.presence_penalty &&
                     rres.frequency_penalty == mres.frequency_penalty && rres.seed == mres.seed,
                 "resolve fields", c);
    }
}

// ---------------------------------------------------------------- acceptance
void diff_acceptance(Rng& g, long n) {
    for (long c = 0; c < n; ++c) {
        const int v = 1 + g.below(12);
        std::vector<double> p(v), q(v);
        double sp = 0, sq = 0;
        for (int i = 0; i < v; ++i) {
            p[i] = g.coin(80) ? g.unit() : 0.0;
            q[i] = g.coin(80) ? g.unit() : 0.0;
            sp += p[i];
            sq += q[i];
        }
        for (int i = 0; i < v; ++i) { p[i] = sp > 0 ? p[i] / sp : 1.0 / v; q[i] = sq > 0 ? q[i] / sq : 1.0 / v; }
        if (g.coin(10)) q = p;                                    // identical
        if (g.coin(5)) p[g.below(v)] += 1e-6;                      // not normalized
        if (g.coin(3)) q[g.below(v)] = std::numeric_limits<double>::quiet_NaN();
        std::uint32_t tok = std::uint32_t(g.below(v + (g.coin(5) ? 1 : 0)));
        double ua = g.coin(3) ? 1.0 : g.unit(), uc = g.coin(3) ? -0.5 : g.unit();
        if (v > 1 && g.coin(5)) {
            // near-identical p and q: a rejection whose residual mass sits at the 1e-9 cut
            q = p;
            const int i = g.below(v), j = (i + 1) % v;
            const double eps = g.coin() ? 1e-12 : 2e-9;
            if (p[i] > eps) { p[i] -= eps; p[j] += eps; tok = std::uint32_t(i); ua = 0x1.fffffffffffffp-1; }
        }
        std::span<const double> ps(p), qs(q);
        if (g.coin(3)) qs = qs.first(qs.size() > 1 ? qs.size() - 1 : 1);
        R::Exl3SampledAcceptanceOutcome ro;
        M::Exl3SampledAcceptanceOutcome mo;
        const int a = outcome([&] { ro = R::Exl3IndependentAcceptanceReference::evaluate(ps, qs, tok, ua, uc); });
        const int b = outcome([&] { mo = M::Exl3IndependentAcceptanceReference::evaluate(ps, qs, tok, ua, uc); });
        same(a == b, "acceptance outcome", c);
        if (a == 0 && b == 0)
            same(ro.accepted == mo.accepted && ro.correction_draw_used == mo.correction_draw_used &&
                     ro.token == mo.token && ro.acceptance_probability == mo.acceptance_probability &&
                     ro.residual == mo.residual,
                 "acceptance fields", c);
    }
}

// ---------------------------------------------------------------- request state + windows
struct Pair {
    R::Exl3RequestSamplingState r;
    M::Exl3RequestSamplingState m;
    std::optional<R::Exl3RequestSamplingState::Transaction> rt;
    std::optional<M::Exl3RequestSamplingState::Transaction> mt;
    Pair(std::uint64_t e, std::uint64_t gen, std::uint64_t f, std::uint64_t s) : r(e, gen, f, s), m(e, gen, f, s) {}
};

void diff_request_state(Rng& g, long n) {
    for (long c = 0; c < n; ++c) {
        const std::uint64_t e = 1 + g.below(3), gen = 1 + g.below(5), f = 1 + g.next() % 1000, s = g.next();
        Pair st(e, gen, f, s);
        std::vector<std::shared_ptr<const int>> roots;
        for (int i = 0; i < 3; ++i) roots.push_back(std::make_shared<const int>(i));
        std::size_t expect_prefix = 0;
        for (int step = 0; step < 40; ++step) {
            const int op = g.below(9);
            int a = -1, b = -1;
            std::uint64_t ra = 0, mb = 0;
            switch (op) {
                case 0: {
                    const std::uint64_t acq = g.below(3);
                    const auto root = g.coin(90) ? roots[g.below(3)] : nullptr;
                    expect_prefix = std::size_t(g.below(4));
                    a = outcome([&] { st.r.bind_acquisition(acq, root, expect_prefix); });
                    b = outcome([&] { st.m.bind_acquisition(acq, root, expect_prefix); });
                    break;
                }
                case 1: {
                    const std::size_t pre = g.coin(80) ? st.r.committed_prefix() : std::size_t(g.below(5));
                    a = outcome([&] { st.rt = st.r.begin(pre); });
                    b = outcome([&] { st.mt = st.m.begin(pre); });
                    break;
                }
                case 2: case 3:
                    if (!st.rt || !st.mt) continue;
                    a = outcome([&] { ra = st.r.draw(*st.rt); });
                    b = outcome([&] { mb = st.m.draw(*st.mt); });
                    same(ra == mb, "draw value", c);
                    break;
                case 4:
                    if (!st.rt || !st.mt) continue;
                    a = outcome([&] { st.r.claim_publication(*st.rt); });
                    b = outcome([&] { st.m.claim_publication(*st.mt); });
                    break;
                case 5: {
                    if (!st.rt || !st.mt) continue;
                    const std::uint64_t k = std::uint64_t(g.below(4));
                    const std::size_t pre = st.r.committed_prefix() + std::size_t(g.below(3)) - (g.coin(10) ? 1 : 0);
                    const auto root = g.coin(90) ? roots[g.below(3)] : nullptr;
                    a = outcome([&] { st.r.commit(*st.rt, k, pre, root); });
                    b = outcome([&] { st.m.commit(*st.mt, k, pre, root); });
                    break;
                }
                case 6:
                    if (!st.rt || !st.mt) continue;
                    a = outcome([&] { st.r.rollback(*st.rt); });
                    b = outcome([&] { st.m.rollback(*st.mt); });
                    break;
                case 7: {
                    const std::size_t t = std::size_t(g.below(3));
                    const bool res = g.coin(85);
                    const auto root = roots[g.below(3)];
                    a = outcome([&] { st.r.advance_forced_control(t, root, res); });
                    b = outcome([&] { st.m.advance_forced_control(t, root, res); });
                    break;
                }
                case 8:
                    if (g.coin(15)) { st.r.cancel(); st.m.cancel(); }
                    continue;
            }
            same(a == b, "request-state step outcome", c * 100 + step);
            same(st.r.committed_draws() == st.m.committed_draws() &&
                     st.r.committed_prefix() == st.m.committed_prefix() && st.r.cancelled() == st.m.cancelled(),
                 "request-state accessors", c * 100 + step);
        }
    }
}

void diff_windows(Rng& g, long n) {
    for (long c = 0; c < n; ++c) {
        const std::uint64_t seed = g.next();
        auto root = std::make_shared<const int>(1);
        R::Exl3RequestSamplingState rs(3, 5, 7, seed);
        M::Exl3RequestSamplingState ms(3, 5, 7, seed);
        rs.bind_acquisition(13, root, 64);
        ms.bind_acquisition(13, root, 64);
        for (int w = 0; w < 6; ++w) {
            const std::size_t cap = std::size_t(1 + g.below(5));
            const std::size_t pre = g.coin(90) ? rs.committed_prefix() : rs.committed_prefix() + 1;
            std::unique_ptr<R::Exl3SamplingWindowTransaction> rw;
            std::unique_ptr<M::Exl3SamplingWindowTransaction> mw;
            const int a0 = outcome([&] { rw = std::make_unique<R::Exl3SamplingWindowTransaction>(rs, pre, cap); });
            const int b0 = outcome([&] { mw = std::make_unique<M::Exl3SamplingWindowTransaction>(ms, pre, cap); });
            same(a0 == b0, "window open", c);
            if (!rw || !mw) continue;
            for (int step = 0; step < 14; ++step) {
                const int op = g.below(10);
                int a = 0, b = 0;
                std::uint64_t x = 0, y = 0;
                if (op <= 2) { a = outcome([&] { x = rw->draw_proposal(); }); b = outcome([&] { y = mw->draw_proposal(); }); }
                else if (op <= 4) { a = outcome([&] { x = rw->draw_acceptance(); }); b = outcome([&] { y = mw->draw_acceptance(); }); }
                else if (op == 5) { a = outcome([&] { rw->accept_proposal(); }); b = outcome([&] { mw->accept_proposal(); }); }
                else if (op == 6) { a = outcome([&] { x = rw->reject_and_draw_correction(); }); b = outcome([&] { y = mw->reject_and_draw_correction(); }); }
                else if (op == 7) { a = outcome([&] { rw->seal_stop_boundary(); }); b = outcome([&] { mw->seal_stop_boundary(); }); }
                else if (op == 8) { a = outcome([&] { rw->claim_publication(); }); b = outcome([&] { mw->claim_publication(); }); }
                else {
                    const std::size_t k = std::size_t(g.below(4));
                    auto nr = std::make_shared<const int>(step);
                    if (g.coin(50)) {
                        a = outcome([&] { rw->commit(k, nr); });
                        b = outcome([&] { mw->commit(k, nr); });
                        if (a == 0) root = nr;
                    } else {
                        a = outcome([&] { rw->rollback(); });
                        b = outcome([&] { mw->rollback(); });
                    }
                }
                same(a == b && x == y, "window step", c * 1000 + w * 20 + step);
                same(rw->sealed() == mw->sealed() && rw->decided_tokens() == mw->decided_tokens() &&
                         rs.committed_draws() == ms.committed_draws() &&
                         rs.committed_prefix() == ms.committed_prefix(),
                     "window accessors", c * 1000 + w * 20 + step);
            }
            if (g.coin(20)) {
                auto nr = std::make_shared<const int>(99);
                const std::size_t t = std::size_t(g.below(3));
                const bool terminal = g.coin(), publish = g.coin();
                R::Exl3SamplingPublicationCount rc;
                M::Exl3SamplingPublicationCount mc;
                const int a = outcome([&] { rc = R::Exl3SamplingControlStopSemantics::commit_model_after_resident(*rw, t, terminal, publish, nr); });
                const int b = outcome([&] { mc = M::Exl3SamplingControlStopSemantics::commit_model_after_resident(*mw, t, terminal, publish, nr); });
                same(a == b && rc.resident_tokens == mc.resident_tokens && rc.visible_tokens == mc.visible_tokens &&
                         rc.terminal == mc.terminal && rc.terminal_visible == mc.terminal_visible,
                     "stop-semantics commit", c);
                if (a == 0) root = nr;
            }
        }
    }
}

// ---------------------------------------------------------------- greedy packet
void diff_packets(Rng& g, long n) {
    for (long c = 0; c < n; ++c) {
        R::Exl3GreedyPacket rp;
        M::Exl3GreedyPacket mp;
        const std::uint32_t rows = std::uint32_t(g.below(18));
        rp.rows = mp.rows = rows;
        rp.generation = mp.generation = 19;
        rp.position = mp.position = 1024;
        rp.serial = mp.serial = g.coin(95) ? 7 : 0;
        rp.ready = mp.ready = g.coin(95);
        rp.abi = mp.abi = g.coin(97) ? 1u : 2u;
        for (unsigned i = 0; i < 16; ++i) {
            const std::uint64_t s = g.coin(97) ? 7 : 6;
            const int t = g.coin(97) ? g.below(248320) : (g.coin() ? -1 : 248320);
            const std::uint32_t nf = g.coin(97) ? 0 : 1;
            rp.decisions[i] = {s, t, nf};
            mp.decisions[i] = {s, t, nf};
        }
        const std::uint32_t er = g.coin(90) ? rows : rows + 1;
        const std::uint64_t eg = g.coin(95) ? 19 : 18;
        const int epos = g.coin(95) ? 1024 : 1023;
        const int vocab = g.coin(95) ? 248320 : 0;
        const int a = outcome([&] { rp.validate(er, eg, epos, 7, vocab); });
        const int b = outcome([&] { mp.validate(er, eg, epos, 7, vocab); });
        same(a == b, "packet validate", c);
        std::vector<std::int64_t> pr(std::size_t(g.below(18))), pm(pr.size());
        const std::int64_t seed = g.coin(95) ? 42 : 248320;
        const int a2 = outcome([&] { R::exl3_greedy_path(seed, rp, pr); });
        const int b2 = outcome([&] { M::exl3_greedy_path(seed, mp, pm); });
        same(a2 == b2 && (a2 != 0 || pr == pm), "greedy path", c);
    }
}

// ---------------------------------------------------------------- workspace + admission
void diff_admission(Rng& g, long n) {
    for (long c = 0; c < n; ++c) {
        RR::ResolvedSamplingParameters r;
        M::ResolvedSamplingParameters m;
        r.temperature = m.temperature = g.coin(20) ? 0.0F : 0.8F;
        r.presence_penalty = m.presence_penalty = g.coin(30) ? 0.5F : 0.0F;
        const std::uint32_t v = g.coin() ? 3 : 248320;
        const auto rpol = R::Exl3SamplingPolicy::normalize(r, v);
        const auto mpol = M::Exl3SamplingPolicy::normalize(m, v);
        R::Exl3DraftDistributionAvailability ra;
        M::Exl3DraftDistributionAvailability ma;
        if (g.coin(20)) { ra = R::Exl3DraftDistributionAvailability::current_dflash2(); ma = M::Exl3DraftDistributionAvailability::current_dflash2(); }
        else {
            ra.normalized_q_available = ma.normalized_q_available = g.coin(90);
            ra.complete_vocabulary_support = ma.complete_vocabulary_support = g.coin(90);
            const bool ar = g.coin(90);
            ra.conditioning = ar ? R::Exl3DraftDistributionConditioning::autoregressive_predecessor
                                 : R::Exl3DraftDistributionConditioning::parallel_masked_target_taps;
            ma.conditioning = ar ? M::Exl3DraftDistributionConditioning::autoregressive_predecessor
                                 : M::Exl3DraftDistributionConditioning::parallel_masked_target_taps;
        }
        const std::uint32_t rows = std::uint32_t(g.below(4));
        const std::uint64_t transient = g.coin(95) ? std::uint64_t(g.below(100000)) : std::numeric_limits<std::uint64_t>::max();
        R::Exl3SamplingWorkspacePlan rplan;
        M::Exl3SamplingWorkspacePlan mplan;
        const int a = outcome([&] { rplan = R::Exl3SamplingWorkspacePlan::derive(rpol, ra, rows, transient); });
        const int b = outcome([&] { mplan = M::Exl3SamplingWorkspacePlan::derive(mpol, ma, rows, transient); });
        same(a == b, "workspace plan outcome", c);
        if (a != 0 || b != 0) continue;
        same(rplan.sampled == mplan.sampled && rplan.occurrence_counts == mplan.occurrence_counts &&
                 rplan.device_bytes == mplan.device_bytes && rplan.configuration == mplan.configuration &&
                 rplan.target_probability_bytes == mplan.target_probability_bytes &&
                 rplan.occurrence_count_bytes == mplan.occurrence_count_bytes &&
                 rplan.requirement().units[0] == mplan.requirement().units[0],
             "workspace plan fields", c);
        // admission with random defects
        auto owner = std::make_shared<std::vector<float>>(8, 0.25F);
        auto root = std::make_shared<const int>(1);
        R::Exl3RequestSamplingState rs(2, 11, 17, 23);
        M::Exl3RequestSamplingState ms(2, 11, 17, 23);
        rs.bind_acquisition(29, root, 31);
        ms.bind_acquisition(29, root, 31);
        if (g.coin(10)) { rs.cancel(); ms.cancel(); }
        R::Exl3DraftDistributionAuthority rq;
        M::Exl3DraftDistributionAuthority mq;
        const bool good_method = g.coin(95), good_cond = g.coin(95);
        rq.method = good_method ? R::Exl3SampledAcceptanceMethod::independent_rejection_with_residual : R::Exl3SampledAcceptanceMethod::unspecified;
        mq.method = good_method ? M::Exl3SampledAcceptanceMethod::independent_rejection_with_residual : M::Exl3SampledAcceptanceMethod::unspecified;
        rq.conditioning = good_cond ? R::Exl3DraftDistributionConditioning::autoregressive_predecessor : R::Exl3DraftDistributionConditioning::parallel_masked_target_taps;
        mq.conditioning = good_cond ? M::Exl3DraftDistributionConditioning::autoregressive_predecessor : M::Exl3DraftDistributionConditioning::parallel_masked_target_taps;
        rq.owner = mq.owner = owner;
        rq.probabilities = mq.probabilities = owner->data();
        rq.rows = mq.rows = g.coin(95) ? rows : rows + 1;
        rq.vocabulary = mq.vocabulary = v;
        rq.row_stride = mq.row_stride = g.coin(95) ? v : v - 1;
        rq.request_generation = mq.request_generation = 11;
        rq.root_revision = mq.root_revision = g.coin(95) ? 37 : 38;
        rq.first_position = mq.first_position = 31;
        rq.normalized = mq.normalized = g.coin(95);
        rq.complete_vocabulary_support = mq.complete_vocabulary_support = true;
        rq.ready = mq.ready = g.coin(95);
        R::Exl3SampledDistributionAuthority rp{owner, owner->data(), rows, v, v, 11, std::uint64_t(g.coin(95) ? 41 : 40), 31, g.coin(95)};
        M::Exl3SampledDistributionAuthority mp{owner, owner->data(), rows, v, v, 11, rp.serial, 31, rp.ready};
        R::Exl3SampledAdmissionRequest rr{rpol, ra};
        M::Exl3SampledAdmissionRequest mr{mpol, ma};
        const bool exposed = g.coin(90);
        rr.exposure = exposed ? R::Exl3SampledApiExposure::unqualified_source_api : R::Exl3SampledApiExposure::public_greedy_only;
        mr.exposure = exposed ? M::Exl3SampledApiExposure::unqualified_source_api : M::Exl3SampledApiExposure::public_greedy_only;
        if (g.coin(95)) { rr.request_state = &rs; mr.request_state = &ms; }
        if (g.coin(95)) { rr.draft_q = &rq; mr.draft_q = &mq; }
        if (g.coin(95)) { rr.target_p = &rp; mr.target_p = &mp; }
        rr.rows = mr.rows = rows;
        rr.vocabulary = mr.vocabulary = v;
        rr.request_generation = mr.request_generation = g.coin(95) ? 11 : 12;
        rr.root_revision = mr.root_revision = 37;
        rr.target_serial = mr.target_serial = 41;
        rr.first_position = mr.first_position = g.coin(95) ? 31 : 30;
        rr.acquisition = mr.acquisition = 29;
        std::optional<R::Exl3SamplingWorkspaceAuthority> rw;
        std::optional<M::Exl3SamplingWorkspaceAuthority> mw;
        if (rplan.sampled && g.coin(90)) {
            const std::uint64_t units = g.coin(95) ? rplan.device_bytes : rplan.device_bytes - 1;
            R::Exl3ResourceInventory::Allocation ralloc;
            ralloc.owner = owner; ralloc.slot = 1; ralloc.domain = R::Exl3ResourceInventory::Domain::device; ralloc.units = units;
            M::Exl3ResourceInventory::Allocation malloc_{owner, 1, M::Exl3ResourceInventory::Domain::device, units};
            const std::uint64_t gen = g.coin(95) ? 11 : 10;
            const int wa = outcome([&] { rw.emplace(R::Exl3SamplingWorkspaceAuthority::from_reserved_allocation(rplan, ralloc, owner.get(), gen, 37, 29)); });
            const int wb = outcome([&] { mw.emplace(M::Exl3SamplingWorkspaceAuthority::from_reserved_allocation(mplan, malloc_, owner.get(), gen, 37, 29)); });
            same(wa == wb, "workspace authority outcome", c);
            if (rw && mw) { rr.workspace = &*rw; mr.workspace = &*mw; }
            rr.workspace_plan = &rplan;
            mr.workspace_plan = &mplan;
        }
        const auto rd = R::Exl3SampledAuthorityBoundary::decide(rr);
        const auto md = M::Exl3SampledAuthorityBoundary::decide(mr);
        same(static_cast<int>(rd.disposition) == static_cast<int>(md.disposition) &&
                 rd.publicly_enabled() == md.publicly_enabled() &&
                 rd.unqualified_source_ready() == md.unqualified_source_ready(),
             "admission disposition", c);
    }
}

}  // namespace

// Verification trees: random top-16 candidate sets with planted ties (equal
// unary values, repeated probability deciles), chain tokens inside or outside
// the candidates, budgets 0..12, sibling caps -1..5, the default and zero row
// costs.
void diff_trees(Rng& g, long n) {
    for (long i = 0; i < n; ++i) {
        const int depth = g.below(9);
        std::vector<std::int64_t> drafts(static_cast<std::size_t>(depth)), ids(static_cast<std::size_t>(depth) * 16);
        std::vector<float> unary(static_cast<std::size_t>(depth) * 16);
        for (int d = 0; d < depth; ++d) {
            const int spread = 1 + g.below(4);
            for (int c = 0; c < 16; ++c) {
                ids[std::size_t(d) * 16 + std::size_t(c)] = 1000 + g.below(40);
                unary[std::size_t(d) * 16 + std::size_t(c)] = g.coin(30) ? float(g.below(3)) : float(g.unit() * 6.0 * spread);
            }
            drafts[std::size_t(d)] = g.coin(80) ? ids[std::size_t(d) * 16 + std::size_t(g.below(16))] : 5;
        }
        const int budget = g.below(13), max_sib = g.below(7) - 1;
        const float cost = g.coin(25) ? 0.0f : (g.coin(50) ? M::kExl3TreeRowCost : float(g.unit() * 0.2));
        const auto a = M::exl3_build_verification_tree(drafts, ids, unary, budget, max_sib, cost);
        const auto b = R::exl3_build_verification_tree(drafts, ids, unary, budget, max_sib, cost);
        same(a.chain_drafts == b.chain_drafts, "tree chain", i);
        same(a.sibling_tokens == b.sibling_tokens, "tree sibling tokens", i);
        same(a.sibling_offsets == b.sibling_offsets, "tree sibling offsets", i);
    }
}

int main(int argc, char** argv) {
    const long n = argc > 1 ? std::atol(argv[1]) : 20000;
    Rng g{0x5eed5eedULL};
    diff_policy(g, n);
    diff_acceptance(g, n);
    diff_request_state(g, n / 10);
    diff_windows(g, n / 20);
    diff_packets(g, n);
    diff_admission(g, n / 2);
    diff_trees(g, n / 2);
    std::printf("ref_diff checks=%ld mismatches=%d\n", checks, mismatches);
    return mismatches ? 1 : 0;
}
