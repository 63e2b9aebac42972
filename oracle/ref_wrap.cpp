// ref_wrap.cpp — C shim over the reference's own host-only headers, compiled from
// where they lie under /root/reference (oracle/Makefile, target `ref`, output
// oracle/_ref/).  Test infrastructure only: it lets tests check the oracle and the
// product's C++20 host layer against the reference's code itself.
#include "exl3/greedy_packet.h"
#include "exl3/request_sampling_state.h"
#include "exl3/sampled_acceptance_reference.h"
#include "exl3/sampling_policy.h"
#include "exl3/sampling_window_transaction.h"
#include "exl3/verification_tree.h"
#include "runtime/contract/sampling.h"

#include <cstdint>
#include <memory>
#include <span>
#include <stdexcept>
#include <vector>

using namespace voidinfer;
using namespace voidinfer::exl3;

namespace {
int classify() {
    try { throw; }
    catch (const std::invalid_argument&) { return 1; }
    catch (const std::logic_error&) { return 2; }
    catch (const std::overflow_error&) { return 3; }
    catch (const std::runtime_error&) { return 4; }
    catch (...) { return 5; }
}
}  // namespace

extern "C" {

// Exl3SamplingPolicy::normalize (sampling_policy.h:33-60).  out: effective_top_k,
// greedy, top_p_enabled, min_p_enabled, occurrence_counts_required,
// requires_sampled_distribution.
int ref_normalize(const float f[6], int32_t top_k, uint64_t seed, uint32_t vocabulary, int32_t out[6]) {
    try {
        runtime::ResolvedSamplingParameters p;
        p.temperature = f[0]; p.top_k = top_k; p.top_p = f[1]; p.min_p = f[2];
        p.presence_penalty = f[3]; p.frequency_penalty = f[4]; p.seed = seed;
        const auto n = Exl3SamplingPolicy::normalize(p, vocabulary);
        out[0] = int32_t(n.effective_top_k); out[1] = n.greedy; out[2] = n.top_p_enabled;
        out[3] = n.min_p_enabled; out[4] = n.occurrence_counts_required; out[5] = n.requires_sampled_distribution();
        return 0;
    } catch (...) { return classify(); }
}

// Exl3NormalizedSamplingPolicy::require_logits (sampling_policy.h:22-29).
int ref_require_logits(uint32_t vocabulary, const float* logits, size_t n) {
    try {
        runtime::ResolvedSamplingParameters p;
        auto pol = Exl3SamplingPolicy::normalize(p, vocabulary);
        pol.require_logits(std::span<const float>(logits, n));
        return 0;
    } catch (...) { return classify(); }
}

// runtime::resolve_sampling (src/runtime/contract/sampling.cpp:35-49).  preset
// [6] floats + top_k; override mask bit i set -> overrides[i] used (i: T, top_k,
// top_p, min_p, presence, frequency, seed).  out: resolved 6 floats, top_k, seed.
int ref_resolve(const float preset[6], int32_t preset_top_k, uint32_t mask, const float ov[6], int32_t ov_top_k,
                uint64_t ov_seed, float out[6], int32_t* out_top_k, uint64_t* out_seed) {
    try {
        ModelSamplingDefaults d;
        d.non_thinking = SamplingPreset{preset[0], preset_top_k, preset[1], preset[2], preset[3], preset[4]};
        SamplingOverrides o;
        if (mask & 1) o.temperature = ov[0];
        if (mask & 2) o.top_k = ov_top_k;
        if (mask & 4) o.top_p = ov[1];
        if (mask & 8) o.min_p = ov[2];
        if (mask & 16) o.presence_penalty = ov[3];
        if (mask & 32) o.frequency_penalty = ov[4];
        if (mask & 64) o.seed = ov_seed;
        const auto r = runtime::resolve_sampling(d, SamplingMode::NonThinking, o);
        out[0] = r.temperature; out[1] = r.top_p; out[2] = r.min_p; out[3] = r.presence_penalty;
        out[4] = r.frequency_penalty; *out_top_k = r.top_k; *out_seed = r.seed;
        return 0;
    } catch (...) { return classify(); }
}

// Exl3IndependentAcceptanceReference::evaluate (sampled_acceptance_reference.h:48-88).
int ref_accept(const double* p, const double* q, size_t n, uint32_t token, double ua, double uc,
               int32_t* accepted, int32_t* correction_used, uint32_t* out_token, double* prob) {
    try {
        const auto r = Exl3IndependentAcceptanceReference::evaluate(std::span<const double>(p, n),
                                                                     std::span<const double>(q, n), token, ua, uc);
        *accepted = r.accepted; *correction_used = r.correction_draw_used; *out_token = r.token;
        *prob = r.acceptance_probability;
        return 0;
    } catch (...) { return classify(); }
}

// The first `n` draws of a fresh transaction (request_sampling_state.h:49-65).
int ref_request_draws(uint64_t epoch, uint64_t generation, uint64_t fingerprint, uint64_t seed, size_t n,
                      uint64_t* out) {
    try {
        Exl3RequestSamplingState s(epoch, generation, fingerprint, seed);
        s.bind_acquisition(1, std::make_shared<const int>(0), 0);
        auto t = s.begin(0);
        for (size_t i = 0; i < n; ++i) out[i] = s.draw(t);
        s.rollback(t);
        return 0;
    } catch (...) { return classify(); }
}

// Exl3GreedyPacket::validate (greedy_packet.h:35-49).
int ref_packet_validate(uint32_t abi, uint32_t rows, uint64_t generation, uint64_t serial, int position, int ready,
                        const uint64_t* row_serial, const int32_t* row_token, const uint32_t* row_nonfinite,
                        uint32_t expected_rows, uint64_t expected_generation, int expected_position,
                        uint64_t expected_serial, int vocabulary) {
    try {
        Exl3GreedyPacket p;
        p.abi = abi; p.rows = rows; p.generation = generation; p.serial = serial; p.position = position;
        p.ready = ready != 0;
        for (uint32_t i = 0; i < 16; ++i) p.decisions[i] = {row_serial[i], row_token[i], row_nonfinite[i]};
        p.validate(expected_rows, expected_generation, expected_position, expected_serial, vocabulary);
        return 0;
    } catch (...) { return classify(); }
}

// Window transaction script: ops string of 'P' (proposal), 'A' (acceptance),
// 'K' (accept), 'R' (reject + correction), 'S' (seal stop); then claim and commit
// `published`.  Records draws; returns committed_draws and prefix.
int ref_window_script(uint64_t seed, const char* ops, size_t published, uint64_t* draws, size_t* n_draws,
                      uint64_t* committed_draws, uint64_t* committed_prefix) {
    try {
        Exl3RequestSamplingState s(3, 5, 7, seed);
        s.bind_acquisition(13, std::make_shared<const int>(1), 64);
        Exl3SamplingWindowTransaction w(s, 64, 64);
        size_t k = 0;
        for (const char* c = ops; *c; ++c) {
            switch (*c) {
                case 'P': draws[k++] = w.draw_proposal(); break;
                case 'A': draws[k++] = w.draw_acceptance(); break;
                case 'K': w.accept_proposal(); break;
                case 'R': draws[k++] = w.reject_and_draw_correction(); break;
                case 'S': w.seal_stop_boundary(); break;
                default: return 9;
            }
        }
        *n_draws = k;
        w.claim_publication();
        w.commit(published, std::make_shared<const int>(2));
        *committed_draws = s.committed_draws();
        *committed_prefix = s.committed_prefix();
        return 0;
    } catch (...) { return classify(); }
}

// exl3_build_verification_tree (verification_tree.h:44-112).
int ref_build_verification_tree(const int64_t* drafts, int depth, const int64_t* ids, const float* unary,
                                int budget, int max_siblings, float row_cost, int* chain_drafts,
                                int64_t* sibling_tokens, int* sibling_offsets, int* n_siblings) {
    try {
        const size_t n = size_t(depth);
        const Exl3VerificationTree t = exl3_build_verification_tree(
            std::span<const std::int64_t>(drafts, n), std::span<const std::int64_t>(ids, n * 16),
            std::span<const float>(unary, n * 16), budget, max_siblings, row_cost);
        *chain_drafts = t.chain_drafts;
        *n_siblings = int(t.sibling_tokens.size());
        for (size_t i = 0; i < t.sibling_tokens.size(); ++i) {
            sibling_tokens[i] = t.sibling_tokens[i];
            sibling_offsets[i] = t.sibling_offsets[i];
        }
        return 0;
    } catch (...) {
        return classify();
    }
}

}  // extern "C"
