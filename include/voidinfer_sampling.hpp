/*
 * voidinfer_sampling.hpp — C++20 engine-facing layer of the MI355X sampling library.
 *
 * The engine's sampling code talks to a set of host contracts (request
 * parameters, the normalised policy, the per-request counter RNG and its draw
 * windows, the greedy packet, the accept decisions, the sampled-admission
 * gates) and to a handful of device launchers.  This header provides each of
 * them under the reference's own type and function names, with the same
 * argument meaning and the same exception types, so that an engine built
 * against The8Darkness/voidinfer can switch by including this header instead
 * of the files cited beside each item.  Device work goes through the C ABI in
 * voidinfer_sampling.h; status codes become exceptions here:
 *   VI_ERR_INVALID / VI_ERR_UNSUPPORTED / VI_ERR_WORKSPACE -> std::invalid_argument
 *   VI_ERR_LAUNCH / VI_ERR_DEVICE                          -> std::runtime_error
 *
 * Streams are hipStream_t passed as void* (hipStream_t converts implicitly), so
 * this header needs no HIP include.
 */
#ifndef VOIDINFER_SAMPLING_HPP
#define VOIDINFER_SAMPLING_HPP

#include "voidinfer_sampling.h"

#include <algorithm>
#include <array>
#include <atomic>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <limits>
#include <memory>
#include <numeric>
#include <optional>
#include <span>
#include <stdexcept>
#include <string>
#include <string_view>
#include <utility>
#include <vector>

namespace voidinfer_amd {

inline constexpr std::uint32_t kDefaultVocabulary = 248320;

namespace detail {

[[noreturn]] inline void raise(vi_status status, const char* what) {
    std::string msg = std::string(what) + ": " + vi_status_string(status);
    if (status == VI_ERR_LAUNCH || status == VI_ERR_DEVICE) throw std::runtime_error(msg);
    throw std::invalid_argument(msg);
}

inline void check(vi_status status, const char* what) {
    if (status != VI_OK) raise(status, what);
}

}  // namespace detail

// =====================================================================
// Request parameters — include/voidinfer/types.h:82-128 and
// src/runtime/contract/sampling.cpp:9-49.  An omitted override takes the
// model's preset for the mode; an omitted seed is 0; the resolved record is
// range-checked (std::invalid_argument).
// =====================================================================

enum class SamplingMode : std::uint8_t { Thinking, NonThinking };

struct SamplingPreset {
    float temperature = 0.0F;
    std::int32_t top_k = 0;
    float top_p = 1.0F;
    float min_p = 0.0F;
    float presence_penalty = 0.0F;
    float frequency_penalty = 0.0F;
};

struct ModelSamplingDefaults {
    SamplingPreset thinking;
    SamplingPreset non_thinking;

    [[nodiscard]] constexpr const SamplingPreset& for_mode(SamplingMode mode) const noexcept {
        return mode == SamplingMode::Thinking ? thinking : non_thinking;
    }
};

struct SamplingOverrides {
    std::optional<float> temperature;
    std::optional<std::int32_t> top_k;
    std::optional<float> top_p;
    std::optional<float> min_p;
    std::optional<float> presence_penalty;
    std::optional<float> frequency_penalty;
    std::optional<std::uint64_t> seed;
};

struct ResolvedSamplingParameters {
    float temperature = 0.0F;
    std::int32_t top_k = 0;
    float top_p = 1.0F;
    float min_p = 0.0F;
    float presence_penalty = 0.0F;
    float frequency_penalty = 0.0F;
    std::uint64_t seed = 0;
};

namespace detail {

// First violated range of a resolved record, or nullptr.  Comparisons are
// written so that a NaN fails them.
[[nodiscard]] inline const char* sampling_range_violation(const ResolvedSamplingParameters& s) noexcept {
    for (const float v : {s.temperature, s.top_p, s.min_p, s.presence_penalty, s.frequency_penalty})
        if (!std::isfinite(v)) return "sampling parameter is not finite";
    if (!(s.temperature >= 0.0F && s.temperature <= 2.0F)) return "temperature outside [0, 2]";
    if (s.top_k < 0) return "top_k is negative";
    if (!(s.top_p >= 0.0F && s.top_p <= 1.0F)) return "top_p outside [0, 1]";
    if (!(s.min_p >= 0.0F && s.min_p <= 1.0F)) return "min_p outside [0, 1]";
    if (!(s.presence_penalty >= -2.0F && s.presence_penalty <= 2.0F)) return "presence_penalty outside [-2, 2]";
    if (!(s.frequency_penalty >= -2.0F && s.frequency_penalty <= 2.0F)) return "frequency_penalty outside [-2, 2]";
    return nullptr;
}

}  // namespace detail

inline void validate_sampling(const ResolvedSamplingParameters& sampling) {
    if (const char* why = detail::sampling_range_violation(sampling)) throw std::invalid_argument(why);
}

[[nodiscard]] inline ResolvedSamplingParameters resolve_sampling(const ModelSamplingDefaults& defaults,
                                                                 SamplingMode mode,
                                                                 const SamplingOverrides& overrides) {
    const SamplingPreset& preset = defaults.for_mode(mode);
    ResolvedSamplingParameters out;
    out.temperature = overrides.temperature.value_or(preset.temperature);
    out.top_k = overrides.top_k.value_or(preset.top_k);
    out.top_p = overrides.top_p.value_or(preset.top_p);
    out.min_p = overrides.min_p.value_or(preset.min_p);
    out.presence_penalty = overrides.presence_penalty.value_or(preset.presence_penalty);
    out.frequency_penalty = overrides.frequency_penalty.value_or(preset.frequency_penalty);
    out.seed = overrides.seed.value_or(0);
    validate_sampling(out);
    return out;
}

// =====================================================================
// Device sampling configuration — src/exl3/sampled_select.h:16-28.  Same
// 40-byte layout as vi_device_sampling (the C ABI names the padding word).
// =====================================================================

inline constexpr std::int32_t kExl3AbsentOccurrence = VI_ABSENT_OCCURRENCE;

struct Exl3DeviceSampling {
    float temperature = 0.0F;
    std::int32_t top_k = 0;
    float top_p = 1.0F;
    float min_p = 0.0F;
    std::uint64_t seed = 0;
    float presence_penalty = 0.0F;
    const std::int32_t* first_occurrence = nullptr;

    [[nodiscard]] bool active() const noexcept { return temperature > 0.0F || presence_penalty != 0.0F; }
    [[nodiscard]] bool sampled() const noexcept { return temperature > 0.0F; }
    [[nodiscard]] vi_device_sampling abi() const noexcept {
        return vi_device_sampling{temperature, top_k, top_p, min_p, seed, presence_penalty, 0, first_occurrence};
    }
};
static_assert(sizeof(Exl3DeviceSampling) == sizeof(vi_device_sampling));
static_assert(offsetof(Exl3DeviceSampling, first_occurrence) == offsetof(vi_device_sampling, first_occurrence));

// =====================================================================
// Normalised policy — src/exl3/sampling_policy.h:13-61.
// =====================================================================

// The coupled sampler's fixed candidate menu: top_k 0 or >= 20 means 20.
inline constexpr std::uint32_t kExl3RegisteredTopK = 20;

struct Exl3NormalizedSamplingPolicy {
    ResolvedSamplingParameters requested;
    std::uint32_t vocabulary = 0;
    std::uint32_t effective_top_k = 0;
    bool greedy = false, top_p_enabled = false, min_p_enabled = false;
    bool occurrence_counts_required = false;

    [[nodiscard]] bool requires_sampled_distribution() const noexcept { return !greedy; }

    void require_logits(std::span<const float> logits) const {
        if (logits.size() != vocabulary) throw std::invalid_argument("sampling logits do not span the vocabulary");
        for (const float v : logits)
            if (!std::isfinite(v)) throw std::invalid_argument("sampling logits hold a non-finite value");
    }

    // Configuration of the coupled (reference-semantics) device route.
    [[nodiscard]] Exl3DeviceSampling device_sampling(const std::int32_t* first_occurrence = nullptr) const noexcept {
        Exl3DeviceSampling d;
        d.temperature = requested.temperature;
        d.top_k = static_cast<std::int32_t>(effective_top_k);
        d.top_p = requested.top_p;
        d.min_p = requested.min_p;
        d.seed = requested.seed;
        d.presence_penalty = requested.presence_penalty;
        d.first_occurrence = first_occurrence;
        return d;
    }

    // Row of the batched full-vocabulary route (vi_sample_rows): the request's
    // own top_k (0 = no cap) and both OpenAI penalties.
    [[nodiscard]] vi_row_params row_params(std::uint32_t lane, std::int32_t position,
                                           float repetition_penalty = 1.0F) const noexcept {
        vi_row_params p{};
        p.temperature = requested.temperature;
        p.top_p = requested.top_p;
        p.min_p = requested.min_p;
        p.repetition_penalty = repetition_penalty;
        p.presence_penalty = requested.presence_penalty;
        p.frequency_penalty = requested.frequency_penalty;
        p.top_k = requested.top_k;
        p.lane = lane;
        p.seed = requested.seed;
        p.position = position;
        return p;
    }
};

class Exl3SamplingPolicy {
public:
    [[nodiscard]] static Exl3NormalizedSamplingPolicy normalize(const ResolvedSamplingParameters& sampling,
                                                                std::uint32_t vocabulary = kDefaultVocabulary) {
        if (vocabulary == 0 || detail::sampling_range_violation(sampling))
            throw std::invalid_argument("resolved sampling policy is invalid");
        Exl3NormalizedSamplingPolicy out;
        out.requested = sampling;
        out.vocabulary = vocabulary;
        const std::uint32_t menu = (sampling.top_k > 0 && std::uint32_t(sampling.top_k) < kExl3RegisteredTopK)
                                       ? std::uint32_t(sampling.top_k)
                                       : kExl3RegisteredTopK;
        out.effective_top_k = std::min(menu, vocabulary);
        out.top_p_enabled = sampling.top_p < 1.0F;
        out.min_p_enabled = sampling.min_p > 0.0F;
        out.occurrence_counts_required = sampling.presence_penalty != 0.0F || sampling.frequency_penalty != 0.0F;
        // Penalties are never dropped at temperature zero: such a request needs
        // the penalized distribution, so it is not "greedy".
        out.greedy = sampling.temperature == 0.0F && !out.occurrence_counts_required;
        return out;
    }
};

// =====================================================================
// Greedy packet and selection authority — src/exl3/greedy_packet.h:12-135.
// =====================================================================

// VOIDINFER_EXL3_DEVICE_GREEDY: unset or "1" selects the device argmax, "0"
// the host-logit path; anything else is refused (greedy_packet.h:12-20).
inline bool exl3_device_greedy_enabled() {
    const char* flag = std::getenv("VOIDINFER_EXL3_DEVICE_GREEDY");
    if (!flag || std::string_view(flag).empty()) return true;
    const std::string_view v(flag);
    if (v == "1") return true;
    if (v == "0") return false;
    throw std::invalid_argument("VOIDINFER_EXL3_DEVICE_GREEDY must be 0 or 1");
}

struct Exl3GreedyRow {
    std::uint64_t serial = 0;
    std::int32_t token = -1;
    std::uint32_t nonfinite = 0;
};
static_assert(sizeof(Exl3GreedyRow) == sizeof(vi_greedy_row) && sizeof(Exl3GreedyRow) == 16);
static_assert(offsetof(Exl3GreedyRow, token) == offsetof(vi_greedy_row, token));

inline constexpr std::uint32_t kExl3GreedyPacketRows = 16;

struct Exl3GreedyPacket {
    static constexpr std::uint32_t version = 1;
    std::uint32_t abi = version, rows = 0;
    std::uint64_t generation = 0, serial = 0;
    int position = 0;
    bool ready = false;
    std::array<Exl3GreedyRow, kExl3GreedyPacketRows> decisions{};

    // A packet authorizes tokens only if it is the one the caller is waiting
    // for (ABI, rows, generation, position, serial) and every produced row —
    // including the last, which authorizes nothing — is finite and in range.
    void validate(std::uint32_t expected_rows, std::uint64_t expected_generation, int expected_position,
                  std::uint64_t expected_serial, int vocabulary = int(kDefaultVocabulary)) const {
        const bool header_ok = abi == version && ready && rows == expected_rows && rows >= 1 &&
                               rows <= kExl3GreedyPacketRows && generation == expected_generation &&
                               position == expected_position && serial != 0 && serial == expected_serial &&
                               vocabulary > 0;
        if (!header_ok) throw std::runtime_error("greedy packet is stale or incomplete");
        for (std::uint32_t r = 0; r < rows; ++r) {
            const Exl3GreedyRow& d = decisions[r];
            if (d.serial != serial || d.nonfinite != 0 || d.token < 0 || d.token >= vocabulary)
                throw std::runtime_error("greedy packet row is stale, non-finite or out of range");
        }
    }
};

// Probabilities of a sampled decision: the compact packet cannot carry them.
struct Exl3SampledDistributionAuthority {
    std::shared_ptr<const void> owner;
    const float* probabilities = nullptr;
    std::uint32_t rows = 0, vocabulary = 0, row_stride = 0;
    std::uint64_t generation = 0, serial = 0;
    int position = 0;
    bool ready = false;
};

enum class Exl3SelectionAuthorityKind : std::uint8_t { greedy_argmax, sampled_distribution };

class Exl3SelectionAuthorityRequirement {
public:
    [[nodiscard]] static Exl3SelectionAuthorityRequirement greedy(std::uint32_t rows, std::uint64_t generation,
                                                                  int position, std::uint64_t serial,
                                                                  std::uint32_t vocabulary = kDefaultVocabulary) {
        if (rows == 0 || rows > kExl3GreedyPacketRows || vocabulary == 0)
            throw std::invalid_argument("greedy authority requirement extent");
        return {Exl3SelectionAuthorityKind::greedy_argmax, rows, vocabulary, generation, serial, position};
    }
    [[nodiscard]] static Exl3SelectionAuthorityRequirement sampled(std::uint32_t rows, std::uint64_t generation,
                                                                   int position, std::uint64_t serial,
                                                                   std::uint32_t vocabulary = kDefaultVocabulary) {
        if (rows == 0 || vocabulary == 0) throw std::invalid_argument("sampled authority requirement extent");
        return {Exl3SelectionAuthorityKind::sampled_distribution, rows, vocabulary, generation, serial, position};
    }
    // What one request needs: any temperature or penalty needs the distribution.
    [[nodiscard]] static Exl3SelectionAuthorityRequirement request(float temperature, float presence_penalty,
                                                                   float frequency_penalty) {
        const bool sampled_needed = temperature != 0.0F || presence_penalty != 0.0F || frequency_penalty != 0.0F;
        return sampled_needed ? sampled(1, 0, 0, 0) : greedy(1, 0, 0, 0);
    }

    [[nodiscard]] Exl3SelectionAuthorityKind kind() const noexcept { return kind_; }
    [[nodiscard]] bool needs_sampled_distribution() const noexcept {
        return kind_ == Exl3SelectionAuthorityKind::sampled_distribution;
    }

    void validate(const Exl3GreedyPacket& packet) const {
        if (kind_ != Exl3SelectionAuthorityKind::greedy_argmax)
            throw std::invalid_argument("an argmax packet cannot authorize a sampled decision");
        packet.validate(rows_, generation_, position_, serial_, static_cast<int>(vocabulary_));
    }
    void validate(const Exl3SampledDistributionAuthority& d) const {
        if (kind_ != Exl3SelectionAuthorityKind::sampled_distribution)
            throw std::invalid_argument("a sampled distribution cannot authorize a greedy decision");
        const bool ok = d.owner && d.probabilities && d.ready && d.rows == rows_ && d.vocabulary == vocabulary_ &&
                        d.row_stride >= vocabulary_ && d.generation == generation_ && d.position == position_ &&
                        d.serial == serial_;
        if (!ok) throw std::invalid_argument("sampled distribution authority is missing, stale or incomplete");
    }

private:
    Exl3SelectionAuthorityRequirement(Exl3SelectionAuthorityKind kind, std::uint32_t rows, std::uint32_t vocabulary,
                                      std::uint64_t generation, std::uint64_t serial, int position)
        : kind_(kind), rows_(rows), vocabulary_(vocabulary), generation_(generation), serial_(serial),
          position_(position) {}

    Exl3SelectionAuthorityKind kind_ = Exl3SelectionAuthorityKind::greedy_argmax;
    std::uint32_t rows_ = 0, vocabulary_ = 0;
    std::uint64_t generation_ = 0, serial_ = 0;
    int position_ = 0;
};

// Tentative path of a verified chain: the seed (the pre-forward root's token),
// then decision r-1 authorizes tentative row r.
inline void exl3_greedy_path(std::int64_t seed, const Exl3GreedyPacket& packet, std::span<std::int64_t> path) {
    if (path.empty() || path.size() > kExl3GreedyPacketRows) throw std::invalid_argument("greedy path extent");
    Exl3SelectionAuthorityRequirement::greedy(static_cast<std::uint32_t>(path.size()), packet.generation,
                                              packet.position, packet.serial)
        .validate(packet);
    if (seed < 0 || seed >= std::int64_t(kDefaultVocabulary)) throw std::invalid_argument("greedy path seed");
    path[0] = seed;
    for (std::size_t i = 1; i < path.size(); ++i) path[i] = packet.decisions[i - 1].token;
}

// ---------------------------------------------------------------------
// Greedy decisions with either authority — branch_reference.h:23-31 and
// exact_outer_reference.h:14-36.  With VOIDINFER_EXL3_DEVICE_GREEDY on, the
// context's device greedy packet decides; with it "0", the context's logits are
// read back and each row's first largest entry decides, every entry of every
// row read having to be finite (std::runtime_error otherwise).
//
// Context is the engine's text context; these members are used:
//   Exl3GreedyPacket greedy_packet(bool continuation, Stream stream);
//   (a float range) logits_host(Stream stream);               // the root row
//   (a float range) continuation_logits_host(Stream stream);  // path.size() rows of
//                                                              // kDefaultVocabulary
// ---------------------------------------------------------------------

namespace detail {
// Index of the first largest entry; nullopt when the row is empty or holds a
// non-finite entry.
inline std::optional<std::int64_t> finite_argmax(std::span<const float> row) noexcept {
    if (row.empty()) return std::nullopt;
    std::size_t best = 0;
    for (std::size_t i = 0; i < row.size(); ++i) {
        if (!std::isfinite(row[i])) return std::nullopt;
        if (row[i] > row[best]) best = i;
    }
    return static_cast<std::int64_t>(best);
}
}  // namespace detail

template <class Context, class Stream = void*>
std::int64_t exl3_branch_greedy(Context& context, Stream stream = nullptr) {
    if (exl3_device_greedy_enabled()) return context.greedy_packet(false, stream).decisions[0].token;
    const auto logits = context.logits_host(stream);
    const auto token = detail::finite_argmax(std::span<const float>(std::data(logits), std::size(logits)));
    if (!token) throw std::runtime_error("host greedy row is empty or non-finite");
    return *token;
}

// path[0] = seed; path[r] = the decision of continuation row r-1; the last
// row's decision, which authorizes no path entry, goes to *deferred_bonus.
template <class Context, class Stream>
void exl3_outer_greedy_path(Context& exact, std::int64_t seed, std::span<std::int64_t> path, Stream stream,
                            std::int64_t* deferred_bonus = nullptr) {
    if (path.empty()) throw std::invalid_argument("greedy path extent");
    if (exl3_device_greedy_enabled()) {
        const Exl3GreedyPacket packet = exact.greedy_packet(true, stream);
        exl3_greedy_path(seed, packet, path);
        if (deferred_bonus) *deferred_bonus = packet.decisions[path.size() - 1].token;
        return;
    }
    const auto logits = exact.continuation_logits_host(stream);
    const std::span<const float> all(std::data(logits), std::size(logits));
    const std::size_t v = kDefaultVocabulary;
    std::vector<std::int64_t> decision(path.size());
    bool usable = all.size() == path.size() * v;
    for (std::size_t r = 0; usable && r < path.size(); ++r) {
        const auto d = detail::finite_argmax(all.subspan(r * v, v));
        usable = d.has_value();
        if (usable) decision[r] = *d;
    }
    if (!usable) throw std::runtime_error("host continuation logits are mis-sized or non-finite");
    path[0] = seed;
    std::copy(decision.begin(), decision.end() - 1, path.begin() + 1);
    if (deferred_bonus) *deferred_bonus = decision.back();
}

// =====================================================================
// Per-request counter RNG — src/exl3/request_sampling_state.h:12-143.
// Draw i of a request is SplitMix64(seed ^ fingerprint ^ generation ^ i); only
// committed draws advance i, so a rolled-back window replays the same values.
// =====================================================================

enum class Exl3SamplingReproducibility : std::uint8_t { seeded_request_replay_across_reload };

inline constexpr std::uint64_t exl3_splitmix64(std::uint64_t x) noexcept {
    x += 0x9e3779b97f4a7c15ULL;
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ULL;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebULL;
    return x ^ (x >> 31);
}

class Exl3RequestSamplingState {
public:
    // One speculative round's lease on the request's draws (begin() to commit()
    // or rollback()).  Callers keep it and hand it back; they do not edit it.
    struct Transaction {
        const Exl3RequestSamplingState* owner = nullptr;
        std::uint64_t nonce = 0, acquisition = 0, base_counter = 0, tentative_counter = 0;
        std::size_t accepted_prefix = 0;
        std::shared_ptr<const void> root_revision;
        bool publication_claimed = false;
    };

    Exl3RequestSamplingState(std::uint64_t engine_epoch, std::uint64_t request_generation,
                             std::uint64_t input_fingerprint, std::uint64_t seed,
                             Exl3SamplingReproducibility reproducibility =
                                 Exl3SamplingReproducibility::seeded_request_replay_across_reload)
        : id_{engine_epoch, request_generation, input_fingerprint, seed}, reproducibility_(reproducibility) {
        if (id_.epoch == 0 || id_.generation == 0 || id_.fingerprint == 0)
            throw std::invalid_argument("request identity needs a non-zero epoch, generation and input fingerprint");
    }

    void bind_acquisition(std::uint64_t acquisition, std::shared_ptr<const void> root_revision,
                          std::size_t accepted_prefix) {
        const bool refused = cancelled() || acquisition == 0 || !owned(root_revision) || lease_ != 0;
        if (refused) throw std::invalid_argument("request state cannot take this acquisition now");
        bound_.acquisition = acquisition;
        bound_.root = std::move(root_revision);
        progress_.prefix = accepted_prefix;
    }

    [[nodiscard]] Transaction begin(std::size_t accepted_prefix) {
        const bool bound = bound_.acquisition != 0 && bound_.root != nullptr;
        if (cancelled() || !bound || lease_ != 0 || next_lease_ == 0 || accepted_prefix != progress_.prefix)
            throw std::logic_error("request state cannot open a round now");
        lease_ = next_lease_++;
        Transaction t;
        t.owner = this;
        t.nonce = lease_;
        t.acquisition = bound_.acquisition;
        t.base_counter = progress_.draws;
        t.tentative_counter = progress_.draws;
        t.accepted_prefix = accepted_prefix;
        t.root_revision = bound_.root;
        return t;
    }

    [[nodiscard]] std::uint64_t draw(Transaction& t) const {
        expect_live(t, false);
        if (t.tentative_counter == std::numeric_limits<std::uint64_t>::max())
            throw std::overflow_error("request draw index exhausted");
        return exl3_splitmix64(id_.seed ^ id_.fingerprint ^ id_.generation ^ t.tentative_counter++);
    }

    void claim_publication(Transaction& t) {
        expect_live(t, false);
        if (t.publication_claimed) throw std::logic_error("round publication is already claimed");
        t.publication_claimed = true;
    }

    void commit(Transaction& t, std::uint64_t draws_to_commit, std::size_t accepted_prefix,
                std::shared_ptr<const void> new_root_revision) {
        expect_live(t, true);
        const std::uint64_t tentative = t.tentative_counter - t.base_counter;
        const bool extent_ok = t.publication_claimed && draws_to_commit <= tentative &&
                               accepted_prefix >= t.accepted_prefix && owned(new_root_revision) &&
                               draws_to_commit <= std::numeric_limits<std::uint64_t>::max() - progress_.draws;
        if (!extent_ok) throw std::invalid_argument("round commit outside what the round drew or claimed");
        progress_.draws += draws_to_commit;
        progress_.prefix = accepted_prefix;
        bound_.root = std::move(new_root_revision);
        end_round(t);
    }

    void rollback(Transaction& t) {
        expect_live(t, t.publication_claimed);
        end_round(t);
    }

    void advance_forced_control(std::size_t tokens, std::shared_ptr<const void> new_root_revision,
                                bool resident_committed) {
        const bool ok = resident_committed && tokens != 0 && bound_.acquisition != 0 && lease_ == 0 &&
                        owned(new_root_revision) && tokens <= std::numeric_limits<std::size_t>::max() - progress_.prefix;
        if (!ok) throw std::invalid_argument("forced control tokens cannot advance the request now");
        progress_.prefix += tokens;
        bound_.root = std::move(new_root_revision);
    }

    void cancel() noexcept { cancelled_.store(true, std::memory_order_release); }

    [[nodiscard]] std::uint64_t engine_epoch() const noexcept { return id_.epoch; }
    [[nodiscard]] std::uint64_t request_generation() const noexcept { return id_.generation; }
    [[nodiscard]] std::uint64_t committed_draws() const noexcept { return progress_.draws; }
    [[nodiscard]] std::size_t committed_prefix() const noexcept { return progress_.prefix; }
    [[nodiscard]] Exl3SamplingReproducibility reproducibility() const noexcept { return reproducibility_; }
    [[nodiscard]] bool cancelled() const noexcept { return cancelled_.load(std::memory_order_acquire); }

private:
    // Why a round handed back is not the live one (none: it is).
    enum class RoundFault : std::uint8_t { none, cancelled, not_ours, no_open_round, other_round, rebound, other_root };

    [[nodiscard]] RoundFault fault(const Transaction& t, bool claimed_outlives_cancel) const noexcept {
        if (cancelled() && !(claimed_outlives_cancel && t.publication_claimed)) return RoundFault::cancelled;
        if (t.owner != this) return RoundFault::not_ours;
        if (lease_ == 0) return RoundFault::no_open_round;
        if (t.nonce != lease_) return RoundFault::other_round;
        if (t.acquisition != bound_.acquisition) return RoundFault::rebound;
        const auto& r = t.root_revision;
        const bool same_root = r.get() == bound_.root.get() && !r.owner_before(bound_.root) && !bound_.root.owner_before(r);
        return same_root ? RoundFault::none : RoundFault::other_root;
    }
    void expect_live(const Transaction& t, bool claimed_outlives_cancel) const {
        static constexpr const char* kWhy[] = {"", "request cancelled", "round of another request state",
                                               "no round is open", "round already closed or superseded",
                                               "request rebound to another acquisition", "root revision changed"};
        const RoundFault f = fault(t, claimed_outlives_cancel);
        if (f != RoundFault::none) throw std::logic_error(std::string("sampling round refused: ") + kWhy[int(f)]);
    }
    // (a root revision without an owner cannot be kept alive by the state)
    static bool owned(const std::shared_ptr<const void>& r) noexcept { return r != nullptr && r.use_count() > 0; }
    void end_round(Transaction& t) noexcept {
        lease_ = 0;
        t.owner = nullptr;
        t.nonce = 0;
        t.publication_claimed = false;
        t.root_revision.reset();
    }

    struct Identity { std::uint64_t epoch, generation, fingerprint, seed; } id_;
    Exl3SamplingReproducibility reproducibility_;
    struct Binding { std::uint64_t acquisition = 0; std::shared_ptr<const void> root; } bound_;
    struct Progress { std::uint64_t draws = 0; std::size_t prefix = 0; } progress_;
    std::uint64_t lease_ = 0;        // the open round's id (0: none)
    std::uint64_t next_lease_ = 1;   // (0 once every id is used)
    std::atomic<bool> cancelled_{false};
};

// =====================================================================
// One speculative round's window of draws — src/exl3/sampling_window_transaction.h:17-128.
// Every decided token spent a proposal draw and an acceptance draw; a rejected
// one also spent a correction draw and closes the round to further tokens.  A
// commit of n published tokens commits the draws of those n tokens only.
// =====================================================================

class Exl3SamplingWindowTransaction {
public:
    Exl3SamplingWindowTransaction(Exl3RequestSamplingState& state, std::size_t accepted_prefix,
                                  std::size_t maximum_tokens)
        : state_(&state), first_(accepted_prefix), capacity_(maximum_tokens) {
        if (maximum_tokens == 0 || maximum_tokens > std::numeric_limits<std::size_t>::max() - accepted_prefix)
            throw std::invalid_argument("a sampling window needs room for at least one token");
        spent_.reserve(maximum_tokens);
        round_ = state.begin(accepted_prefix);
        stage_ = Stage::idle;
    }

    ~Exl3SamplingWindowTransaction() {
        if (stage_ != Stage::closed && !state_->cancelled()) {
            try { state_->rollback(round_); } catch (...) {}
        }
    }

    Exl3SamplingWindowTransaction(const Exl3SamplingWindowTransaction&) = delete;
    Exl3SamplingWindowTransaction& operator=(const Exl3SamplingWindowTransaction&) = delete;

    [[nodiscard]] std::uint64_t draw_proposal() {
        expect_open_to_tokens();
        if (stage_ != Stage::idle || spent_.size() >= capacity_)
            throw std::logic_error("a proposal draw needs a decided previous token and room in the window");
        stage_ = Stage::proposed;   // (kept when the state refuses the draw)
        return state_->draw(round_);
    }

    [[nodiscard]] std::uint64_t draw_acceptance() {
        expect_open_to_tokens();
        if (stage_ != Stage::proposed) throw std::logic_error("an acceptance draw follows a proposal draw");
        stage_ = Stage::acceptance_drawn;
        return state_->draw(round_);
    }

    void accept_proposal() {
        expect_decision();
        spent_.push_back(2);
        stage_ = Stage::idle;
    }

    [[nodiscard]] std::uint64_t reject_and_draw_correction() {
        expect_decision();
        const std::uint64_t correction = state_->draw(round_);
        spent_.push_back(3);
        stage_ = Stage::idle;
        sealed_ = true;
        return correction;
    }

    void seal_stop_boundary() {
        expect_open_to_tokens();
        if (stage_ != Stage::idle) throw std::logic_error("a stop cannot split an undecided token");
        sealed_ = true;
    }

    void claim_publication() {
        expect_round();
        if (stage_ != Stage::idle) throw std::logic_error("publication with an undecided token");
        state_->claim_publication(round_);
        claimed_ = true;
    }

    void commit(std::size_t published_tokens, std::shared_ptr<const void> new_root_revision) {
        expect_round();
        if (!claimed_ || stage_ != Stage::idle || published_tokens > spent_.size())
            throw std::invalid_argument("commit needs a claimed publication of decided tokens");
        const std::uint64_t draws = std::accumulate(spent_.begin(), spent_.begin() + std::ptrdiff_t(published_tokens),
                                                    std::uint64_t(0));
        state_->commit(round_, draws, first_ + published_tokens, std::move(new_root_revision));
        stage_ = Stage::closed;
    }

    void rollback() {
        expect_round();
        stage_ = Stage::idle;
        state_->rollback(round_);
        stage_ = Stage::closed;
    }

    [[nodiscard]] std::size_t decided_tokens() const noexcept { return spent_.size(); }
    [[nodiscard]] bool sealed() const noexcept { return sealed_; }

private:
    // Where the current token stands; closed once committed or rolled back.
    enum class Stage : std::uint8_t { idle, proposed, acceptance_drawn, closed };

    void expect_round() const {
        if (stage_ == Stage::closed) throw std::logic_error("the sampling window is closed");
    }
    void expect_open_to_tokens() const {
        expect_round();
        if (sealed_) throw std::logic_error("the sampling window takes no more tokens");
    }
    void expect_decision() const {
        expect_open_to_tokens();
        if (stage_ != Stage::acceptance_drawn) throw std::logic_error("a decision needs the acceptance draw");
    }

    Exl3RequestSamplingState* state_;
    std::size_t first_, capacity_;
    std::vector<std::uint8_t> spent_;   // draws spent by each decided token (2, or 3 with a correction)
    Exl3RequestSamplingState::Transaction round_;
    Stage stage_ = Stage::closed;
    bool sealed_ = false, claimed_ = false;
};

// Forced control tokens and terminal tokens — src/exl3/sampling_control_stop_semantics.h:13-42.
struct Exl3SamplingPublicationCount {
    std::size_t resident_tokens = 0, visible_tokens = 0;
    bool terminal = false, terminal_visible = false;
};

class Exl3SamplingControlStopSemantics {
public:
    // Control tokens the engine forced advance the prefix once resident; they
    // spend no draw.
    static void commit_forced_control_after_resident(Exl3RequestSamplingState& state, std::size_t tokens,
                                                     std::shared_ptr<const void> new_root_revision) {
        state.advance_forced_control(tokens, std::move(new_root_revision), true);
    }
    static void claim_model_publication(Exl3SamplingWindowTransaction& window) { window.claim_publication(); }
    // All resident tokens' draws are committed; a terminal token the caller does
    // not publish is left out of the visible count only.
    static Exl3SamplingPublicationCount commit_model_after_resident(Exl3SamplingWindowTransaction& window,
                                                                    std::size_t resident_tokens, bool terminal,
                                                                    bool publish_terminal,
                                                                    std::shared_ptr<const void> new_root_revision) {
        if (resident_tokens == 0 || (publish_terminal && !terminal))
            throw std::invalid_argument("publishing a terminal token needs one among the resident tokens");
        window.commit(resident_tokens, std::move(new_root_revision));
        const bool hidden_terminal = terminal && !publish_terminal;
        return {resident_tokens, resident_tokens - (hidden_terminal ? 1u : 0u), terminal, terminal && publish_terminal};
    }
    static void abandon_before_correction(Exl3SamplingWindowTransaction& window) { window.rollback(); }
};

// =====================================================================
// Accept decisions.
// =====================================================================

// Greedy longest prefix — src/exl3/exact_outer_reference.h:45-82.  Row r
// commits the target's token; a mismatch (rejected) or a terminal token
// (stopped) ends the walk after committing that row.
struct Exl3OuterDecision {
    std::vector<std::int64_t> committed_tokens;
    std::size_t accepted = 0;
    bool rejected = false, stopped = false;
};

inline bool exl3_terminal_token(std::int64_t token, std::span<const std::int64_t> terminal) {
    return std::find(terminal.begin(), terminal.end(), token) != terminal.end();
}

inline Exl3OuterDecision decide_exl3_outer_prefix(std::span<const std::int64_t> target_path,
                                                  std::span<const std::int64_t> tentative,
                                                  std::span<const std::int64_t> terminal = {}) {
    if (target_path.empty() || target_path.size() != tentative.size())
        throw std::invalid_argument("outer decision extent");
    Exl3OuterDecision d;
    d.committed_tokens.reserve(target_path.size());
    for (std::size_t r = 0; r < target_path.size() && !d.rejected && !d.stopped; ++r) {
        const std::int64_t t = target_path[r];
        d.committed_tokens.push_back(t);
        if (tentative[r] == t) ++d.accepted;
        else d.rejected = true;
        d.stopped = exl3_terminal_token(t, terminal);
    }
    return d;
}

// Sibling promotion of a verification tree — src/exl3/exact_outer_reference.h:401-436.
// tentative = [chain rows..., sibling rows...]; a chain rejected at depth d
// continues through the first sibling drafted at offset d whose token equals
// the target's correction: that sibling row's own target decision
// (sibling_decisions[j]) is committed next and the accepted count becomes d + 1.
// Returns the promoted tentative row index, or -1.
inline int exl3_promote_sibling(Exl3OuterDecision& decision, std::span<const std::int64_t> tentative,
                                std::size_t chain_rows, std::span<const int> sibling_offsets,
                                std::span<const std::int64_t> sibling_decisions,
                                std::span<const std::int64_t> terminal = {}) {
    if (chain_rows > tentative.size() || sibling_offsets.size() != tentative.size() - chain_rows ||
        sibling_decisions.size() != sibling_offsets.size())
        throw std::invalid_argument("sibling promotion extent");
    if (!decision.rejected || decision.stopped || decision.committed_tokens.empty()) return -1;
    const int depth = static_cast<int>(decision.accepted);
    for (std::size_t j = 0; j < sibling_offsets.size(); ++j) {
        if (sibling_offsets[j] != depth || tentative[chain_rows + j] != decision.committed_tokens.back()) continue;
        const std::int64_t next = sibling_decisions[j];
        decision.committed_tokens.push_back(next);
        decision.accepted = static_cast<std::size_t>(depth) + 1;
        decision.stopped = exl3_terminal_token(next, terminal);
        return static_cast<int>(chain_rows + j);
    }
    return -1;
}

// =====================================================================
// Verification tree of a DFlash2 round — src/exl3/verification_tree.h:27-112.
// The tree is a prefix of the draft chain plus leaves: at each depth, the
// draft's best candidates other than the chain token, each standing in for the
// chain token at that position.  Of all (chain length, leaves) shapes within
// the row budget, the builder keeps the first with the highest
// (1 + expected accepted tokens) / (1 + row_cost x rows).  Expected acceptance
// comes from the draft's top-16 scores through a softmax: the chain token's by
// the tenth its probability falls in, a leaf's by its rank among the other
// candidates (three ranks) and its probability's tenth, read from tables
// measured on the engine's rounds.
// =====================================================================

struct Exl3VerificationTree {
    int chain_drafts = 0;                   // drafts 1..chain_drafts are verified as a chain
    std::vector<std::int64_t> sibling_tokens;
    std::vector<int> sibling_offsets;       // the chain position each leaf stands in for (1-based)
};

// Row cost as a fraction of a verifier round, and the measured hit rates by
// probability tenth (verification_tree.h:31-40): chain tokens, then leaves of
// rank 1, 2, 3.
inline constexpr float kExl3TreeRowCost = 0.0141f;
inline constexpr std::array<float, 10> kExl3TreeChainHit{
    0.32f, 0.38f, 0.35f, 0.44f, 0.42f, 0.49f, 0.57f, 0.67f, 0.78f, 0.97f};
inline constexpr std::array<std::array<float, 10>, 3> kExl3TreeSiblingHit{{
    {0.04f, 0.13f, 0.18f, 0.23f, 0.26f, 0.27f, 0.13f, 0.09f, 0.06f, 0.07f},
    {0.03f, 0.10f, 0.15f, 0.09f, 0.12f, 0.12f, 0.12f, 0.12f, 0.12f, 0.12f},
    {0.03f, 0.10f, 0.15f, 0.15f, 0.15f, 0.15f, 0.15f, 0.15f, 0.15f, 0.15f},
}};

namespace tree_detail {
inline constexpr int kCandidates = 16, kLeafRanks = 3;

struct LeafOption {
    float expected;        // expected accepted tokens it adds (hit rate x chance its position is reached)
    int position;          // 1-based chain position it stands in for
    std::int64_t token;    // -1: no such candidate
};

// What one depth of the draft offers: the chain token's hit rate and the best
// three other candidates as leaves.
struct DepthOffer {
    float chain_hit = 0.0f;
    std::array<LeafOption, kLeafRanks> leaves{};
};

inline int probability_tenth(float p) { return std::clamp(static_cast<int>(p * 10.0f), 0, 9); }

inline DepthOffer offer_at(const std::int64_t* ids, const float* scores, std::int64_t chain_token, int depth) {
    // softmax of the candidate scores, accumulated in candidate order
    const float peak = *std::max_element(scores, scores + kCandidates);
    std::array<float, kCandidates> weight{};
    float total = 0.0f;
    for (int c = 0; c < kCandidates; ++c) {
        weight[std::size_t(c)] = std::exp(scores[c] - peak);
        total += weight[std::size_t(c)];
    }
    DepthOffer offer;
    float chain_p = 0.0f;   // (of the chain token's last occurrence in the list)
    for (int c = 0; c < kCandidates; ++c)
        if (ids[c] == chain_token) chain_p = weight[std::size_t(c)] / total;
    offer.chain_hit = kExl3TreeChainHit[std::size_t(probability_tenth(chain_p))];
    // candidates by descending score, equal scores in list order
    std::array<int, kCandidates> by_score{};
    std::iota(by_score.begin(), by_score.end(), 0);
    std::stable_sort(by_score.begin(), by_score.end(), [&](int x, int y) { return scores[x] > scores[y]; });
    int rank = 0;
    for (const int c : by_score) {
        if (rank == kLeafRanks) break;
        if (ids[c] == chain_token) continue;
        const float hit = kExl3TreeSiblingHit[std::size_t(rank)][std::size_t(probability_tenth(weight[std::size_t(c)] / total))];
        offer.leaves[std::size_t(rank++)] = {hit, depth + 1, ids[c]};
    }
    for (; rank < kLeafRanks; ++rank) offer.leaves[std::size_t(rank)] = {0.0f, depth + 1, -1};
    return offer;
}
}  // namespace tree_detail

// drafts: the chain proposals at positions 1..D; candidate_ids /
// candidate_unary: [D][16], the draft's top-16 per position in unary order;
// budget: verifier rows besides the anchor.  Ties are settled as the reference
// settles them: equal scores keep list order; among leaves of equal value,
// the order std::partial_sort leaves a pool built in the same order in; the
// first strictly best shape wins.  Candidate arrays shorter than D x 16 are
// refused (std::invalid_argument).
inline Exl3VerificationTree exl3_build_verification_tree(std::span<const std::int64_t> drafts,
                                                         std::span<const std::int64_t> candidate_ids,
                                                         std::span<const float> candidate_unary, int budget,
                                                         int max_siblings, float row_cost = kExl3TreeRowCost) {
    using namespace tree_detail;
    const int depth = std::max(0, std::min(static_cast<int>(drafts.size()), budget));
    if (candidate_ids.size() < std::size_t(depth) * kCandidates || candidate_unary.size() < std::size_t(depth) * kCandidates)
        throw std::invalid_argument("verification tree needs 16 candidates per draft position");
    std::vector<DepthOffer> offers;
    offers.reserve(std::size_t(depth));
    for (int d = 0; d < depth; ++d)
        offers.push_back(offer_at(candidate_ids.data() + std::size_t(d) * kCandidates,
                                  candidate_unary.data() + std::size_t(d) * kCandidates, drafts[std::size_t(d)], d));
    // For a chain of length L: its expected accepted length (the chance each of
    // its positions is reached and hit, summed) and the leaves it can carry
    // (each leaf's hit rate times the chance its position is reached).
    std::vector<float> chain_gain(std::size_t(depth) + 1, 0.0f);
    std::vector<std::vector<LeafOption>> carried(std::size_t(depth) + 1);
    for (int len = 1; len <= depth; ++len) {
        float reach = 1.0f, gain = 0.0f;
        for (int d = 0; d < len; ++d) {
            for (const LeafOption& l : offers[std::size_t(d)].leaves)
                if (l.token >= 0) carried[std::size_t(len)].push_back({reach * l.expected, l.position, l.token});
            reach *= offers[std::size_t(d)].chain_hit;
            gain += reach;
        }
        chain_gain[std::size_t(len)] = gain;
    }
    Exl3VerificationTree best;
    float best_rate = -1.0f;
    std::vector<LeafOption> pick;
    for (int rows = 1; rows <= budget; ++rows) {
        const int shortest = std::max(1, rows - std::max(0, max_siblings)), longest = std::min(depth, rows);
        for (int len = shortest; len <= longest; ++len) {
            const int leaves = rows - len;
            if (leaves > static_cast<int>(carried[std::size_t(len)].size())) continue;
            pick = carried[std::size_t(len)];
            std::partial_sort(pick.begin(), pick.begin() + leaves, pick.end(),
                              [](const LeafOption& x, const LeafOption& y) { return x.expected > y.expected; });
            float gain = chain_gain[std::size_t(len)];
            for (int i = 0; i < leaves; ++i) gain += pick[std::size_t(i)].expected;
            const float rate = (1.0f + gain) / (1.0f + row_cost * static_cast<float>(rows));
            if (!(rate > best_rate)) continue;
            best_rate = rate;
            best.chain_drafts = len;
            best.sibling_tokens.resize(std::size_t(leaves));
            best.sibling_offsets.resize(std::size_t(leaves));
            for (int i = 0; i < leaves; ++i) {
                best.sibling_tokens[std::size_t(i)] = pick[std::size_t(i)].token;
                best.sibling_offsets[std::size_t(i)] = pick[std::size_t(i)].position;
            }
        }
    }
    return best;
}

// FP64 rejection sampling of one speculative position —
// src/exl3/sampled_acceptance_reference.h:15-89.  The proposed token was drawn
// from the draft's q; it is kept when the acceptance uniform is below
// min(1, p / q), otherwise the correction uniform draws from the normalised
// residual max(0, p - q) by inverse CDF in token-id order.
struct Exl3SampledAcceptanceOutcome {
    bool accepted = false;
    bool correction_draw_used = false;
    std::uint32_t token = 0;
    double acceptance_probability = 0;
    std::vector<double> residual;
};

class Exl3IndependentAcceptanceReference {
public:
    static Exl3SampledAcceptanceOutcome evaluate(std::span<const double> target_p, std::span<const double> draft_q,
                                                 std::uint32_t proposed_token, double acceptance_draw,
                                                 double correction_draw) {
        // input checks, in this order: p, q, the two uniforms, the extents, q of the proposal
        for (const std::span<const double> dist : {target_p, draft_q})
            if (const char* why = distribution_fault(dist)) throw std::invalid_argument(why);
        for (const double u : {acceptance_draw, correction_draw})
            if (!(std::isfinite(u) && u >= 0.0 && u < 1.0)) throw std::invalid_argument("uniform draw outside [0, 1)");
        if (target_p.size() != draft_q.size() || proposed_token >= target_p.size())
            throw std::invalid_argument("p, q and the proposed token disagree on the vocabulary");
        if (draft_q[proposed_token] == 0.0)
            throw std::invalid_argument("the proposed token has zero draft probability");

        Exl3SampledAcceptanceOutcome out;
        out.acceptance_probability = std::min(1.0, target_p[proposed_token] / draft_q[proposed_token]);
        out.accepted = acceptance_draw < out.acceptance_probability;
        if (out.accepted) {
            out.token = proposed_token;
            return out;
        }
        out.residual = normalised_residual(target_p, draft_q);
        out.correction_draw_used = true;
        out.token = inverse_cdf(out.residual, correction_draw);
        return out;
    }

private:
    static constexpr double kSumTolerance = 1e-9;

    // nullptr when `v` is a distribution: entries in [0, 1] summing to 1 within
    // kSumTolerance
    static const char* distribution_fault(std::span<const double> v) {
        if (v.empty()) return "empty distribution";
        double sum = 0.0;
        for (const double x : v) {
            if (!std::isfinite(x) || x < 0.0 || x > 1.0) return "distribution entry outside [0, 1]";
            sum += x;
        }
        return std::isfinite(sum) && std::abs(sum - 1.0) <= kSumTolerance ? nullptr : "distribution does not sum to one";
    }
    // max(0, p - q), summed in id order, then divided by that sum
    static std::vector<double> normalised_residual(std::span<const double> p, std::span<const double> q) {
        std::vector<double> r(p.size());
        double mass = 0.0;
        for (std::size_t i = 0; i < p.size(); ++i) mass += (r[i] = std::max(0.0, p[i] - q[i]));
        if (!std::isfinite(mass) || mass <= kSumTolerance) throw std::logic_error("a rejection left no residual mass");
        for (double& x : r) x /= mass;
        return r;
    }
    // first id whose running sum exceeds u; past the end (rounding), the last id
    // with residual mass
    static std::uint32_t inverse_cdf(const std::vector<double>& r, double u) {
        double running = 0.0;
        std::uint32_t last_supported = 0;
        for (std::uint32_t t = 0; t < r.size(); ++t) {
            if (r[t] > 0.0) last_supported = t;
            running += r[t];
            if (u < running) return t;
        }
        return last_supported;
    }
};

// VeriCache keep rule — src/exl3/fast_device_round.h:31-43,841-866.  Row i
// scores drafted token tokens[i+1]: it is kept while gap <= delta (delta > 0)
// or while it equals the exact choice (delta == 0).  The first refused row
// commits the exact choice as a correction and ends the block.
struct Exl3RowScore {
    std::int64_t greedy = -1;
    float gap = 0.0F;
};

struct Exl3VeriCacheDecision {
    std::vector<std::int64_t> tokens;  // kept prefix (+ correction)
    std::size_t reject = 0;            // index of the first refused token, or tokens.size()
    std::int64_t correction = -1;
    float max_gap = 0.0F;              // largest gap among kept rows
};

// Delta of a VOIDINFER_EXL3_VERICACHE mode: "1" / "exact" keep within 0.0625
// logits, "tolerance" within 1.0; an explicit delta overrides (must be >= 0).
[[nodiscard]] inline float exl3_vericache_delta(std::string_view mode, const char* delta_override = nullptr) {
    if (mode != "1" && mode != "exact" && mode != "tolerance")
        throw std::invalid_argument("VeriCache mode must be 1, exact or tolerance");
    float delta = mode == "tolerance" ? 1.0F : 0.0625F;
    if (delta_override) delta = std::strtof(delta_override, nullptr);
    if (!(delta >= 0.0F)) throw std::invalid_argument("VeriCache delta must be >= 0");
    return delta;
}

[[nodiscard]] inline Exl3VeriCacheDecision exl3_vericache_decide(std::span<const std::int64_t> tokens,
                                                                std::span<const Exl3RowScore> scores,
                                                                float delta) {
    if (tokens.empty() || scores.size() + 1 < tokens.size()) throw std::invalid_argument("VeriCache block extent");
    Exl3VeriCacheDecision d;
    d.reject = tokens.size();
    for (std::size_t i = 0; i + 1 < tokens.size(); ++i) {
        const bool refused = delta > 0.0F ? scores[i].gap > delta : scores[i].greedy != tokens[i + 1];
        if (refused) {
            d.reject = i + 1;
            d.correction = scores[i].greedy;
            break;
        }
        d.max_gap = std::max(d.max_gap, scores[i].gap);
    }
    d.tokens.assign(tokens.begin(), tokens.begin() + static_cast<std::ptrdiff_t>(d.reject));
    if (d.correction >= 0) d.tokens.push_back(d.correction);
    return d;
}

// =====================================================================
// Sampled-admission gates — src/exl3/draft_distribution_contract.h:10-76,
// src/exl3/sampling_workspace_reservation.h:17-127,
// src/exl3/sampled_authority_boundary.h:15-123.
// =====================================================================

enum class Exl3SampledAcceptanceMethod : std::uint8_t { unspecified, independent_rejection_with_residual };
enum class Exl3DraftDistributionConditioning : std::uint8_t { parallel_masked_target_taps, autoregressive_predecessor };

struct Exl3DraftDistributionAvailability {
    bool greedy_tokens_available = false;
    bool internal_selector_scores = false;
    bool normalized_q_available = false;
    bool complete_vocabulary_support = false;
    Exl3DraftDistributionConditioning conditioning = Exl3DraftDistributionConditioning::parallel_masked_target_taps;

    // What the DFlash2 drafter publishes today: greedy tokens and selector
    // scores, no complete autoregressive q.
    [[nodiscard]] static Exl3DraftDistributionAvailability current_dflash2() noexcept {
        Exl3DraftDistributionAvailability a;
        a.greedy_tokens_available = true;
        a.internal_selector_scores = true;
        return a;
    }
    [[nodiscard]] bool supports(Exl3SampledAcceptanceMethod method) const noexcept {
        return method == Exl3SampledAcceptanceMethod::independent_rejection_with_residual && normalized_q_available &&
               complete_vocabulary_support &&
               conditioning == Exl3DraftDistributionConditioning::autoregressive_predecessor;
    }
    [[nodiscard]] bool permits_explicit_greedy_fallback() const noexcept { return greedy_tokens_available; }
};

struct Exl3DraftDistributionAuthority {
    Exl3SampledAcceptanceMethod method = Exl3SampledAcceptanceMethod::unspecified;
    Exl3DraftDistributionConditioning conditioning = Exl3DraftDistributionConditioning::parallel_masked_target_taps;
    std::shared_ptr<const void> owner;
    const float* probabilities = nullptr;
    std::uint32_t rows = 0, vocabulary = 0, row_stride = 0;
    std::uint64_t request_generation = 0, root_revision = 0;
    int first_position = 0;
    bool normalized = false, complete_vocabulary_support = false, ready = false;

    void require(Exl3SampledAcceptanceMethod expected_method, std::uint32_t expected_rows,
                 std::uint32_t expected_vocabulary, std::uint64_t expected_request_generation,
                 std::uint64_t expected_root_revision, int expected_first_position) const {
        if (expected_method != Exl3SampledAcceptanceMethod::independent_rejection_with_residual ||
            method != expected_method)
            throw std::invalid_argument("draft distribution: unsupported acceptance method");
        if (conditioning != Exl3DraftDistributionConditioning::autoregressive_predecessor)
            throw std::invalid_argument("draft distribution: q is not conditioned on the actual predecessor");
        const bool ok = owner && probabilities && ready && normalized && complete_vocabulary_support &&
                        expected_rows != 0 && expected_vocabulary != 0 && rows == expected_rows &&
                        vocabulary == expected_vocabulary && row_stride >= expected_vocabulary &&
                        request_generation == expected_request_generation &&
                        root_revision == expected_root_revision && first_position == expected_first_position;
        if (!ok) throw std::invalid_argument("draft distribution authority is missing or stale");
    }
};

// The engine's resource accounting, reduced to what a sampling workspace needs
// (src/exl3/resource_inventory.h:28-60): device bytes and an owning handle.
struct Exl3ResourceInventory {
    enum class Domain : unsigned { device, registered_host, host_metadata, graph_count, event_count, count };
    using Totals = std::array<std::uint64_t, static_cast<unsigned>(Domain::count)>;
    struct Requirement {
        Totals units{};
        std::uint64_t configuration = 0;
        void add(Domain domain, std::uint64_t count, std::uint64_t bytes) {
            if (domain >= Domain::count || count == 0 || bytes == 0)
                throw std::invalid_argument("resource requirement extent");
            std::uint64_t& total = units[static_cast<unsigned>(domain)];
            if (count > (std::numeric_limits<std::uint64_t>::max() - total) / bytes)
                throw std::overflow_error("resource requirement overflow");
            total += count * bytes;
        }
    };
    struct Allocation {
        std::shared_ptr<const void> owner;
        std::uint64_t slot = 0;
        Domain domain = Domain::device;
        std::uint64_t units = 0;
    };
};

struct Exl3SamplingWorkspacePlan {
    bool sampled = false, occurrence_counts = false;
    std::uint32_t rows = 0, vocabulary = 0;
    std::uint64_t target_probability_bytes = 0, draft_probability_bytes = 0;
    std::uint64_t residual_bytes = 0, occurrence_count_bytes = 0;
    std::uint64_t sampler_transient_bytes = 0, device_bytes = 0;
    std::uint64_t configuration = 0;

    // Greedy requests reserve nothing.  Sampled requests reserve fp32 p, q and
    // residual rows (3 x rows x V x 4 B), an int32 occurrence table when a
    // penalty is active, and the sampler's own transient workspace (for this
    // library: vi_sample_workspace_bytes / vi_verify_workspace_bytes).
    [[nodiscard]] static Exl3SamplingWorkspacePlan derive(const Exl3NormalizedSamplingPolicy& policy,
                                                          const Exl3DraftDistributionAvailability& availability,
                                                          std::uint32_t rows, std::uint64_t sampler_transient_bytes) {
        if (!policy.requires_sampled_distribution()) return {};
        if (!availability.supports(Exl3SampledAcceptanceMethod::independent_rejection_with_residual))
            throw std::invalid_argument("sampling workspace needs a complete draft q");
        if (rows == 0 || policy.vocabulary == 0) throw std::invalid_argument("sampling workspace shape");
        Exl3SamplingWorkspacePlan p;
        p.sampled = true;
        p.occurrence_counts = policy.occurrence_counts_required;
        p.rows = rows;
        p.vocabulary = policy.vocabulary;
        const std::uint64_t fp32_rows = mul(mul(rows, policy.vocabulary), sizeof(float));
        p.target_probability_bytes = p.draft_probability_bytes = p.residual_bytes = fp32_rows;
        p.occurrence_count_bytes = p.occurrence_counts ? mul(policy.vocabulary, sizeof(std::int32_t)) : 0;
        p.sampler_transient_bytes = sampler_transient_bytes;
        p.device_bytes = add(add(add(fp32_rows, fp32_rows), fp32_rows),
                             add(p.occurrence_count_bytes, sampler_transient_bytes));
        p.configuration = 0x53414D50574B0000ULL ^ (std::uint64_t(rows) << 32) ^ policy.vocabulary ^
                          (p.occurrence_counts ? 0x80000000ULL : 0ULL);
        return p;
    }

    [[nodiscard]] Exl3ResourceInventory::Requirement requirement() const {
        Exl3ResourceInventory::Requirement r;
        r.configuration = configuration;
        if (sampled) r.add(Exl3ResourceInventory::Domain::device, 1, device_bytes);
        return r;
    }

    [[nodiscard]] bool same_shape(const Exl3SamplingWorkspacePlan& o) const noexcept {
        return sampled == o.sampled && occurrence_counts == o.occurrence_counts && rows == o.rows &&
               vocabulary == o.vocabulary && target_probability_bytes == o.target_probability_bytes &&
               draft_probability_bytes == o.draft_probability_bytes && residual_bytes == o.residual_bytes &&
               occurrence_count_bytes == o.occurrence_count_bytes &&
               sampler_transient_bytes == o.sampler_transient_bytes && device_bytes == o.device_bytes &&
               configuration == o.configuration;
    }

private:
    static std::uint64_t mul(std::uint64_t a, std::uint64_t b) {
        if (b != 0 && a > std::numeric_limits<std::uint64_t>::max() / b)
            throw std::overflow_error("sampling workspace size overflows");
        return a * b;
    }
    static std::uint64_t add(std::uint64_t a, std::uint64_t b) {
        if (b > std::numeric_limits<std::uint64_t>::max() - a)
            throw std::overflow_error("sampling workspace size overflows");
        return a + b;
    }
};

class Exl3SamplingWorkspaceAuthority {
public:
    [[nodiscard]] static Exl3SamplingWorkspaceAuthority from_reserved_allocation(
        Exl3SamplingWorkspacePlan plan, const Exl3ResourceInventory::Allocation& allocation, void* data,
        std::uint64_t request_generation, std::uint64_t root_revision, std::uint64_t acquisition) {
        if (!plan.sampled || plan.device_bytes == 0 || !data || !allocation.owner ||
            allocation.domain != Exl3ResourceInventory::Domain::device || allocation.units != plan.device_bytes ||
            request_generation == 0 || root_revision == 0 || acquisition == 0)
            throw std::invalid_argument("sampling workspace reservation does not bind");
        return Exl3SamplingWorkspaceAuthority(std::move(plan), allocation.owner, data, request_generation,
                                              root_revision, acquisition);
    }

    Exl3SamplingWorkspaceAuthority(const Exl3SamplingWorkspaceAuthority&) = delete;
    Exl3SamplingWorkspaceAuthority& operator=(const Exl3SamplingWorkspaceAuthority&) = delete;
    Exl3SamplingWorkspaceAuthority(Exl3SamplingWorkspaceAuthority&&) = default;
    Exl3SamplingWorkspaceAuthority& operator=(Exl3SamplingWorkspaceAuthority&&) = default;

    [[nodiscard]] bool matches(const Exl3SamplingWorkspacePlan& expected, std::uint64_t request_generation,
                               std::uint64_t root_revision, std::uint64_t acquisition) const noexcept {
        return owner_ && data_ && plan_.same_shape(expected) && request_generation_ == request_generation &&
               root_revision_ == root_revision && acquisition_ == acquisition;
    }
    [[nodiscard]] const std::shared_ptr<const void>& owner() const noexcept { return owner_; }
    [[nodiscard]] const Exl3SamplingWorkspacePlan& plan() const noexcept { return plan_; }
    [[nodiscard]] void* data() const noexcept { return data_; }

private:
    Exl3SamplingWorkspaceAuthority(Exl3SamplingWorkspacePlan plan, std::shared_ptr<const void> owner, void* data,
                                   std::uint64_t request_generation, std::uint64_t root_revision,
                                   std::uint64_t acquisition)
        : plan_(std::move(plan)), owner_(std::move(owner)), data_(data), request_generation_(request_generation),
          root_revision_(root_revision), acquisition_(acquisition) {}

    Exl3SamplingWorkspacePlan plan_;
    std::shared_ptr<const void> owner_;
    void* data_ = nullptr;
    std::uint64_t request_generation_ = 0, root_revision_ = 0, acquisition_ = 0;
};

enum class Exl3SampledApiExposure : std::uint8_t { public_greedy_only, unqualified_source_api };

enum class Exl3SampledAdmissionDisposition : std::uint8_t {
    greedy,
    draft_distribution_unavailable,
    public_sampled_disabled,
    request_state_unavailable,
    target_distribution_unavailable,
    draft_distribution_invalid,
    target_distribution_invalid,
    workspace_unavailable,
    unqualified_source_ready
};

struct Exl3SampledAdmissionRequest {
    Exl3NormalizedSamplingPolicy policy;
    Exl3DraftDistributionAvailability draft_availability;
    Exl3SampledApiExposure exposure = Exl3SampledApiExposure::public_greedy_only;
    const Exl3RequestSamplingState* request_state = nullptr;
    const Exl3DraftDistributionAuthority* draft_q = nullptr;
    const Exl3SampledDistributionAuthority* target_p = nullptr;
    const Exl3SamplingWorkspaceAuthority* workspace = nullptr;
    const Exl3SamplingWorkspacePlan* workspace_plan = nullptr;
    std::uint32_t rows = 0, vocabulary = 0;
    std::uint64_t request_generation = 0, root_revision = 0, target_serial = 0, acquisition = 0;
    int first_position = 0;
};

struct Exl3SampledAdmissionDecision {
    Exl3SampledAdmissionDisposition disposition = Exl3SampledAdmissionDisposition::public_sampled_disabled;
    [[nodiscard]] bool greedy() const noexcept { return disposition == Exl3SampledAdmissionDisposition::greedy; }
    [[nodiscard]] bool unqualified_source_ready() const noexcept {
        return disposition == Exl3SampledAdmissionDisposition::unqualified_source_ready;
    }
    [[nodiscard]] bool publicly_enabled() const noexcept { return greedy(); }
};

class Exl3SampledAuthorityBoundary {
public:
    // Admission gates (sampled_authority_boundary.h:58-98), in the contract's
    // order: the first gate a request fails names its disposition; one that
    // passes them all is source-ready.
    static Exl3SampledAdmissionDecision decide(const Exl3SampledAdmissionRequest& r) noexcept {
        for (const Gate& g : kGates)
            if (!g.passes(r)) return {g.refusal};
        return {Exl3SampledAdmissionDisposition::unqualified_source_ready};
    }

    static std::string_view message(Exl3SampledAdmissionDisposition value) noexcept {
        using D = Exl3SampledAdmissionDisposition;
        switch (value) {
            case D::greedy: return "greedy authority";
            case D::draft_distribution_unavailable: return "the drafter publishes no complete autoregressive q";
            case D::public_sampled_disabled: return "public sampled speculative execution is disabled";
            case D::request_state_unavailable: return "sampled request state is missing, cancelled or stale";
            case D::target_distribution_unavailable: return "target sampled distribution is unavailable";
            case D::draft_distribution_invalid: return "draft sampled distribution authority is invalid";
            case D::target_distribution_invalid: return "target sampled distribution authority is invalid";
            case D::workspace_unavailable: return "request-local sampled workspace is unavailable";
            case D::unqualified_source_ready: return "sampled authority is source-ready but unqualified";
        }
        return "invalid sampled admission disposition";
    }

private:
    using Request = Exl3SampledAdmissionRequest;
    struct Gate {
        bool (*passes)(const Request&) noexcept;
        Exl3SampledAdmissionDisposition refusal;
    };
    template <class F> static bool holds(F&& f) noexcept {   // an authority check that throws fails
        try { f(); return true; } catch (...) { return false; }
    }
    static bool wants_sampling(const Request& r) noexcept { return r.policy.requires_sampled_distribution(); }
    static bool drafter_has_q(const Request& r) noexcept {
        return r.draft_availability.supports(Exl3SampledAcceptanceMethod::independent_rejection_with_residual);
    }
    static bool exposed(const Request& r) noexcept { return r.exposure == Exl3SampledApiExposure::unqualified_source_api; }
    static bool state_current(const Request& r) noexcept {
        const Exl3RequestSamplingState* s = r.request_state;
        return s && !s->cancelled() && s->request_generation() == r.request_generation &&
               s->committed_prefix() == static_cast<std::size_t>(r.first_position);
    }
    static bool has_draft(const Request& r) noexcept { return r.draft_q != nullptr; }
    static bool has_target(const Request& r) noexcept { return r.target_p != nullptr; }
    static bool draft_valid(const Request& r) noexcept {
        return holds([&] {
            r.draft_q->require(Exl3SampledAcceptanceMethod::independent_rejection_with_residual, r.rows, r.vocabulary,
                               r.request_generation, r.root_revision, r.first_position);
        });
    }
    static bool target_valid(const Request& r) noexcept {
        return holds([&] {
            Exl3SelectionAuthorityRequirement::sampled(r.rows, r.request_generation, r.first_position, r.target_serial,
                                                       r.vocabulary).validate(*r.target_p);
        });
    }
    static bool workspace_fits(const Request& r) noexcept {
        return r.workspace && r.workspace_plan &&
               r.workspace->matches(*r.workspace_plan, r.request_generation, r.root_revision, r.acquisition);
    }
    static constexpr Gate kGates[] = {
        {&wants_sampling, Exl3SampledAdmissionDisposition::greedy},
        {&drafter_has_q, Exl3SampledAdmissionDisposition::draft_distribution_unavailable},
        {&exposed, Exl3SampledAdmissionDisposition::public_sampled_disabled},
        {&state_current, Exl3SampledAdmissionDisposition::request_state_unavailable},
        {&has_draft, Exl3SampledAdmissionDisposition::draft_distribution_invalid},
        {&has_target, Exl3SampledAdmissionDisposition::target_distribution_unavailable},
        {&draft_valid, Exl3SampledAdmissionDisposition::draft_distribution_invalid},
        {&target_valid, Exl3SampledAdmissionDisposition::target_distribution_invalid},
        {&workspace_fits, Exl3SampledAdmissionDisposition::workspace_unavailable},
    };
};

// =====================================================================
// Device launchers (stream-ordered, asynchronous; throw on a refused launch).
// =====================================================================

// Caller-owned scratch of the greedy packet (greedy_packet.cuh:139-161).  The
// library sizes it per (rows, V); zero-fill it once, it stays reusable.
struct Exl3GreedySplitScratch {
    void* base = nullptr;
    std::size_t size = 0;
    [[nodiscard]] static std::size_t bytes(int rows = int(kExl3GreedyPacketRows),
                                           int vocabulary = int(kDefaultVocabulary)) {
        return vi_greedy_workspace_bytes(rows, vocabulary);
    }
    [[nodiscard]] static Exl3GreedySplitScratch carve(void* storage, std::size_t storage_bytes) {
        return {storage, storage_bytes};
    }
};

// greedy_packet.cuh:256-272.  `warp` selected a CUDA kernel variant; the gfx950
// kernel has one shape, so it is accepted and ignored.
inline void exl3_launch_greedy_packet(bool warp, int rows, void* stream, const std::uint16_t* scores, int vocabulary,
                                      int stride, std::uint64_t serial, Exl3GreedyRow* output,
                                      const Exl3GreedySplitScratch& scratch) {
    (void)warp;
    detail::check(vi_greedy_rows(scores, VI_F16, rows, vocabulary, stride, serial,
                                 reinterpret_cast<vi_greedy_row*>(output), scratch.base, scratch.size, stream),
                  "greedy packet");
}

// resource_inventory.h:18-23: a bounded pool had no free reservation.
class Exl3ResourceReservationExhausted : public std::runtime_error {
public:
    Exl3ResourceReservationExhausted() : std::runtime_error("resource allocation reservation exhausted") {}
};

class Exl3GreedyPacketTransport;

// A submitted packet whose rows are on their way to the host
// (Exl3PendingGreedyPacket, text_model.h:159-173): the transport slot and the
// identity (generation, position, serial, rows) of each packet it carries.
// Move-only; dropping an unfinished one waits for its copy and frees the slot.
class Exl3PendingGreedyPacket {
public:
    struct Member {
        int rows = 0;
        std::uint64_t generation = 0;
        int position = 0;
        std::uint64_t serial = 0;
    };
    Exl3PendingGreedyPacket() = default;
    Exl3PendingGreedyPacket(Exl3PendingGreedyPacket&& o) noexcept { *this = std::move(o); }
    Exl3PendingGreedyPacket& operator=(Exl3PendingGreedyPacket&& o) noexcept {
        if (this != &o) {
            drop();
            transport_ = std::exchange(o.transport_, nullptr);
            slot_ = std::exchange(o.slot_, -1);
            rows_ = std::exchange(o.rows_, 0);
            members_ = std::move(o.members_);
        }
        return *this;
    }
    Exl3PendingGreedyPacket(const Exl3PendingGreedyPacket&) = delete;
    Exl3PendingGreedyPacket& operator=(const Exl3PendingGreedyPacket&) = delete;
    ~Exl3PendingGreedyPacket() { drop(); }
    [[nodiscard]] bool valid() const noexcept { return transport_ != nullptr; }
    [[nodiscard]] std::span<const Member> members() const noexcept { return members_; }

private:
    friend class Exl3GreedyPacketTransport;
    void drop() noexcept {
        if (!transport_) return;
        std::vector<vi_greedy_row> sink(static_cast<std::size_t>(rows_));
        (void)vi_packet_finish(transport_, slot_, sink.data(), rows_);
        transport_ = nullptr;
    }
    vi_packet_transport* transport_ = nullptr;
    int slot_ = -1, rows_ = 0;
    std::vector<Member> members_;
};

// The readback side of Exl3TextContext::submit_greedy_packet /
// finish_greedy_packet (text_model.cu:12225-12355) and of the cross-context
// batch (engine_greedy_packet_batch.h:17-60), over vi_packet_*: the packet
// launch writes its rows to device memory, submit starts their copy, finish
// waits and returns the validated packet.  A batch is several lanes' packets
// laid end to end by one launch, copied once and split and validated per lane.
class Exl3GreedyPacketTransport {
public:
    explicit Exl3GreedyPacketTransport(int slots = 2, int max_rows = int(kExl3GreedyPacketRows)) {
        detail::check(vi_packet_transport_create(slots, max_rows, &t_), "greedy packet transport");
    }
    ~Exl3GreedyPacketTransport() {
        if (t_) (void)vi_packet_transport_destroy(t_);
    }
    Exl3GreedyPacketTransport(const Exl3GreedyPacketTransport&) = delete;
    Exl3GreedyPacketTransport& operator=(const Exl3GreedyPacketTransport&) = delete;

    // One context's packet of `rows` rows (1..16) at `device_rows`.
    [[nodiscard]] Exl3PendingGreedyPacket submit(const Exl3GreedyRow* device_rows, int rows, std::uint64_t generation,
                                                 int position, std::uint64_t serial, void* stream) {
        const Exl3PendingGreedyPacket::Member m{rows, generation, position, serial};
        return submit_batch(device_rows, std::span<const Exl3PendingGreedyPacket::Member>(&m, 1), stream);
    }
    // Several lanes' packets, member i's rows following member i-1's.
    [[nodiscard]] Exl3PendingGreedyPacket submit_batch(const Exl3GreedyRow* device_rows,
                                                       std::span<const Exl3PendingGreedyPacket::Member> members,
                                                       void* stream) {
        int total = 0;
        for (const auto& m : members) {
            if (m.rows < 1 || m.rows > int(kExl3GreedyPacketRows) || m.serial == 0)
                throw std::invalid_argument("greedy packet rows/serial");
            total += m.rows;
        }
        if (members.empty()) throw std::invalid_argument("greedy packet batch is empty");
        int slot = -1;
        const vi_status st = vi_packet_submit(t_, reinterpret_cast<const vi_greedy_row*>(device_rows), total, stream,
                                              &slot);
        if (st == VI_ERR_WORKSPACE) throw Exl3ResourceReservationExhausted();
        detail::check(st, "pending greedy packet download");
        Exl3PendingGreedyPacket p;
        p.transport_ = t_;
        p.slot_ = slot;
        p.rows_ = total;
        p.members_.assign(members.begin(), members.end());
        return p;
    }
    [[nodiscard]] bool ready(const Exl3PendingGreedyPacket& p) const {
        if (p.transport_ != t_) throw std::logic_error("pending greedy packet belongs to another transport");
        int r = 0;
        detail::check(vi_packet_query(t_, p.slot_, &r), "pending greedy packet poll");
        return r != 0;
    }
    // finish_greedy_packet: the packet must still be the one the caller waits
    // for (its current generation, position and serial), else runtime_error.
    Exl3GreedyPacket finish(Exl3PendingGreedyPacket&& p, std::uint64_t generation, int position,
                            std::uint64_t serial, int vocabulary = int(kDefaultVocabulary)) {
        if (p.members_.size() != 1) throw std::logic_error("finish takes a single packet; use finish_batch");
        const auto m = p.members_[0];
        auto packets = finish_batch(std::move(p), vocabulary);
        if (m.generation != generation || m.position != position || m.serial != serial)
            throw std::runtime_error("stale pending greedy packet");
        return packets[0];
    }
    std::vector<Exl3GreedyPacket> finish_batch(Exl3PendingGreedyPacket&& p, int vocabulary = int(kDefaultVocabulary)) {
        if (!p.valid() || p.transport_ != t_) throw std::logic_error("pending greedy packet is empty or foreign");
        std::vector<vi_greedy_row> rows(static_cast<std::size_t>(p.rows_));
        const vi_status st = vi_packet_finish(t_, p.slot_, rows.data(), p.rows_);
        p.transport_ = nullptr;   // the slot is free (or retired) either way
        if (st != VI_OK) throw std::runtime_error("pending greedy packet completion failed");
        std::vector<Exl3GreedyPacket> out;
        std::size_t at = 0;
        for (const auto& m : p.members_) {
            Exl3GreedyPacket g;
            g.rows = std::uint32_t(m.rows);
            g.generation = m.generation;
            g.position = m.position;
            g.serial = m.serial;
            g.ready = true;
            for (int r = 0; r < m.rows; ++r, ++at)
                g.decisions[std::size_t(r)] = Exl3GreedyRow{rows[at].serial, rows[at].token, rows[at].nonfinite};
            g.validate(std::uint32_t(m.rows), m.generation, m.position, m.serial, vocabulary);
            out.push_back(g);
        }
        return out;
    }

private:
    vi_packet_transport* t_ = nullptr;
};

// Caller-owned scratch of the sampled packet (sampled_select.cuh:200-216).
struct Exl3SampledSliceScratch {
    void* base = nullptr;
    std::size_t size = 0;
    [[nodiscard]] static std::size_t bytes(int rows = int(kExl3GreedyPacketRows),
                                           int vocabulary = int(kDefaultVocabulary)) {
        return vi_sampled_packet_workspace_bytes(rows, vocabulary);
    }
    [[nodiscard]] static Exl3SampledSliceScratch carve(void* storage, std::size_t storage_bytes) {
        return {storage, storage_bytes};
    }
};

// sampled_select.cuh:362-377.
inline void exl3_launch_sampled_packet(int rows, void* stream, const std::uint16_t* scores, int vocabulary,
                                       int stride, const Exl3DeviceSampling& cfg, int first_key,
                                       std::span<const int> depths, std::span<const int> inputs,
                                       std::uint64_t serial, Exl3GreedyRow* output, Exl3SampledSliceScratch scratch) {
    const vi_device_sampling c = cfg.abi();
    detail::check(vi_sampled_packet(scores, VI_F16, rows, vocabulary, stride, &c, first_key, depths.data(),
                                    static_cast<int>(depths.size()), inputs.data(),
                                    static_cast<int>(inputs.size()), serial,
                                    reinterpret_cast<vi_greedy_row*>(output), scratch.base, scratch.size, stream),
                  "sampled packet");
}

// sampled_select.h:33-35 (the table spans the vocabulary).
inline void exl3_presence_reset(std::int32_t* table, void* stream, int vocabulary = int(kDefaultVocabulary)) {
    detail::check(vi_presence_reset(table, vocabulary, stream), "presence reset");
}
inline void exl3_presence_truncate(std::int32_t* table, int from, void* stream,
                                   int vocabulary = int(kDefaultVocabulary)) {
    detail::check(vi_presence_truncate(table, vocabulary, from, stream), "presence truncate");
}
inline void exl3_presence_record(std::int32_t* table, int first, const std::int64_t* tokens, std::size_t count,
                                 void* stream, int vocabulary = int(kDefaultVocabulary)) {
    detail::check(vi_presence_record(table, vocabulary, first, tokens, count, stream), "presence record");
}

// DFlash2 draft proposal configuration — src/exl3/dflash2_draft.cu:2562-2572
// (the 48-byte layout of vi_draft_sampling).
struct DraftSelectSampling {
    float inv_temperature = 0.0F, top_p = 1.0F, min_p = 0.0F;
    int top_k = 0;
    unsigned long long seed = 0;
    int key_base = 0, pad = 0;
    float presence_penalty = 0.0F;
    const std::int32_t* first_occurrence = nullptr;
};
static_assert(sizeof(DraftSelectSampling) == sizeof(vi_draft_sampling) && sizeof(DraftSelectSampling) == 48);
static_assert(offsetof(DraftSelectSampling, first_occurrence) == offsetof(vi_draft_sampling, first_occurrence));

// dflash_sampled_choice (dflash2_draft.cu:2574-2610) for every position of every
// lane: `sampling` is a device array of one DraftSelectSampling per lane.
inline void dflash_sampled_choices(int lanes, int positions, const float* scores, const std::int64_t* candidates,
                                   const std::int64_t* seed_tokens, const DraftSelectSampling* sampling,
                                   std::int64_t* proposals, void* stream,
                                   int vocabulary = int(kDefaultVocabulary)) {
    detail::check(vi_draft_choice(lanes, positions, vocabulary, scores, candidates, seed_tokens,
                                  reinterpret_cast<const vi_draft_sampling*>(sampling), proposals, stream),
                  "draft sampled choice");
}

// Scratch of the top-k route (vi_topk_workspace_bytes).  Left empty, the
// library's own is used, as the reference's qualification entry keeps its own.
struct Exl3TopkScratch {
    void* base = nullptr;
    std::size_t size = 0;
};

// dflash2_draft.h:198-202.  `parallel` / `local_merge` chose CUDA routes; the
// gfx950 kernel is exact on every route, so both are accepted and ignored.
inline void dflash2_topk16_for_test(const std::uint16_t* logits, int rows, int vocab, std::int64_t* ids,
                                    float* values, bool parallel, bool local_merge = false, void* stream = nullptr,
                                    unsigned int* nonfinite_flag = nullptr, Exl3TopkScratch scratch = {}) {
    (void)parallel;
    (void)local_merge;
    if (rows == 0) return;
    if (!scratch.base) {
        detail::check(vi_topk16_for_test(logits, rows, vocab, ids, values, nonfinite_flag, stream), "top-16");
        return;
    }
    detail::check(vi_topk_rows(logits, VI_F16, rows, vocab, vocab, 16, ids, values, nullptr, nonfinite_flag,
                               scratch.base, scratch.size, stream),
                  "top-16");
}

}  // namespace voidinfer_amd

#endif  // VOIDINFER_SAMPLING_HPP
