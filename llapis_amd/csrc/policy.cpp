// policy.cpp -- the expert residency policy behind moert_policy.h.  Host code,
// standard library only.
//
// The pieces:
//   Ema        one exponential-average step over n observation steps, with the
//              weight of counts spread evenly over those steps;
//   Book       one layer: its page table (slot -> expert, expert -> slot, slot
//              states) with the blend-path mirrors derived from it (a mirror
//              entry is set exactly while its expert's slot is READY), and the
//              layer's score rows (routes since the last fold, session and
//              recent EMAs ranking survivors at resize, per-visible-token use
//              rate that the decision forecasts from);
//   Ranking    lazy best-first extraction from a binary heap: the decision
//              needs the head of each order only as far as its pairing goes;
//   Decision   one refresh: every layer proposes moves (a non-resident into a
//              free slot, or in place of a weaker resident), the moves are
//              taken highest saving first up to the token's cap, re-checked
//              against the page table as they go;
//   Timeline   one sample per visible token for the windowed rates.
//
// Decisions equal the reference's call for call (moert/policy/policy.cpp):
// the float EMA arithmetic (its :85-125), the forecast H min(1, rate (1 - d))
// (:131-135), the two pairing orders -- non-residents by forecast, highest
// first, ties by id; residents by forecast, lowest first, ties by id -- and
// the pairing rule (:262-300), and the order the moves are taken in: the
// whole list of moves, built layer by layer (free-slot moves, then swaps),
// passed through std::sort on the saving (:303-315), which fixes the order of
// equal savings as well.
#include "../../include/moert_policy.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <vector>

namespace {

constexpr int32_t kFree = MOERT_SLOT_FREE, kFilling = MOERT_SLOT_FILLING, kReady = MOERT_SLOT_READY;

struct Ema {
    float keep, take;     // s <- keep s + take c
    // n <= 1: one plain step; n > 1: keep = d^n, take = (1 - d^n) / ((1 - d) n),
    // the exact result of n single steps of c / n each
    static Ema over(float d, long long n) {
        if (n <= 1) return {d, 1.0f};
        const float keep = (float)std::pow((double)d, (double)n);
        return {keep, (float)((1.0 - keep) / ((1.0 - (double)d) * (double)n))};
    }
    float step(float s, float c) const { return keep * s + take * c; }
};

struct Book {
    int n_expert = 0;
    int active = 0;                          // slots the decision may use
    std::vector<int32_t> slot_of;            // [E] slot | -1
    std::vector<int32_t> hotmap;             // [E] slot while READY, else 0
    std::vector<float> resid;                // [E] 1 while READY, else 0
    std::vector<int32_t> held_by;            // [slots] expert | -1
    std::vector<int32_t> state;              // [slots] FREE / FILLING / READY
    std::vector<float> routes, session, recent, rate;   // [E]

    void init(int E, int slots) {
        n_expert = E;
        active = slots;
        slot_of.assign(E, -1);
        hotmap.assign(E, 0);
        resid.assign(E, 0.0f);
        routes.assign(E, 0.0f);
        session.assign(E, 0.0f);
        recent.assign(E, 0.0f);
        rate.assign(E, 0.0f);
        held_by.assign(slots, -1);
        state.assign(slots, kFree);
    }
    bool valid_slot(int s) const { return s >= 0 && s < active; }
    // the partition's predicate: resident in an active slot that is READY
    bool serves_hot(int e) const {
        const int s = slot_of[e];
        return s >= 0 && s < active && state[s] == kReady;
    }
    void show(int e, int s) {                // mirrors of a READY resident
        hotmap[e] = s;
        resid[e] = 1.0f;
    }
    void hide(int e) {
        hotmap[e] = 0;
        resid[e] = 0.0f;
    }
    void seat(int e, int s, int st) {
        slot_of[e] = s;
        held_by[s] = e;
        state[s] = st;
        if (st == kReady) show(e, s);
    }
    // empties slot s; returns its expert (-1 if it held none)
    int vacate(int s) {
        const int e = held_by[s];
        if (e < 0) return -1;
        slot_of[e] = -1;
        held_by[s] = -1;
        state[s] = kFree;
        hide(e);
        return e;
    }
    float blended(const moert_policy_config & c, int e) const {
        float v = c.blend_a * recent[e] + c.blend_b * session[e];
        if (c.blend_c != 0.0f && resid[e] > 0.0f) v += c.blend_c * c.seed_prior;
        return v;
    }
};

// Best-first extraction under a strict weak order `first(a, b)` (a comes before b).
template <typename First>
class Ranking {
public:
    Ranking(std::vector<int> & items, First first) : v_(items), first_(first) {
        std::make_heap(v_.begin(), v_.end(), [this](int a, int b) { return first_(b, a); });
    }
    bool empty() const { return v_.empty(); }
    int head() const { return v_.front(); }
    void drop() {
        std::pop_heap(v_.begin(), v_.end(), [this](int a, int b) { return first_(b, a); });
        v_.pop_back();
    }

private:
    std::vector<int> & v_;
    First first_;
};

struct Move {
    float gain;          // forecast uses saved beyond the price
    int layer, expert, slot;
    int victim;          // the resident it replaces, -1 for a free slot
};

struct Timeline {
    static constexpr int kCap = 128;
    struct Point {
        double t_ms;
        long long hot, cold;
    } pts[kCap] = {};
    long long n = 0;
    void push(double t, long long hot, long long cold) { pts[n++ % kCap] = {t, hot, cold}; }
    const Point & back(long long i) const { return pts[(n - 1 - i) % kCap]; }   // i = 0: the latest
};

double clock_ms() {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

}  // namespace

struct moert_policy {
    moert_policy_config cfg{};
    moert_policy_callbacks cbs{};
    std::vector<Book> books;

    bool external = false;             // counts arrive through add_external_counts
    long long unfolded_steps = 0;      // steps the external counts not yet folded cover
    long long unfolded_visible = 0;    // ... of them visible decode tokens

    int boundary_layer = -1;           // a boundary pass decides this layer alone
    float boundary_price = -1.0f;
    const float * ext_f = nullptr;     // [L][E] host forecast, or NULL
    float ext_price = 0.0f;
    int32_t ext_cap = 0;

    moert_policy_stats ledger{};       // occupancy is computed when read
    Timeline timeline;

    int n_layers() const { return (int)books.size(); }
    bool has(int il) const { return il >= 0 && il < n_layers(); }
    void pull() {
        if (external && cbs.fetch_external) cbs.fetch_external(cbs.user);
    }

    // routes -> use rate (visible steps only), then routes -> session / recent
    void fold(long long steps, long long visible) {
        const Ema es = Ema::over(cfg.session_decay, steps), er = Ema::over(cfg.recent_decay, steps);
        const Ema eu = Ema::over(cfg.cost_rate_decay, visible);
        for (Book & b : books)
            for (int e = 0; e < b.n_expert; ++e) {
                const float c = b.routes[e];
                if (visible > 0) b.rate[e] = eu.step(b.rate[e], c);
                b.session[e] = es.step(b.session[e], c);
                b.recent[e] = er.step(b.recent[e], c);
                b.routes[e] = 0.0f;
            }
    }

    // expected uses of each expert of layer il over the next H visible tokens
    void forecast(int il, std::vector<float> & f) const {
        const Book & b = books[il];
        f.resize(b.n_expert);
        if (ext_f && boundary_layer < 0) {
            std::copy(ext_f + (size_t)il * cfg.n_expert, ext_f + (size_t)(il + 1) * cfg.n_expert, f.begin());
            return;
        }
        const float H = (float)cfg.cost_horizon, per_use = 1.0f - cfg.cost_rate_decay;
        for (int e = 0; e < b.n_expert; ++e) f[e] = H * std::min(1.0f, b.rate[e] * per_use);
    }

    void propose(int il, float price, std::vector<Move> & moves) const;
    bool promote(int il, int e, int slot);
    void decide(int32_t reason);
};

// Layer il's moves in pairing order: the best non-residents go to the free
// slots (ascending) while a promotion pays its price, then replace the weakest
// residents while the saving over the resident pays it; the first move that
// does not pay ends each of the two runs.
void moert_policy::propose(int il, float price, std::vector<Move> & moves) const {
    const Book & b = books[il];
    std::vector<float> f;
    forecast(il, f);
    std::vector<int> outside, free_slots, residents;
    for (int e = 0; e < b.n_expert; ++e)
        if (b.slot_of[e] < 0) outside.push_back(e);
    if (outside.empty()) return;
    for (int s = 0; s < b.active; ++s) {
        if (b.held_by[s] < 0) free_slots.push_back(s);
        else residents.push_back(b.held_by[s]);
    }
    auto stronger = [&](int a, int c) { return f[a] > f[c] || (f[a] == f[c] && a < c); };
    auto weaker = [&](int a, int c) { return f[a] < f[c] || (f[a] == f[c] && a < c); };
    Ranking<decltype(stronger)> in(outside, stronger);
    for (int s : free_slots) {
        if (in.empty()) break;
        const int e = in.head();
        if (f[e] <= price) break;
        moves.push_back({f[e] - price, il, e, s, -1});
        in.drop();
    }
    if (in.empty() || residents.empty()) return;
    Ranking<decltype(weaker)> out(residents, weaker);
    while (!in.empty() && !out.empty()) {
        const int e = in.head(), v = out.head();
        const float saving = f[e] - f[v];
        if (saving <= price) break;
        moves.push_back({saving - price, il, e, b.slot_of[v], v});
        in.drop();
        out.drop();
    }
}

// ask the host for expert e's hot bytes in (il, slot): 1 READY now, 2 FILLING
// until complete_fill, 0 refused
bool moert_policy::promote(int il, int e, int slot) {
    const int32_t r = cbs.stream_expert ? cbs.stream_expert(cbs.user, il, e, slot) : 0;
    if (r == 0) return false;
    books[il].seat(e, slot, r == 2 ? kFilling : kReady);
    if (r == 2) ++ledger.fills_async;
    ++ledger.promotions;
    return true;
}

void moert_policy::decide(int32_t reason) {
    if (external) {
        // the one place the scores must be current: pour in the counts and
        // fold the whole span at once
        if (cbs.fetch_external) cbs.fetch_external(cbs.user);
        fold(std::max<long long>(1, unfolded_steps), unfolded_visible);
        unfolded_steps = unfolded_visible = 0;
    }
    const double t0 = clock_ms();
    const bool ext = ext_f && boundary_layer < 0;
    long long cap = (long long)1 << 40;
    if (reason == MOERT_REFRESH_VISIBLE_INTERVAL) cap = ext && ext_cap > 0 ? ext_cap : cfg.cost_per_token;
    const float price = boundary_price >= 0.0f ? boundary_price : (ext ? ext_price : cfg.cost_reuse);

    std::vector<Move> moves;
    for (int il = 0; il < n_layers(); ++il)
        if (boundary_layer < 0 || il == boundary_layer) propose(il, price, moves);
    std::sort(moves.begin(), moves.end(), [](const Move & a, const Move & b) { return a.gain > b.gain; });

    std::vector<char> touched((size_t)n_layers(), 0);
    long long promoted = 0, demoted = 0;
    for (const Move & m : moves) {
        if (promoted >= cap) break;
        Book & b = books[m.layer];
        if (b.slot_of[m.expert] >= 0) continue;                 // an earlier move seated it
        const int in_slot = b.held_by[m.slot];
        if (in_slot != m.victim) continue;                      // the slot changed since the proposal
        if (m.victim >= 0) {
            b.vacate(m.slot);
            ++ledger.demotions;
            ++demoted;
        }
        if (!promote(m.layer, m.expert, m.slot)) continue;      // refused: the slot stays free
        touched[m.layer] = 1;
        ++promoted;
    }
    if (cbs.publish_layer)
        for (int il = 0; il < n_layers(); ++il)
            if (touched[il]) cbs.publish_layer(cbs.user, il);

    const double ms = clock_ms() - t0;
    ++ledger.refresh_count;
    ledger.refresh_promotions += promoted;
    ledger.refresh_demotions += demoted;
    ledger.refresh_pause_ms_total += ms;
    ledger.refresh_pause_ms_max = std::max(ledger.refresh_pause_ms_max, ms);
    ledger.last_refresh_tok = ledger.visible_tokens;
    ledger.last_refresh_promos = promoted;
    ledger.last_refresh_pause_ms = ms;
}

extern "C" {

void moert_policy_config_defaults(moert_policy_config * cfg) {
    if (!cfg) return;
    memset(cfg, 0, sizeof(*cfg));
    cfg->seed_prior = 5.0f;
    cfg->session_decay = 0.995f;
    cfg->recent_decay = 0.95f;
    cfg->blend_a = 1.0f;
    cfg->blend_b = 0.25f;
    cfg->blend_c = 0.0f;
    cfg->cost_horizon = 16;
    cfg->cost_reuse = 2.0f;
    cfg->cost_rate_decay = 0.97857206f;   // 0.5^(1/32): a use counts half after 32 visible tokens
    cfg->cost_per_token = 4;
}

moert_policy * moert_policy_create(const moert_policy_config * cfg, const moert_policy_callbacks * cbs) {
    if (!cfg || cfg->n_layers <= 0 || cfg->n_expert <= 0 || cfg->k <= 0 || cfg->k > cfg->n_expert) return nullptr;
    const int L = cfg->n_layers, E = cfg->n_expert;
    if (cfg->k_per_layer)
        for (int il = 0; il < L; ++il)
            if (cfg->k_per_layer[il] < 1 || cfg->k_per_layer[il] > E) return nullptr;
    moert_policy * p = new moert_policy();
    p->cfg = *cfg;
    p->cfg.k_per_layer = nullptr;          // the table is copied into the books
    p->cfg.cost_per_token = std::max(1, p->cfg.cost_per_token);
    if (cbs) p->cbs = *cbs;
    p->books.resize(L);
    for (int il = 0; il < L; ++il) p->books[il].init(E, cfg->k_per_layer ? cfg->k_per_layer[il] : cfg->k);
    return p;
}

void moert_policy_free(moert_policy * p) { delete p; }

void moert_policy_set_external_observation(moert_policy * p, int32_t on) {
    if (p) p->external = on != 0;
}

void moert_policy_observe(moert_policy * p, int32_t il, const int32_t * ids, int32_t n_used, int64_t n_tok) {
    if (!p || !p->has(il) || !ids) return;
    Book & b = p->books[il];
    const int64_t n = n_tok * (int64_t)n_used;
    for (int64_t i = 0; i < n; ++i) {
        const int e = ids[i];
        if (e < 0 || e >= b.n_expert) continue;
        b.routes[e] += 1.0f;
        ++(b.serves_hot(e) ? p->ledger.hot_routes : p->ledger.cold_routes);
    }
}

void moert_policy_set_external_forecast(moert_policy * p, const float * f, float r, int32_t cap) {
    if (!p) return;
    p->ext_f = f;
    p->ext_price = r;
    p->ext_cap = cap;
}

void moert_policy_on_prompt_token(moert_policy * p, int64_t n_tokens) {
    if (!p) return;
    const long long n = std::max<int64_t>(1, n_tokens);
    p->ledger.tokens += n;
    if (p->external) p->unfolded_steps += n;
    else p->fold(n_tokens, 0);            // prompt routing never moves the use rate
}

void moert_policy_on_token_end(moert_policy * p) {
    if (!p) return;
    ++p->ledger.tokens;
    ++p->ledger.visible_tokens;
    p->timeline.push(clock_ms(), p->ledger.hot_routes, p->ledger.cold_routes);
    if (p->external) {
        ++p->unfolded_steps;
        ++p->unfolded_visible;
    } else {
        p->fold(1, 1);
    }
    p->decide(MOERT_REFRESH_VISIBLE_INTERVAL);
}

void moert_policy_refresh(moert_policy * p, int32_t reason) {
    if (p) p->decide(reason);
}

int32_t moert_policy_resize_k(moert_policy * p, int32_t k_new) {
    if (!p || k_new < 1 || k_new > p->cfg.n_expert) return 0;
    for (Book & b : p->books) {
        // survivors: the residents by blended score, highest first (ties by id)
        std::vector<int> res;
        for (int s = 0; s < b.active; ++s)
            if (b.held_by[s] >= 0) res.push_back(b.held_by[s]);
        std::vector<float> score(b.n_expert, 0.0f);
        for (int e : res) score[e] = b.blended(p->cfg, e);
        std::sort(res.begin(), res.end(),
                  [&](int a, int c) { return score[a] != score[c] ? score[a] > score[c] : a < c; });
        const int keep = std::min((int)res.size(), (int)k_new);
        for (size_t i = keep; i < res.size(); ++i) {
            b.slot_of[res[i]] = -1;
            b.hide(res[i]);
            ++p->ledger.demotions;
        }
        // the new slot arrays: survivors packed into slots 0.. in rank order,
        // READY (the host re-streams each into its new slot before the next
        // fire)
        b.held_by.assign(k_new, -1);
        b.state.assign(k_new, kFree);
        b.active = k_new;
        for (int i = 0; i < keep; ++i) b.seat(res[i], i, kReady);
    }
    p->cfg.k = k_new;
    return 1;
}

int32_t moert_policy_set_active_k(moert_policy * p, int32_t k) {
    if (!p || k < 1) return 0;
    for (Book & b : p->books) {
        const int slots = (int)b.held_by.size();
        const int keep = std::min((int)k, slots);
        for (int s = keep; s < slots; ++s) {
            const bool was_ready = b.state[s] == kReady;
            if (b.vacate(s) >= 0 && was_ready) ++p->ledger.demotions;   // an unfinished fill is no demotion
        }
        b.active = keep;
    }
    return 1;
}

// a completion or an abort matches only the slot's FILLING resident
static bool filling_match(moert_policy * p, int32_t il, int32_t slot, int32_t e) {
    const Book & b = p->books[il];
    if (b.held_by[slot] == e && b.state[slot] == kFilling) return true;
    ++p->ledger.fills_stale;
    return false;
}

int32_t moert_policy_complete_fill(moert_policy * p, int32_t il, int32_t slot, int32_t e) {
    if (!p || !p->has(il) || !p->books[il].valid_slot(slot) || !filling_match(p, il, slot, e)) return 0;
    Book & b = p->books[il];
    b.state[slot] = kReady;
    b.show(e, slot);
    ++p->ledger.fills_completed;
    return 1;
}

int32_t moert_policy_abort_fill(moert_policy * p, int32_t il, int32_t slot, int32_t e) {
    if (!p || !p->has(il) || !p->books[il].valid_slot(slot) || !filling_match(p, il, slot, e)) return 0;
    p->books[il].vacate(slot);
    ++p->ledger.fills_aborted;
    return 1;
}

int32_t moert_policy_boundary_layer(moert_policy * p, int32_t il, const int32_t * counts, int64_t n_tok, float weight,
                                    float r) {
    if (!p || !p->has(il) || !counts || n_tok <= 0) return -1;
    Book & b = p->books[il];
    const float w = std::min(1.0f, std::max(0.0f, weight));
    const float d = p->cfg.cost_rate_decay;
    // the prompt's routes per token move the rate toward the steady state
    // whose per-token use rate (1 - d) equals them
    for (int e = 0; e < b.n_expert; ++e) {
        const float per_tok = std::min(1.0f, (float)counts[e] / (float)n_tok);
        b.rate[e] = (1.0f - w) * b.rate[e] + w * per_tok / (1.0f - d);
    }
    const long long before = p->ledger.refresh_promotions;
    p->boundary_layer = il;
    p->boundary_price = std::max(0.0f, r);
    p->decide(MOERT_REFRESH_BOUNDARY);
    p->boundary_layer = -1;
    p->boundary_price = -1.0f;
    return (int32_t)(p->ledger.refresh_promotions - before);
}

int32_t moert_policy_can_seed(const moert_policy * p, int32_t il, int32_t e) {
    if (!p || !p->has(il)) return 0;
    const Book & b = p->books[il];
    return e >= 0 && e < b.n_expert && b.slot_of[e] < 0 ? 1 : 0;
}

int32_t moert_policy_commit_seed(moert_policy * p, int32_t il, int32_t e, int32_t slot) {
    if (!moert_policy_can_seed(p, il, e) || !p->books[il].valid_slot(slot)) return 0;
    Book & b = p->books[il];
    b.seat(e, slot, kReady);
    b.session[e] = b.recent[e] = p->cfg.seed_prior;
    return 1;
}

void moert_policy_add_external_counts(moert_policy * p, int32_t il, const int32_t * counts, int64_t hot,
                                      int64_t cold) {
    if (!p || !p->has(il) || !counts) return;
    Book & b = p->books[il];
    for (int e = 0; e < b.n_expert; ++e) b.routes[e] += (float)counts[e];
    p->ledger.hot_routes += hot;
    p->ledger.cold_routes += cold;
}

void moert_policy_reset_stats(moert_policy * p) {
    if (!p) return;
    p->ledger = moert_policy_stats{};      // the page table and the scores stay
    p->timeline.n = 0;
}

int32_t moert_policy_layer_k(const moert_policy * p, int32_t il) {
    return p && p->has(il) ? p->books[il].active : -1;
}

double moert_policy_hit_rate(moert_policy * p) {
    if (!p) return 0.0;
    p->pull();
    const long long all = p->ledger.hot_routes + p->ledger.cold_routes;
    return all > 0 ? (double)p->ledger.hot_routes / (double)all : 0.0;
}

void moert_policy_get_stats(moert_policy * p, moert_policy_stats * out) {
    if (!p || !out) return;
    p->pull();
    *out = p->ledger;
    long long ready = 0, slots = 0;
    for (const Book & b : p->books) {
        slots += b.active;
        ready += std::count(b.state.begin(), b.state.begin() + b.active, kReady);
    }
    out->occupancy = slots > 0 ? (double)ready / (double)slots : 0.0;
}

void moert_policy_get_window(moert_policy * p, int32_t n_tokens, moert_policy_window * out) {
    if (!out) return;
    memset(out, 0, sizeof(*out));
    if (!p || n_tokens < 2) return;
    p->pull();
    const Timeline & tl = p->timeline;
    const long long n = std::min<long long>(n_tokens, std::min<long long>(tl.n, Timeline::kCap));
    if (n < 2) return;
    const Timeline::Point & first = tl.back(n - 1), & last = tl.back(0);
    out->tokens = (int32_t)n;
    out->span_ms = last.t_ms - first.t_ms;
    if (out->span_ms > 0.0) {
        out->tok_per_s = 1000.0 * (double)(n - 1) / out->span_ms;
        out->ms_per_tok = out->span_ms / (double)(n - 1);
    }
    // the routes since the window's first sample, up to now
    out->hot_routes = p->ledger.hot_routes - first.hot;
    out->cold_routes = p->ledger.cold_routes - first.cold;
    const long long all = out->hot_routes + out->cold_routes;
    if (all > 0) out->hit_rate = (double)out->hot_routes / (double)all;
}

const int32_t * moert_policy_exp_slot_view(const moert_policy * p, int32_t il) {
    return p && p->has(il) ? p->books[il].slot_of.data() : nullptr;
}
const int32_t * moert_policy_slot_exp_view(const moert_policy * p, int32_t il) {
    return p && p->has(il) ? p->books[il].held_by.data() : nullptr;
}
const int32_t * moert_policy_slot_state_view(const moert_policy * p, int32_t il) {
    return p && p->has(il) ? p->books[il].state.data() : nullptr;
}
const int32_t * moert_policy_hotmap_view(const moert_policy * p, int32_t il) {
    return p && p->has(il) ? p->books[il].hotmap.data() : nullptr;
}
const float * moert_policy_resid_view(const moert_policy * p, int32_t il) {
    return p && p->has(il) ? p->books[il].resid.data() : nullptr;
}

}  // extern "C"
