// policy.cpp -- the expert residency policy (moert_policy.h).  Host code,
// standard library only.
//
// State per layer: the page table (exp_slot, slot_exp, slot_state), the
// blend-path mirrors (hotmap, resid) and four score rows (routes since the
// last fold, the session and recent EMAs that rank survivors at resize, the
// per-visible-token use rate the decision forecasts from).  Expert-indexed
// rows live in flat [n_layers][n_expert] arrays; slot-indexed rows per layer
// (their length changes with resize_k).
//
// The arithmetic follows moert/policy/policy.cpp step for step so that the
// same calls leave the same page table: the float EMAs and their
// chunk-corrected weights (policy.cpp:85-125), the forecast (:131-135), the
// candidate lists and their orders (:262-300) and the application order of
// the pairs (:303-315, std::sort on the net saving, as the reference).
#include "../../include/moert_policy.h"
#include "../../include/llapis_moe.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <vector>

struct moert_policy {
    moert_policy_config cfg{};
    moert_policy_callbacks cbs{};
    int L = 0, E = 0;
    std::vector<int32_t> cap;               // [L] active capacity of each layer

    bool external = false;                  // counts arrive through add_external_counts
    long long pending_steps = 0;            // steps the unfolded external counts cover
    long long pending_visible = 0;          // ... of which visible decode steps

    std::vector<float> routes;              // [L][E] since the last fold
    std::vector<float> session, recent;     // [L][E] slow / fast EMA
    std::vector<float> rate;                // [L][E] per-visible-token use rate

    std::vector<int32_t> exp_slot, hotmap;  // [L][E]
    std::vector<float> resid;               // [L][E]
    std::vector<std::vector<int32_t>> slot_exp, slot_state;   // [L][cap]

    int only_layer = -1;                    // boundary pass: the one layer decided
    float price_override = -1.0f;           // boundary pass: its price
    const float * ext_forecast = nullptr;   // [L][E] or NULL
    float ext_price = 0.0f;
    int32_t ext_cap = 0;

    moert_policy_stats st{};                // occupancy is computed on read
    static constexpr int RING = 128;        // one sample per visible token
    struct Sample {
        double t_ms;
        long long hot, cold;
    } ring[RING] = {};
    long long n_samples = 0;

    size_t at(int il, int e) const { return (size_t)il * E + e; }
};

namespace {

constexpr int32_t FREE = MOERT_SLOT_FREE, FILLING = MOERT_SLOT_FILLING, READY = MOERT_SLOT_READY;

bool layer_ok(const moert_policy * p, int32_t il) { return p && il >= 0 && il < p->L; }

// EMA step for counts spread uniformly over n steps (n = 1: s = d s + c):
// s = d^n s + c (1 - d^n) / ((1 - d) n).  Returns {d^n, weight of c}.
void chunk_coef(float d, long long n_steps, float * dn, float * w) {
    if (n_steps > 1) {
        const double n = (double)n_steps;
        *dn = (float)std::pow((double)d, n);
        *w = (float)((1.0 - *dn) / ((1.0 - (double)d) * n));
    } else {
        *dn = d;
        *w = 1.0f;
    }
}

// routes -> session / recent EMAs, then clear the routes
void fold_scores(moert_policy & g, long long n_steps) {
    float ds, ws, dr, wr;
    chunk_coef(g.cfg.session_decay, n_steps, &ds, &ws);
    chunk_coef(g.cfg.recent_decay, n_steps, &dr, &wr);
    for (size_t i = 0; i < g.routes.size(); ++i) {
        const float c = g.routes[i];
        g.session[i] = ds * g.session[i] + ws * c;
        g.recent[i] = dr * g.recent[i] + wr * c;
        g.routes[i] = 0.0f;
    }
}

// routes -> use-rate EMA over n visible steps (before fold_scores clears them);
// prompt-only folds (n = 0) leave the rate alone
void fold_rate(moert_policy & g, long long n_visible) {
    if (n_visible <= 0) return;
    const double d = (double)g.cfg.cost_rate_decay;
    const float dn = (float)std::pow(d, (double)n_visible);
    const float w = n_visible > 1 ? (float)((1.0 - dn) / ((1.0 - d) * (double)n_visible)) : 1.0f;
    for (size_t i = 0; i < g.routes.size(); ++i) g.rate[i] = dn * g.rate[i] + w * g.routes[i];
}

// expected uses over the next H visible tokens (at most one per token)
float forecast(const moert_policy & g, int il, int e) {
    if (g.ext_forecast && g.only_layer < 0) return g.ext_forecast[g.at(il, e)];
    const float H = (float)g.cfg.cost_horizon;
    return H * std::min(1.0f, g.rate[g.at(il, e)] * (1.0f - g.cfg.cost_rate_decay));
}

float blended(const moert_policy & g, int il, int e) {
    float v = g.cfg.blend_a * g.recent[g.at(il, e)] + g.cfg.blend_b * g.session[g.at(il, e)];
    if (g.cfg.blend_c != 0.0f && g.resid[g.at(il, e)] > 0.0f) v += g.cfg.blend_c * g.cfg.seed_prior;
    return v;
}

void set_hot(moert_policy & g, int il, int e, int slot) {
    g.hotmap[g.at(il, e)] = slot;
    g.resid[g.at(il, e)] = 1.0f;
}
void set_cold(moert_policy & g, int il, int e) {
    g.hotmap[g.at(il, e)] = 0;
    g.resid[g.at(il, e)] = 0.0f;
}

void evict(moert_policy & g, int il, int slot) {
    const int e = g.slot_exp[il][slot];
    if (e < 0) return;
    g.exp_slot[g.at(il, e)] = -1;
    g.slot_exp[il][slot] = -1;
    g.slot_state[il][slot] = FREE;
    set_cold(g, il, e);
    ++g.st.demotions;
}

// ask the host for the bytes; 1 -> READY now, 2 -> FILLING until complete_fill
bool fill(moert_policy & g, int il, int e, int slot) {
    const int32_t r = g.cbs.stream_expert ? g.cbs.stream_expert(g.cbs.user, il, e, slot) : 0;
    if (!r) return false;
    g.slot_exp[il][slot] = e;
    g.exp_slot[g.at(il, e)] = slot;
    if (r == 2) {
        g.slot_state[il][slot] = FILLING;
        ++g.st.fills_async;
    } else {
        g.slot_state[il][slot] = READY;
        set_hot(g, il, e, slot);
    }
    ++g.st.promotions;
    return true;
}

void pull_external(moert_policy * p) {
    if (p->external && p->cbs.fetch_external) p->cbs.fetch_external(p->cbs.user);
}

double now_ms() {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

}  // namespace

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
    std::vector<int32_t> cap((size_t)cfg->n_layers, cfg->k);
    if (cfg->k_per_layer)
        for (int il = 0; il < cfg->n_layers; ++il) {
            if (cfg->k_per_layer[il] < 1 || cfg->k_per_layer[il] > cfg->n_expert) return nullptr;
            cap[il] = cfg->k_per_layer[il];
        }
    moert_policy * p = new moert_policy();
    p->cfg = *cfg;
    p->cfg.k_per_layer = nullptr;
    p->cfg.cost_per_token = std::max(1, p->cfg.cost_per_token);
    if (cbs) p->cbs = *cbs;
    p->L = cfg->n_layers;
    p->E = cfg->n_expert;
    p->cap = cap;
    const size_t n = (size_t)p->L * p->E;
    p->routes.assign(n, 0.0f);
    p->session.assign(n, 0.0f);
    p->recent.assign(n, 0.0f);
    p->rate.assign(n, 0.0f);
    p->exp_slot.assign(n, -1);
    p->hotmap.assign(n, 0);
    p->resid.assign(n, 0.0f);
    p->slot_exp.resize(p->L);
    p->slot_state.resize(p->L);
    for (int il = 0; il < p->L; ++il) {
        p->slot_exp[il].assign(cap[il], -1);
        p->slot_state[il].assign(cap[il], FREE);
    }
    return p;
}

void moert_policy_free(moert_policy * p) { delete p; }

void moert_policy_set_external_observation(moert_policy * p, int32_t on) {
    if (p) p->external = on != 0;
}

void moert_policy_observe(moert_policy * p, int32_t il, const int32_t * ids, int32_t n_used, int64_t n_tok) {
    if (!layer_ok(p, il) || !ids) return;
    moert_policy & g = *p;
    for (int64_t i = 0; i < n_tok * (int64_t)n_used; ++i) {
        const int e = ids[i];
        if (e < 0 || e >= g.E) continue;
        g.routes[g.at(il, e)] += 1.0f;
        const int s = g.exp_slot[g.at(il, e)];
        if (s >= 0 && s < g.cap[il] && g.slot_state[il][s] == READY) ++g.st.hot_routes;
        else ++g.st.cold_routes;
    }
}

void moert_policy_set_external_forecast(moert_policy * p, const float * f, float r, int32_t cap) {
    if (!p) return;
    p->ext_forecast = f;
    p->ext_price = r;
    p->ext_cap = cap;
}

void moert_policy_on_prompt_token(moert_policy * p, int64_t n_tokens) {
    if (!p) return;
    const long long n = std::max<int64_t>(1, n_tokens);
    p->st.tokens += n;
    if (p->external) p->pending_steps += n;
    else fold_scores(*p, n_tokens);
}

void moert_policy_on_token_end(moert_policy * p) {
    if (!p) return;
    moert_policy & g = *p;
    ++g.st.tokens;
    ++g.st.visible_tokens;
    moert_policy::Sample & s = g.ring[g.n_samples % moert_policy::RING];
    s.t_ms = now_ms();
    s.hot = g.st.hot_routes;
    s.cold = g.st.cold_routes;
    ++g.n_samples;
    if (g.external) {
        ++g.pending_steps;
        ++g.pending_visible;
    } else {
        fold_rate(g, 1);
        fold_scores(g, 1);
    }
    moert_policy_refresh(p, MOERT_REFRESH_VISIBLE_INTERVAL);
}

void moert_policy_refresh(moert_policy * p, int32_t reason) {
    if (!p) return;
    moert_policy & g = *p;
    if (g.external) {
        if (g.cbs.fetch_external) g.cbs.fetch_external(g.cbs.user);
        fold_rate(g, g.pending_visible);
        fold_scores(g, std::max<long long>(1, g.pending_steps));
        g.pending_steps = g.pending_visible = 0;
    }
    const double t0 = now_ms();
    struct Pair {
        int il, e, slot, victim;
        bool swap;
        float gain;
    };
    std::vector<Pair> pairs;
    const bool ext = g.ext_forecast && g.only_layer < 0;
    const long long budget = reason == MOERT_REFRESH_VISIBLE_INTERVAL
                                 ? (long long)(ext && g.ext_cap > 0 ? g.ext_cap : g.cfg.cost_per_token)
                                 : (long long)1 << 40;
    std::vector<int> outside, free_slots, held;
    std::vector<float> fc((size_t)g.E);
    for (int il = 0; il < g.L; ++il) {
        if (g.only_layer >= 0 && il != g.only_layer) continue;
        const float r = g.price_override >= 0.0f ? g.price_override : (ext ? g.ext_price : g.cfg.cost_reuse);
        outside.clear();
        free_slots.clear();
        held.clear();
        // the layer's forecasts, once (nothing changes them during the pairing)
        bool finite = true;
        for (int e = 0; e < g.E; ++e) {
            fc[e] = forecast(g, il, e);
            finite = finite && std::isfinite(fc[e]);
        }
        float f_max = -INFINITY, f_min = INFINITY;
        for (int e = 0; e < g.E; ++e)
            if (g.exp_slot[g.at(il, e)] < 0) {
                outside.push_back(e);
                f_max = std::max(f_max, fc[e]);
            }
        for (int s = 0; s < g.cap[il]; ++s) {
            const int e = g.slot_exp[il][s];
            if (e < 0) {
                free_slots.push_back(s);
            } else {
                held.push_back(s);
                f_min = std::min(f_min, fc[e]);
            }
        }
        if (outside.empty()) continue;
        // both pairings below stop at their first candidate unless the best
        // non-resident beats the price (free slot) or the weakest resident by
        // more than the price (swap): then the layer adds no pair
        if (finite && (free_slots.empty() || f_max <= r) && (held.empty() || f_max - f_min <= r)) continue;
        // non-residents by forecast, highest first (ties: lower id first)
        std::stable_sort(outside.begin(), outside.end(), [&](int a, int b) { return fc[a] > fc[b]; });
        // occupied slots by their expert's forecast, lowest first (ties: lower id)
        std::sort(held.begin(), held.end(), [&](int a, int b) {
            const int ea = g.slot_exp[il][a], eb = g.slot_exp[il][b];
            const float fa = fc[ea], fb = fc[eb];
            return fa != fb ? fa < fb : ea < eb;
        });
        size_t next = 0;
        for (size_t i = 0; i < free_slots.size() && next < outside.size(); ++i, ++next) {
            const float f_in = fc[outside[next]];
            if (f_in <= r) break;
            pairs.push_back({il, outside[next], free_slots[i], -1, false, f_in - r});
        }
        for (size_t i = 0; i < held.size() && next < outside.size(); ++i, ++next) {
            const int victim = g.slot_exp[il][held[i]];
            const float f_in = fc[outside[next]], f_out = fc[victim];
            if (f_in - f_out <= r) break;
            pairs.push_back({il, outside[next], held[i], victim, true, f_in - f_out - r});
        }
    }
    std::sort(pairs.begin(), pairs.end(), [](const Pair & a, const Pair & b) { return a.gain > b.gain; });
    std::vector<char> touched((size_t)g.L, 0);
    long long promoted = 0, demoted = 0;
    for (const Pair & c : pairs) {
        if (promoted >= budget) break;
        if (g.exp_slot[g.at(c.il, c.e)] >= 0) continue;              // became resident meanwhile
        if (c.swap) {
            if (g.slot_exp[c.il][c.slot] != c.victim) continue;      // the victim moved
            evict(g, c.il, c.slot);
            ++demoted;
        } else if (g.slot_exp[c.il][c.slot] >= 0) {
            continue;                                                // the slot was taken
        }
        if (!fill(g, c.il, c.e, c.slot)) continue;
        touched[c.il] = 1;
        ++promoted;
    }
    if (g.cbs.publish_layer)
        for (int il = 0; il < g.L; ++il)
            if (touched[il]) g.cbs.publish_layer(g.cbs.user, il);
    const double ms = now_ms() - t0;
    ++g.st.refresh_count;
    g.st.refresh_promotions += promoted;
    g.st.refresh_demotions += demoted;
    g.st.refresh_pause_ms_total += ms;
    g.st.refresh_pause_ms_max = std::max(g.st.refresh_pause_ms_max, ms);
    g.st.last_refresh_tok = g.st.visible_tokens;
    g.st.last_refresh_promos = promoted;
    g.st.last_refresh_pause_ms = ms;
}

int32_t moert_policy_resize_k(moert_policy * p, int32_t k_new) {
    if (!p || k_new < 1 || k_new > p->E) return 0;
    moert_policy & g = *p;
    for (int il = 0; il < g.L; ++il) {
        std::vector<int> held;
        for (int s = 0; s < g.cap[il]; ++s)
            if (g.slot_exp[il][s] >= 0) held.push_back(s);
        std::sort(held.begin(), held.end(), [&](int a, int b) {
            const int ea = g.slot_exp[il][a], eb = g.slot_exp[il][b];
            const float sa = blended(g, il, ea), sb = blended(g, il, eb);
            return sa != sb ? sa > sb : ea < eb;
        });
        const int keep = std::min((int)held.size(), (int)k_new);
        for (size_t i = keep; i < held.size(); ++i) {
            const int e = g.slot_exp[il][held[i]];
            g.exp_slot[g.at(il, e)] = -1;
            set_cold(g, il, e);
            ++g.st.demotions;
        }
        // survivors compact into slots 0..keep-1 in rank order and stay READY
        // (the host re-streams each into its new slot before the next fire)
        std::vector<int32_t> se((size_t)k_new, -1), ss((size_t)k_new, FREE);
        for (int i = 0; i < keep; ++i) {
            const int e = g.slot_exp[il][held[i]];
            se[i] = e;
            ss[i] = READY;
            g.exp_slot[g.at(il, e)] = i;
            set_hot(g, il, e, i);
        }
        g.slot_exp[il].swap(se);
        g.slot_state[il].swap(ss);
        g.cap[il] = k_new;
    }
    g.cfg.k = k_new;
    return 1;
}

int32_t moert_policy_set_active_k(moert_policy * p, int32_t k) {
    if (!p || k < 1) return 0;
    moert_policy & g = *p;
    for (int il = 0; il < g.L; ++il) {
        const int alloc = (int)g.slot_exp[il].size();
        const int active = std::min((int)k, alloc);
        for (int s = active; s < alloc; ++s) {
            const int e = g.slot_exp[il][s];
            if (e < 0) continue;
            if (g.slot_state[il][s] == READY) {
                set_cold(g, il, e);
                ++g.st.demotions;
            }
            g.exp_slot[g.at(il, e)] = -1;
            g.slot_exp[il][s] = -1;
            g.slot_state[il][s] = FREE;
        }
        g.cap[il] = active;
    }
    return 1;
}

int32_t moert_policy_complete_fill(moert_policy * p, int32_t il, int32_t slot, int32_t e) {
    if (!layer_ok(p, il) || slot < 0 || slot >= p->cap[il]) return 0;
    moert_policy & g = *p;
    if (g.slot_exp[il][slot] != e || g.slot_state[il][slot] != FILLING) {
        ++g.st.fills_stale;
        return 0;
    }
    g.slot_state[il][slot] = READY;
    set_hot(g, il, e, slot);
    ++g.st.fills_completed;
    return 1;
}

int32_t moert_policy_abort_fill(moert_policy * p, int32_t il, int32_t slot, int32_t e) {
    if (!layer_ok(p, il) || slot < 0 || slot >= p->cap[il]) return 0;
    moert_policy & g = *p;
    if (g.slot_exp[il][slot] != e || g.slot_state[il][slot] != FILLING) {
        ++g.st.fills_stale;
        return 0;
    }
    g.exp_slot[g.at(il, e)] = -1;
    g.slot_exp[il][slot] = -1;
    g.slot_state[il][slot] = FREE;
    ++g.st.fills_aborted;
    return 1;
}

int32_t moert_policy_boundary_layer(moert_policy * p, int32_t il, const int32_t * counts, int64_t n_tok, float weight,
                                    float r) {
    if (!layer_ok(p, il) || !counts || n_tok <= 0) return -1;
    moert_policy & g = *p;
    const float w = std::min(1.0f, std::max(0.0f, weight));
    const float d = g.cfg.cost_rate_decay;
    for (int e = 0; e < g.E; ++e) {
        // the prompt's routes per token become the rate's steady state: rate (1 - d) = q
        const float q = std::min(1.0f, (float)counts[e] / (float)n_tok);
        float & rt = g.rate[g.at(il, e)];
        rt = (1.0f - w) * rt + w * q / (1.0f - d);
    }
    g.only_layer = il;
    g.price_override = std::max(0.0f, r);
    const long long before = g.st.refresh_promotions;
    moert_policy_refresh(p, MOERT_REFRESH_BOUNDARY);
    g.only_layer = -1;
    g.price_override = -1.0f;
    return (int32_t)(g.st.refresh_promotions - before);
}

int32_t moert_policy_can_seed(const moert_policy * p, int32_t il, int32_t e) {
    if (!layer_ok(p, il)) return 0;
    return e >= 0 && e < p->E && p->exp_slot[p->at(il, e)] < 0 ? 1 : 0;
}

int32_t moert_policy_commit_seed(moert_policy * p, int32_t il, int32_t e, int32_t slot) {
    if (!moert_policy_can_seed(p, il, e) || slot < 0 || slot >= p->cap[il]) return 0;
    moert_policy & g = *p;
    g.slot_exp[il][slot] = e;
    g.exp_slot[g.at(il, e)] = slot;
    g.slot_state[il][slot] = READY;
    set_hot(g, il, e, slot);
    g.session[g.at(il, e)] = g.recent[g.at(il, e)] = g.cfg.seed_prior;
    return 1;
}

void moert_policy_add_external_counts(moert_policy * p, int32_t il, const int32_t * counts, int64_t hot,
                                      int64_t cold) {
    if (!layer_ok(p, il) || !counts) return;
    moert_policy & g = *p;
    for (int e = 0; e < g.E; ++e) g.routes[g.at(il, e)] += (float)counts[e];
    g.st.hot_routes += hot;
    g.st.cold_routes += cold;
}

void moert_policy_reset_stats(moert_policy * p) {
    if (!p) return;
    p->st = moert_policy_stats{};   // residency and scores are kept
    p->n_samples = 0;
}

int32_t moert_policy_layer_k(const moert_policy * p, int32_t il) { return layer_ok(p, il) ? p->cap[il] : -1; }

double moert_policy_hit_rate(moert_policy * p) {
    if (!p) return 0.0;
    pull_external(p);
    const long long tot = p->st.hot_routes + p->st.cold_routes;
    return tot > 0 ? (double)p->st.hot_routes / (double)tot : 0.0;
}

void moert_policy_get_stats(moert_policy * p, moert_policy_stats * out) {
    if (!p || !out) return;
    pull_external(p);
    *out = p->st;
    out->occupancy = 0.0;
    long long ready = 0, slots = 0;
    for (int il = 0; il < p->L; ++il) {
        slots += p->cap[il];
        for (int s = 0; s < p->cap[il]; ++s) ready += p->slot_state[il][s] == READY;
    }
    if (slots > 0) out->occupancy = (double)ready / (double)slots;
}

void moert_policy_get_window(moert_policy * p, int32_t n_tokens, moert_policy_window * out) {
    if (!out) return;
    memset(out, 0, sizeof(*out));
    if (!p || n_tokens < 2) return;
    pull_external(p);
    const long long n = std::min<long long>(n_tokens, std::min<long long>(p->n_samples, moert_policy::RING));
    if (n < 2) return;
    const moert_policy::Sample & a = p->ring[(p->n_samples - n) % moert_policy::RING];
    const moert_policy::Sample & b = p->ring[(p->n_samples - 1) % moert_policy::RING];
    out->tokens = (int32_t)n;
    out->span_ms = b.t_ms - a.t_ms;
    if (out->span_ms > 0.0) {
        out->tok_per_s = 1000.0 * (double)(n - 1) / out->span_ms;
        out->ms_per_tok = out->span_ms / (double)(n - 1);
    }
    // routes from the window's first sample to now
    out->hot_routes = p->st.hot_routes - a.hot;
    out->cold_routes = p->st.cold_routes - a.cold;
    const long long tot = out->hot_routes + out->cold_routes;
    if (tot > 0) out->hit_rate = (double)out->hot_routes / (double)tot;
}

const int32_t * moert_policy_exp_slot_view(const moert_policy * p, int32_t il) {
    return layer_ok(p, il) ? p->exp_slot.data() + p->at(il, 0) : nullptr;
}
const int32_t * moert_policy_slot_exp_view(const moert_policy * p, int32_t il) {
    return layer_ok(p, il) ? p->slot_exp[il].data() : nullptr;
}
const int32_t * moert_policy_slot_state_view(const moert_policy * p, int32_t il) {
    return layer_ok(p, il) ? p->slot_state[il].data() : nullptr;
}
const int32_t * moert_policy_hotmap_view(const moert_policy * p, int32_t il) {
    return layer_ok(p, il) ? p->hotmap.data() + p->at(il, 0) : nullptr;
}
const float * moert_policy_resid_view(const moert_policy * p, int32_t il) {
    return layer_ok(p, il) ? p->resid.data() + p->at(il, 0) : nullptr;
}

// K re-fit (kfit_policy.hpp:61-94): the slot count the device can hold now.
void llapis_kfit(const llapis_kfit_inputs * in, llapis_kfit_decision * out) {
    if (!in || !out) return;
    llapis_kfit_decision d = {};
    // one pool for both regimes (a resident slab's bytes are inside free),
    // bounded by the per-process budget when there is one
    d.pool_mib = in->slab_mib_now + in->free_mib;
    if (in->headroom_mib >= 0 && in->slab_mib_now + in->headroom_mib < d.pool_mib) {
        d.pool_mib = in->slab_mib_now + in->headroom_mib;
        d.wddm_bound = 1;
    }
    const long long per_k = in->per_k_mib > 0 ? in->per_k_mib : 1;
    const long long affordable = d.pool_mib / per_k;      // physics, before the preference
    long long k = (d.pool_mib - in->keep_free_mib) / per_k;
    k = std::max<long long>(k, in->k_min);
    k = std::min<long long>(k, in->n_expert);
    if (k > affordable) {
        k = std::max<long long>(affordable, 1);
        d.floor_capped = 1;
    }
    d.k = (int32_t)k;
    // hysteresis: a one-slot change is not worth a rebuild, unless the
    // rebuild is the restore of an evicted slab
    d.rebuild = in->evicted || d.k <= in->k_cur - 2 || d.k >= in->k_cur + 2;
    if (!d.rebuild) d.k = in->k_cur;
    *out = d;
}

}  // extern "C"
