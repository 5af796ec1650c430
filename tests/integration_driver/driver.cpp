// Runs the C++ blocks of INTEGRATION.md on the GPU, as an adapter would call
// them, and checks what they produce against the oracle's C library.
// tests/integration_driver/build.py compiles every ```cpp block of
// INTEGRATION.md unchanged next to this file; tests/test_gpu_integration_driver.py
// runs the result.
//
// The history: 2 layers x 12 blocks x 128 tokens of 4 KV heads x 256, f16
// from a fixed LCG, on the device (layer-major) and in pinned host memory
// (block-major, K rows then V rows per layer).  Each part prints one line
// and the program exits 0 only if every check holds:
//   1. kvmem_write_blocks_to_gpu: three blocks from the pinned history into
//      chosen slots; every row bit-exact against ggml's q8_0 (the oracle).
//   2. kvmem_score_into_store: per-token max scores of all 12 blocks (the
//      last one partial) within 1e-3 of the oracle's fp64 scorer.
//   3. kvmem_stagein_raw_k: two blocks with NeoX RoPE 256 at their original
//      positions and the Hadamard rotation (K 256, V 64) before q8_0 / q4_0;
//      every row bit-exact against the oracle's transform and quantizers.
//   4. kvmem_meank_step (one layer): the query harvest, the key sums of the
//      full blocks, decode tokens summed into the open block and the
//      reference's mean-K scorer: scores within 1e-5 of the oracle's chain.
//   5. kvmem_engine_for_adapter + kvmem_on_qcur + kvmem_apply_retrieval +
//      kvmem_apply_selection: the engine with the mean-K scorer and the
//      Hadamard rotation; the selection equals the oracle's top-k over its
//      mean-K scores of the captured query, and every resident block's rows
//      are the oracle's rotated q8_0 rows in window order.
//   6. kvmem_query_turn: a query turn whose decode appends rows resident and
//      writes their cells; it takes the query_replay path, its selection is
//      the oracle's top-k over the grown history (partial last block), and
//      every resident block's rows are the oracle's afterwards.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "kvmem_hip.h"
#include "kvmem_host.h"
#include "kvmem_oracle.h"

// ---- the INTEGRATION.md blocks (compiled from the document itself)
bool kvmem_write_blocks_to_gpu(kvmem_hip_ctx *hctx, const std::vector<uint32_t> &ids,
                               const std::vector<uint32_t> &slots, void *const *k_layers,
                               void *const *v_layers, uint32_t n_attn, uint32_t n_slots,
                               uint32_t block_tokens, uint32_t n_embd_k, uint32_t n_embd_v,
                               const void *pinned_f16_blocks, uint32_t n_blocks,
                               uint32_t last_block_tokens);
int kvmem_score_into_store(kvmem_hip_ctx *hctx, const void *k_mirror_dev, uint32_t n_attn,
                           uint32_t n_blocks, uint32_t block_tokens, uint32_t n_embd_k,
                           uint32_t last_block_tokens, uint32_t capacity_blocks, const void *q_dev,
                           uint32_t n_q_tokens, uint32_t n_head, uint32_t n_head_kv,
                           uint32_t head_dim, float *scores_dev, std::vector<double> &scores);
int kvmem_meank_step(kvmem_hip_ctx *hctx, const float *q_rows_dev, uint32_t n_attn, uint32_t n_rows,
                     uint32_t n_head, uint32_t n_head_kv, uint32_t head_dim,
                     const std::vector<uint32_t> &query_tokens, bool first_batch, float *q_sum_dev,
                     const uint32_t *q_count, const kvmem_hip_history *kh,
                     const std::vector<uint32_t> &new_block_ids, float *k_sum_dev,
                     uint32_t *mean_tokens_dev, uint32_t n_blocks, uint32_t capacity_blocks,
                     float *scores_dev, const void *gpu_k, int32_t k_type, size_t nb0, size_t nb1,
                     size_t nb2, uint32_t tok0, uint32_t n_add, uint32_t open_block, bool first_tokens);
int kvmem_stagein_raw_k(kvmem_hip_ctx *hctx, const kvmem_hip_history *kh, kvmem_hip_pool pool,
                        const std::vector<uint32_t> &ids, const std::vector<uint32_t> &slots,
                        const std::vector<int32_t> &orig_pos_start, uint32_t head_dim, uint32_t n_rot,
                        float freq_base, float freq_scale, uint32_t nrot_k, uint32_t nrot_v);
kvmem_engine *kvmem_engine_for_adapter(uint32_t n_attn, uint32_t block_tokens, uint32_t n_head,
                                       uint32_t n_head_kv, uint32_t head_dim, uint32_t budget,
                                       uint32_t gen_reserve, uint32_t sink_blocks, int32_t type_k,
                                       int32_t type_v, uint32_t n_rot, float freq_base,
                                       void *const *k_layers, void *const *v_layers,
                                       const void *k_hist_dev, const void *v_hist_dev,
                                       uint32_t capacity_blocks, uint32_t n_tokens);
int kvmem_on_qcur(kvmem_engine *eng, uint32_t il, const void *qcur_data, int32_t qcur_type,
                  size_t nb0, size_t nb1, size_t nb2, const std::vector<int32_t> &cur_pos);
void kvmem_apply_retrieval(kvmem_engine *eng, int32_t query_begin, int32_t query_end, int32_t force_pos);
void kvmem_apply_selection(kvmem_engine *eng);
typedef void (*kvmem_decode_fn)(void *user, uint32_t begin, uint32_t end);
const char *kvmem_query_turn(kvmem_engine *eng, uint32_t query, uint32_t eval_end, uint32_t gen_rows,
                             uint32_t block_tokens, kvmem_decode_fn decode, void *user);

namespace {

constexpr uint32_t L = 2, B = 12, T = 128, HKV = 4, HQ = 24, D = 256, E = HKV * D, EQ = HQ * D;

void require(bool ok, const std::string &what) {
    if (!ok) {
        throw std::runtime_error(what);
    }
}

void hip(hipError_t e, const char *what) {
    require(e == hipSuccess, std::string(what) + ": " + hipGetErrorString(e));
}

uint64_t g_lcg = 0x9e3779b97f4a7c15ull;
float uniform() {   // [-2, 2)
    g_lcg = g_lcg * 6364136223846793005ull + 1442695040888963407ull;
    return static_cast<float>((g_lcg >> 40) & 0xffffff) / 4194304.0f - 2.0f;
}

struct DevBuf {
    void *p = nullptr;
    explicit DevBuf(size_t n) { hip(hipMalloc(&p, n), "hipMalloc"); }
    ~DevBuf() { (void) hipFree(p); }
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
};

std::vector<uint8_t> to_host(const void *dev, size_t n) {
    std::vector<uint8_t> h(n);
    hip(hipMemcpy(h.data(), dev, n, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    return h;
}

// rows [0, n) of history block b of layer l (K or V), f16 bits
const uint16_t *rows_of(const std::vector<uint16_t> &hist, uint32_t l, uint32_t b) {
    return hist.data() + (static_cast<size_t>(l) * B + b) * T * E;
}

// the oracle's pool rows for n rows of a block: f16 -> f32, RoPE at pos0,
// Hadamard of `width`, quantized to `type` (no transform: quantized from f16)
std::vector<uint8_t> want_rows(int type, const uint16_t *src, uint32_t n, uint32_t n_rot, const float *theta,
                               int32_t pos0, uint32_t width) {
    std::vector<uint8_t> out(ko_row_bytes(type, E) * n);
    if (n_rot == 0 && width == 0) {
        require(ko_quantize_rows_f16(type, src, out.data(), n, E) == 0, "oracle quantize");
        return out;
    }
    std::vector<float> x(static_cast<size_t>(n) * E);
    for (size_t i = 0; i < x.size(); ++i) {
        x[i] = ko_f16_to_f32(src[i]);
    }
    if (n_rot) {
        ko_rope_rows(x.data(), n, E, D, n_rot, theta, pos0);
    }
    if (width) {
        ko_hadamard_rows(x.data(), x.size(), width);
    }
    require(ko_quantize_rows_f32(type, x.data(), out.data(), n, E) == 0, "oracle quantize f32");
    return out;
}

// rows [slot*T, slot*T + n) of a pool tensor equal `want`
void check_rows(const void *layer, int type, uint32_t slot, uint32_t n, const std::vector<uint8_t> &want,
                const std::string &what) {
    const size_t rb = ko_row_bytes(type, E);
    std::vector<uint8_t> got(rb * n);
    hip(hipMemcpy(got.data(), static_cast<const uint8_t *>(layer) + static_cast<size_t>(slot) * T * rb, got.size(),
                  hipMemcpyDeviceToHost),
        "pool read");
    require(got == want, what + ": slot " + std::to_string(slot) + " differs from the oracle");
}

struct Pool {
    uint32_t n_slots;
    int type_k, type_v;
    std::vector<void *> k, v;
    Pool(uint32_t slots, int tk, int tv) : n_slots(slots), type_k(tk), type_v(tv) {
        for (uint32_t l = 0; l < L; ++l) {
            void *pk = nullptr, *pv = nullptr;
            hip(hipMalloc(&pk, ko_row_bytes(tk, E) * n_slots * T), "pool K");
            hip(hipMalloc(&pv, ko_row_bytes(tv, E) * n_slots * T), "pool V");
            hip(hipMemset(pk, 0, ko_row_bytes(tk, E) * n_slots * T), "pool K clear");
            hip(hipMemset(pv, 0, ko_row_bytes(tv, E) * n_slots * T), "pool V clear");
            k.push_back(pk);
            v.push_back(pv);
        }
    }
    ~Pool() {
        for (void *p : k) (void) hipFree(p);
        for (void *p : v) (void) hipFree(p);
    }
    void check(uint32_t l, bool is_v, uint32_t slot, uint32_t n, const std::vector<uint8_t> &want,
               const std::string &what) const {
        check_rows(is_v ? v[l] : k[l], is_v ? type_v : type_k, slot, n, want,
                   what + ": layer " + std::to_string(l) + (is_v ? " V" : " K"));
    }
};

struct World {
    std::vector<uint16_t> k, v;              // [L][B][T][E] f16
    void *k_dev = nullptr, *v_dev = nullptr;
    void *pinned = nullptr;                  // [B][L][K rows, V rows] f16
    World() : k(static_cast<size_t>(L) * B * T * E), v(k.size()) {
        for (auto &x : k) x = ko_f32_to_f16(uniform());
        for (auto &x : v) x = ko_f32_to_f16(uniform());
        hip(hipMalloc(&k_dev, k.size() * 2), "history K");
        hip(hipMalloc(&v_dev, v.size() * 2), "history V");
        hip(hipMemcpy(k_dev, k.data(), k.size() * 2, hipMemcpyHostToDevice), "history K copy");
        hip(hipMemcpy(v_dev, v.data(), v.size() * 2, hipMemcpyHostToDevice), "history V copy");
        hip(hipHostMalloc(&pinned, k.size() * 4, hipHostMallocDefault), "pinned history");
        uint16_t *p = static_cast<uint16_t *>(pinned);
        for (uint32_t b = 0; b < B; ++b) {
            for (uint32_t l = 0; l < L; ++l) {
                std::memcpy(p, rows_of(k, l, b), static_cast<size_t>(T) * E * 2);
                p += static_cast<size_t>(T) * E;
                std::memcpy(p, rows_of(v, l, b), static_cast<size_t>(T) * E * 2);
                p += static_cast<size_t>(T) * E;
            }
        }
    }
    ~World() {
        (void) hipFree(k_dev);
        (void) hipFree(v_dev);
        (void) hipHostFree(pinned);
    }
};

// bf16 query rows [L][n][HQ][D]: the bits and their exact f32 image
struct Query {
    std::vector<uint16_t> bits;
    std::vector<float> f32;
    explicit Query(size_t n) : bits(n), f32(n) {
        for (size_t i = 0; i < n; ++i) {
            float x = uniform();
            uint32_t u;
            std::memcpy(&u, &x, 4);
            bits[i] = static_cast<uint16_t>(u >> 16);
            f32[i] = ko_bf16_to_f32(bits[i]);
        }
    }
};

void part1_write_blocks(kvmem_hip_ctx *ctx, const World &w) {
    Pool pool(8, KO_TYPE_Q8_0, KO_TYPE_Q8_0);
    const std::vector<uint32_t> ids = {1, 4, 7}, slots = {5, 0, 3};
    require(kvmem_write_blocks_to_gpu(ctx, ids, slots, pool.k.data(), pool.v.data(), L, 8, T, E, E, w.pinned, B, 0),
            "kvmem_write_blocks_to_gpu failed");
    for (size_t i = 0; i < ids.size(); ++i) {
        for (uint32_t l = 0; l < L; ++l) {
            pool.check(l, false, slots[i], T, want_rows(KO_TYPE_Q8_0, rows_of(w.k, l, ids[i]), T, 0, nullptr, 0, 0),
                       "write_blocks");
            pool.check(l, true, slots[i], T, want_rows(KO_TYPE_Q8_0, rows_of(w.v, l, ids[i]), T, 0, nullptr, 0, 0),
                       "write_blocks");
        }
    }
    std::printf("[driver] kvmem_write_blocks_to_gpu: 3 blocks x %u layers bit-exact\n", L);
}

void part2_score(kvmem_hip_ctx *ctx, const World &w) {
    const uint32_t tq = 8, last = 77;
    Query q(static_cast<size_t>(L) * tq * EQ);
    DevBuf qd(q.bits.size() * 2), sd(B * sizeof(float));
    hip(hipMemcpy(qd.p, q.bits.data(), q.bits.size() * 2, hipMemcpyHostToDevice), "query copy");
    std::vector<double> scores;
    require(kvmem_score_into_store(ctx, w.k_dev, L, B, T, E, last, B, qd.p, tq, HQ, HKV, D,
                                   static_cast<float *>(sd.p), scores) == KVMEM_HIP_OK,
            "kvmem_score_into_store failed");
    std::vector<double> ls(static_cast<size_t>(L) * B), want(B);
    ko_score_pertoken_max(q.f32.data(), w.k.data(), L, tq, HQ, HKV, D, B, T, last, nullptr, 0, ls.data());
    ko_combine_layers(ls.data(), L, B, 0, want.data());
    require(scores.size() == B, "score count");
    for (uint32_t b = 0; b < B; ++b) {
        const double err = std::fabs(scores[b] - want[b]) / std::fmax(std::fabs(want[b]), 1e-6);
        require(err <= 1e-3, "kvmem_score_into_store: block " + std::to_string(b) + " off by " + std::to_string(err));
    }
    std::printf("[driver] kvmem_score_into_store: %u blocks within 1e-3 of the fp64 oracle\n", B);
}

void part3_raw_k(kvmem_hip_ctx *ctx, const World &w) {
    Pool pool(8, KO_TYPE_Q8_0, KO_TYPE_Q4_0);
    kvmem_hip_history kh = {w.k_dev, w.v_dev, L, B, T, E, E, 0, B};
    kvmem_hip_pool pd = {L, 8, T, E, E, KVMEM_TYPE_Q8_0, KVMEM_TYPE_Q4_0, pool.k.data(), pool.v.data(), nullptr};
    const std::vector<uint32_t> ids = {2, 9}, slots = {6, 1};
    const std::vector<int32_t> pos = {2 * static_cast<int32_t>(T), 9 * static_cast<int32_t>(T)};
    const uint32_t n_rot = 256;
    const float base = 1e6f;
    require(kvmem_stagein_raw_k(ctx, &kh, pd, ids, slots, pos, D, n_rot, base, 1.0f, 256, 64) == KVMEM_HIP_OK,
            "kvmem_stagein_raw_k failed");
    hip(hipDeviceSynchronize(), "sync");
    std::vector<float> theta(n_rot / 2);   // rope.cpp:20-23, as the block forms it
    for (uint32_t i = 0; i < n_rot / 2; ++i) {
        theta[i] = powf(base, -2.0f * static_cast<float>(i) / static_cast<float>(n_rot));
    }
    for (size_t i = 0; i < ids.size(); ++i) {
        for (uint32_t l = 0; l < L; ++l) {
            pool.check(l, false, slots[i], T,
                       want_rows(KO_TYPE_Q8_0, rows_of(w.k, l, ids[i]), T, n_rot, theta.data(), pos[i], 256),
                       "stagein_raw_k");
            pool.check(l, true, slots[i], T, want_rows(KO_TYPE_Q4_0, rows_of(w.v, l, ids[i]), T, 0, nullptr, 0, 64),
                       "stagein_raw_k");
        }
    }
    std::printf("[driver] kvmem_stagein_raw_k: RoPE 256 + Hadamard 256 / 64, 2 blocks bit-exact\n");
}

void part4_meank(kvmem_hip_ctx *ctx, const World &w) {
    // one layer: the history's layer 0
    const uint32_t n_rows = 10, n_full = 10, open = 10, n_add = 50, nb = 11;
    const std::vector<uint32_t> tokens = {2, 3, 4, 5, 6, 7};
    std::vector<float> qrows(static_cast<size_t>(n_rows) * EQ);
    for (auto &x : qrows) x = uniform();
    DevBuf qd(qrows.size() * 4), qsum(EQ * 4), ksum(static_cast<size_t>(B) * E * 4), mt(B * 4), sd(nb * 4);
    hip(hipMemcpy(qd.p, qrows.data(), qrows.size() * 4, hipMemcpyHostToDevice), "rows copy");
    const uint32_t q_count = static_cast<uint32_t>(tokens.size());
    kvmem_hip_history kh = {w.k_dev, nullptr, 1, nb, T, E, 0, 0, B};
    std::vector<uint32_t> full;
    for (uint32_t b = 0; b < n_full; ++b) full.push_back(b);
    const uint8_t *open_rows = static_cast<const uint8_t *>(w.k_dev) + static_cast<size_t>(open) * T * E * 2;
    require(kvmem_meank_step(ctx, static_cast<const float *>(qd.p), 1, n_rows, HQ, HKV, D, tokens, true,
                             static_cast<float *>(qsum.p), &q_count, &kh, full, static_cast<float *>(ksum.p),
                             static_cast<uint32_t *>(mt.p), nb, B, static_cast<float *>(sd.p), open_rows,
                             KVMEM_TYPE_F16, 2, D * 2, E * 2, 0, n_add, open, true) == KVMEM_HIP_OK,
            "kvmem_meank_step failed");
    hip(hipDeviceSynchronize(), "sync");
    std::vector<float> want_q(EQ);
    ko_q_accumulate(qrows.data(), 1, n_rows, EQ, tokens.data(), q_count, 1, want_q.data());
    std::vector<float> want_k(static_cast<size_t>(nb) * E);
    std::vector<uint32_t> want_mt(nb);
    for (uint32_t b = 0; b < nb; ++b) {
        want_mt[b] = b < n_full ? T : n_add;
        ko_meank_sum_f16(rows_of(w.k, 0, b), want_mt[b], E, E, want_k.data() + static_cast<size_t>(b) * E);
    }
    std::vector<double> want(nb);
    ko_score_meank(want_q.data(), &q_count, want_k.data(), want_mt.data(), 1, nb, HQ, HKV, D, want.data());
    std::vector<uint8_t> got = to_host(sd.p, nb * 4);
    for (uint32_t b = 0; b < nb; ++b) {
        float s;
        std::memcpy(&s, got.data() + b * 4, 4);
        require(std::fabs(s - want[b]) <= 1e-5, "kvmem_meank_step: block " + std::to_string(b));
    }
    std::printf("[driver] kvmem_meank_step: harvest, key sums, decode sums, mean-K scores within 1e-5\n");
}

// the oracle's mean-K selection over the captured query rows (engine
// parameters of kvmem_engine_for_adapter: sink 1, recent 0, higher-id ties)
std::vector<uint32_t> oracle_meank_topk(const World &w, const Query &q, uint32_t tq, uint32_t total,
                                        uint32_t budget, const std::vector<uint32_t> &mandatory) {
    const uint32_t nb = (total + T - 1) / T;
    std::vector<float> q_sum(static_cast<size_t>(L) * EQ);
    ko_q_accumulate(q.f32.data(), L, tq, EQ, nullptr, tq, 1, q_sum.data());
    std::vector<float> k_sum(static_cast<size_t>(L) * nb * E);
    std::vector<uint32_t> mt(static_cast<size_t>(L) * nb);
    for (uint32_t l = 0; l < L; ++l) {
        for (uint32_t b = 0; b < nb; ++b) {
            mt[l * nb + b] = std::min(T, total - b * T);
            ko_meank_sum_f16(rows_of(w.k, l, b), mt[l * nb + b], E, E,
                             k_sum.data() + (static_cast<size_t>(l) * nb + b) * E);
        }
    }
    const std::vector<uint32_t> counts(L, tq);
    std::vector<double> s(nb);
    ko_score_meank(q_sum.data(), counts.data(), k_sum.data(), mt.data(), L, nb, HQ, HKV, D, s.data());
    for (auto &x : s) x = static_cast<double>(static_cast<float>(x));   // the device's f32 scores
    std::vector<uint32_t> out(nb);
    uint32_t n = 0;
    ko_pick_topk(s.data(), nb, budget, 1, 0, mandatory.data(), static_cast<uint32_t>(mandatory.size()), 0,
                 out.data(), &n);
    out.resize(n);
    return out;
}

// every block holding a slot carries the oracle's rotated q8_0 rows (its
// history rows so far, Hadamard 256 on K and 64 on V, no RoPE)
void check_engine_pool(kvmem_engine *eng, const World &w, const std::string &what) {
    const uint32_t nb = kvmem_engine_block_count(eng), total = kvmem_engine_total_tokens(eng);
    std::vector<int32_t> slots(nb);
    require(kvmem_engine_block_slots(eng, slots.data()) == KVMEM_HIP_OK, "block_slots");
    for (uint32_t l = 0; l < L; ++l) {
        void *pk = nullptr, *pv = nullptr;
        require(kvmem_engine_pool_layer(eng, l, &pk, &pv) == KVMEM_HIP_OK, "pool_layer");
        for (uint32_t b = 0; b < nb; ++b) {
            if (slots[b] < 0) continue;
            const uint32_t n = std::min(T, total - b * T);
            const std::string at = what + ": layer " + std::to_string(l) + " block " + std::to_string(b);
            check_rows(pk, KO_TYPE_Q8_0, static_cast<uint32_t>(slots[b]), n,
                       want_rows(KO_TYPE_Q8_0, rows_of(w.k, l, b), n, 0, nullptr, 0, 256), at + " K");
            check_rows(pv, KO_TYPE_Q8_0, static_cast<uint32_t>(slots[b]), n,
                       want_rows(KO_TYPE_Q8_0, rows_of(w.v, l, b), n, 0, nullptr, 0, 64), at + " V");
        }
    }
}

struct Decode {
    kvmem_engine *eng;
    const World *w;
    int calls = 0;
};

// the caller's decode: rows appended resident, then the cells of the blocks they
// touch written from the history (whole blocks, rotated q8_0 as the cache holds them)
void decode_rows(void *user, uint32_t begin, uint32_t end) {
    Decode &d = *static_cast<Decode *>(user);
    ++d.calls;
    require(kvmem_engine_append_resident(d.eng, end - begin) == KVMEM_HIP_OK,
            std::string("append_resident: ") + kvmem_engine_last_error(d.eng));
    const uint32_t nb = kvmem_engine_block_count(d.eng);
    std::vector<int32_t> slots(nb);
    require(kvmem_engine_block_slots(d.eng, slots.data()) == KVMEM_HIP_OK, "block_slots");
    std::vector<uint32_t> ids, sl;
    for (uint32_t b = begin / T; b < (end + T - 1) / T; ++b) {
        require(slots[b] >= 0, "a decoded block has no slot");
        ids.push_back(b);
        sl.push_back(static_cast<uint32_t>(slots[b]));
    }
    std::vector<void *> pk(L), pv(L);
    for (uint32_t l = 0; l < L; ++l) {
        require(kvmem_engine_pool_layer(d.eng, l, &pk[l], &pv[l]) == KVMEM_HIP_OK, "pool_layer");
    }
    const uint32_t total = kvmem_engine_total_tokens(d.eng);
    const uint32_t last = total - (nb - 1) * T;
    kvmem_hip_history kh = {d.w->k_dev, d.w->v_dev, L, nb, T, E, E, last == T ? 0 : last, B};
    kvmem_hip_transform xf = {D, 0, nullptr, 256, 64, nullptr};
    kvmem_hip_pool pool = {L, kvmem_engine_n_slots(d.eng), T, E, E, KVMEM_TYPE_Q8_0, KVMEM_TYPE_Q8_0,
                           pk.data(), pv.data(), &xf};
    kvmem_hip_ctx *ctx = kvmem_engine_ctx(d.eng);
    require(kvmem_hip_stagein_blocks(ctx, &kh, &pool, ids.data(), sl.data(), static_cast<uint32_t>(ids.size())) ==
                    KVMEM_HIP_OK &&
                kvmem_hip_sync(ctx) == KVMEM_HIP_OK,
            std::string("decode cells: ") + kvmem_hip_last_error(ctx));
}

// the blocks holding a slot, checked to sit in slots 0, 1, ... in block order
std::vector<uint32_t> resident_in_window_order(kvmem_engine *eng, const std::string &what) {
    std::vector<int32_t> slots(kvmem_engine_block_count(eng));
    require(kvmem_engine_block_slots(eng, slots.data()) == KVMEM_HIP_OK, "block_slots");
    std::vector<uint32_t> res;
    for (uint32_t b = 0; b < slots.size(); ++b) {
        if (slots[b] >= 0) {
            require(slots[b] == static_cast<int32_t>(res.size()), what + ": not in window order");
            res.push_back(b);
        }
    }
    return res;
}

// kvmem_engine_retrieval_mandatory, sorted
std::vector<uint32_t> mandatory_of(kvmem_engine *eng) {
    std::vector<uint32_t> out(kvmem_engine_block_count(eng));
    uint32_t n = 0;
    require(kvmem_engine_retrieval_mandatory(eng, out.data(), static_cast<uint32_t>(out.size()), &n) ==
                KVMEM_HIP_OK,
            "retrieval_mandatory");
    out.resize(n);
    std::sort(out.begin(), out.end());
    return out;
}

void part5_engine(const World &w) {
    Pool pool(8, KO_TYPE_Q8_0, KO_TYPE_Q8_0);
    const uint32_t n_tok = 10 * T;
    kvmem_engine *eng = kvmem_engine_for_adapter(L, T, HQ, HKV, D, 5 * T, 3 * T, 1, KVMEM_TYPE_Q8_0, KVMEM_TYPE_Q8_0,
                                                 0, 1e4f, pool.k.data(), pool.v.data(), w.k_dev, w.v_dev, B, n_tok);
    require(eng != nullptr, "kvmem_engine_for_adapter failed");
    // a 16-token query ubatch at rows 1200..1215 of every layer, captured from a Qcur view
    const uint32_t tq = 16;
    Query q(static_cast<size_t>(L) * tq * EQ);
    DevBuf qd(q.bits.size() * 2);
    hip(hipMemcpy(qd.p, q.bits.data(), q.bits.size() * 2, hipMemcpyHostToDevice), "qcur copy");
    std::vector<int32_t> pos;
    for (uint32_t t = 0; t < tq; ++t) pos.push_back(static_cast<int32_t>(1200 + t));
    kvmem_engine_set_request_span(eng, 1200, 0, -1);   // the captured rows are the query
    for (uint32_t l = 0; l < L; ++l) {
        const uint8_t *layer = static_cast<const uint8_t *>(qd.p) + static_cast<size_t>(l) * tq * EQ * 2;
        require(kvmem_on_qcur(eng, l, layer, KVMEM_TYPE_BF16, 2, D * 2, EQ * 2, pos) == KVMEM_HIP_OK,
                "kvmem_on_qcur failed");
    }
    kvmem_apply_retrieval(eng, 1200, 0, 0);   // the span's block 9 and force_pos 0's block 0 are mandatory
    const std::vector<uint32_t> res = resident_in_window_order(eng, "kvmem_apply_retrieval");
    require(mandatory_of(eng) == std::vector<uint32_t>({0, 9}), "retrieval_mandatory: expected blocks 0 and 9");
    require(res == oracle_meank_topk(w, q, tq, n_tok, 5, {9, 0}),
            "kvmem_apply_retrieval: the selection differs from the oracle's mean-K top-k");
    check_engine_pool(eng, w, "apply_retrieval");
    kvmem_apply_selection(eng);   // the same query: the same selection, applied through preview + apply
    check_engine_pool(eng, w, "apply_selection");
    std::printf("[driver] kvmem_engine_for_adapter + kvmem_on_qcur + kvmem_apply_retrieval + "
                "kvmem_apply_selection: selection = oracle mean-K top-%zu, pool bit-exact\n", res.size());

    // One query turn over rows [1280, 1400) with 64 generation rows.  The whole
    // history (11 blocks) does not fit the 8 slots, so it is not all_resident;
    // the span now ends at row 1400, so blocks 0, 9 and 10 are mandatory and the
    // view of 5 blocks before the turn cannot be kept unchanged; the new
    // selection of 5 blocks (block 10 among them) plus block 11 for the
    // generation rows fits the pool: the query is replayed.
    Decode d{eng, &w};
    const char *path = kvmem_query_turn(eng, n_tok, n_tok + 120, 64, T, decode_rows, &d);
    require(d.calls == 1, "kvmem_query_turn: the decode ran " + std::to_string(d.calls) + " times");
    require(std::string(path) == "query_replay", std::string("kvmem_query_turn: path ") + path);
    require(mandatory_of(eng) == std::vector<uint32_t>({0, 9, 10}), "retrieval_mandatory: expected 0, 9, 10");
    require(resident_in_window_order(eng, "kvmem_query_turn") ==
                oracle_meank_topk(w, q, tq, n_tok + 120, 5, {9, 10, 0}),
            "kvmem_query_turn: the selection differs from the oracle's mean-K top-k");
    check_engine_pool(eng, w, "query_turn");
    std::printf("[driver] kvmem_query_turn: path %s, pool bit-exact\n", path);
    kvmem_engine_destroy(eng);
}

}  // namespace

int main() {
    try {
        World w;
        kvmem_hip_ctx *ctx = nullptr;
        require(kvmem_hip_create(0, &ctx) == KVMEM_HIP_OK, "kvmem_hip_create");
        part1_write_blocks(ctx, w);
        part2_score(ctx, w);
        part3_raw_k(ctx, w);
        part4_meank(ctx, w);
        kvmem_hip_destroy(ctx);
        part5_engine(w);
    } catch (const std::exception &ex) {
        std::printf("[driver] FAILED: %s\n", ex.what());
        return 1;
    }
    std::printf("[driver] ok\n");
    return 0;
}
