// prefill.hip - dense chunked prefill on MFMA for gfx950.
//
// Computes rows [q_offset, q_offset + len) of causal (or full) attention for one
// or more sequence chunks whose first q_offset tokens are already in the paged
// pool (kernels.metal:693-917 semantics: scale 1/sqrt(d), GQA head h reads kv
// head h / G, a fixed window start max(0, kv_len - W) for every row).
//
// Head sizes 64 and 128 (f16 or e4m3 pools); the layouts are in prefill_body.h.
// Matrix work runs on v_mfma_f32_32x32x16_f16, which on gfx950 retires twice
// the flops per cycle of the 16x16 shapes.  A workgroup (8 waves, two per SIMD)
// owns 256 query rows of one kv head: the (token, head) pairs of 256 / G
// consecutive tokens, so the G query heads sharing a kv head share every K/V
// tile.  Each wave owns RB blocks of 32 rows (RB = 2 would halve the LDS
// traffic but needs AGPR accumulators and one wave per SIMD, measured slower).
// Per 32-key tile t a wave runs two phases separated by workgroup barriers:
//   * matrix phase M_t: S^T(t+1) = K Q^T (32 keys x 32 rows, 8 MFMAs over d; K
//     from LDS is the A operand, Q^T stays in registers as B) and
//     O^T += V^T(t) P^T(t) (8 MFMAs; V^T read with the transposing
//     ds_read_b64_tr_b16), then the global loads of tile t + 4;
//   * vector phase V_t: mask and reference max of S(t), exponentials to P(t) in
//     f16, row sums, the K operands of M_t and the LDS staging of tile t + 2.
//   The S^T accumulator leaves lane (n, h) holding keys 8q + 4h + r (q, r < 4) of
//   row n, and the 8 of them with q in {2c, 2c+1} are exactly the B operand of
//   O^T += V^T P^T over key chunk c (16 keys), so P never leaves registers.
//   Waves 4-7 run one phase behind waves 0-3; waves w and w + 4 share a SIMD,
//   so its MFMA pipe works on one wave's matrix phase while the other wave's
//   vector phase runs.
// A workgroup runs the segments the host's work list gives it (one item, or
// pieces of items whose partial states are merged by the last workgroup to
// finish one; prefill_split_plan below).
// Softmax keeps a per-row reference max that is only raised (and O rescaled)
// when some score exceeds it by more than 2^8, so P is bounded by 2^8 and goes
// to the MFMA in f16; the common case needs no cross-lane reduction.
#include <algorithm>
#include <functional>

#include "prefill_body.h"

namespace pam {

// The kernel (the fat binary's entry); prefill_body also backs the named
// entries of the code object (module_entry.hip).
template <int HD, int RB, bool FUSED, typename KV>
__global__ __launch_bounds__(64 * kPrefillWaves, 1) void prefill_mfma_kernel(AttnParams p) {
    prefill_body<HD, RB, FUSED, KV>(p);
}

bool prefill_mfma_supported(int32_t dtype, int32_t head_dim, int32_t group, int32_t block_size) {
    return (dtype == kF16 || dtype == kFP8) && (head_dim == 128 || head_dim == 64) && group >= 1 && group <= 32 &&
           (kPrefillRows % group) == 0 && block_size > 0 && (block_size & (block_size - 1)) == 0;
}

hipError_t launch_prefill_mfma(const AttnParams &p_in, int32_t dtype, hipStream_t stream, const KernelTable *kt) {
    AttnParams p = p_in;
    p.epoch = next_launch_epoch();
    if (p.pf_work == nullptr || p.pf_range == nullptr || p.pf_groups <= 0) return hipErrorInvalidValue;
    const int G = p.num_heads / p.num_kv_heads;
    if (!prefill_mfma_supported(dtype, p.head_dim, G, p.block_size)) return hipErrorInvalidValue;
    const dim3 grid(p.pf_groups), block(64 * kPrefillWaves);
    if (dtype == kFP8 && (p.fuse_k != nullptr || p.k_scale == nullptr || p.v_scale == nullptr))
        return hipErrorInvalidValue;
    hipError_t e;  // the code object's entry of this configuration, when it has one
    hipFunction_t f =
        kt ? kt->prefill[p.head_dim == 64 ? 1 : 0][dtype == kFP8 ? 2 : (p.fuse_k != nullptr ? 1 : 0)] : nullptr;
    if (via_module(kt, f, &e, grid, block, stream, p)) return e;
    if (p.head_dim == 64) {
        if (dtype == kFP8)
            hipLaunchKernelGGL((prefill_mfma_kernel<64, kPrefillRB, false, uint8_t>), grid, block, 0, stream, p);
        else if (p.fuse_k != nullptr)
            hipLaunchKernelGGL((prefill_mfma_kernel<64, kPrefillRB, true, f16>), grid, block, 0, stream, p);
        else
            hipLaunchKernelGGL((prefill_mfma_kernel<64, kPrefillRB, false, f16>), grid, block, 0, stream, p);
    } else if (dtype == kFP8) {
        hipLaunchKernelGGL((prefill_mfma_kernel<128, kPrefillRB, false, uint8_t>), grid, block, 0, stream, p);
    } else if (p.fuse_k != nullptr) {
        hipLaunchKernelGGL((prefill_mfma_kernel<128, kPrefillRB, true, f16>), grid, block, 0, stream, p);
    } else {
        hipLaunchKernelGGL((prefill_mfma_kernel<128, kPrefillRB, false, f16>), grid, block, 0, stream, p);
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------ host plan
//
// Three schedules, chosen by estimated makespan (costs in key tiles: a segment
// costs its tiles plus kSegCost for the Q load, block-table segment, ring fill,
// masked edge tiles and output; a piece of a split item kSplitCost more for
// publishing and merging partials; both measured per workgroup with s_memtime
// on gfx950):
//  * grid order: one item per workgroup, hardware-dispatched (see below);
//  * static grid: the same items and XCDs, dealt ahead of the launch to one
//    workgroup per CU, each running its items back to back (see below);
//  * balanced split, one workgroup per CU: items are laid out group by group
//    (chunk, kv head), token blocks in order, and workgroups are filled in line
//    order up to a common capacity, the smallest with which the line fits
//    `groups` workgroups.  An item that does not fit is cut into pieces of an
//    even number of tiles (>= kMinPiece; the tile loop runs pairs).  Consecutive
//    parts of the line go to workgroups of one XCD (workgroup b runs on XCD
//    b mod 8), so a group's pieces share its L2.
namespace {
constexpr int kSegCost = 12;
constexpr int kSplitCost = 4;
constexpr int kMinPiece = 8;
constexpr int kPrefetchCost = 4;  // start-up tiles an item saves when its descriptors were prefetched
static_assert(kSegCost > kPrefetchCost, "every item costs more than its prefetch credit");

// the paired deal is taken when its estimate is at most this times the others'
constexpr double kPairedSlack = 1.0;

struct PfItem {
    int4 chunk;
    int32_t kvh, tok0, t_lo, t_hi;
};

// Fills the line at capacity `cap`.  Returns the workgroups used; without `out`
// it stops at groups + 1 once the line does not fit.
int32_t pf_fill(const std::vector<PfItem> &items, int64_t cap, int32_t groups, PrefillSplit *out,
                std::vector<int32_t> *part_first) {
    int32_t wg = 0;
    int64_t budget = cap;
    bool used = false;  // workgroup wg has a segment
    for (const PfItem &it : items) {
        const int32_t n = it.t_hi - it.t_lo;
        int32_t done = 0, pieces = 0;
        const size_t first_seg = out ? out->work.size() / 3 : 0;
        for (;;) {
            const int32_t r = n - done;
            const bool whole_fits = r <= budget - kSegCost - (pieces ? kSplitCost : 0);
            if (used && !whole_fits && budget - kSegCost - kSplitCost < kMinPiece) {  // next workgroup
                wg++;
                budget = cap;
                used = false;
                if (!out && wg >= groups) return groups + 1;
            }
            int32_t take = r;
            int64_t cost = kSegCost + r + (pieces ? kSplitCost : 0);
            if (cost > budget) {
                int64_t a = (budget - kSegCost - kSplitCost) & ~(int64_t)1;
                if (r - a < kMinPiece) a = (r - kMinPiece) & ~1;
                if (a >= kMinPiece) {
                    take = (int32_t)a;
                    cost = kSegCost + kSplitCost + a;
                }  // else the whole rest, over capacity
            }
            if (!used && part_first) (*part_first)[wg] = (int32_t)(first_seg + pieces);
            if (out) {
                out->work.push_back(it.chunk);
                out->work.push_back(make_int4(it.kvh, it.tok0, it.t_lo + done, it.t_lo + done + take));
                out->work.push_back(make_int4(0, pieces, 1, 0));
            }
            used = true;
            budget -= cost;
            done += take;
            pieces++;
            if (done >= n) break;
            wg++;
            budget = cap;
            used = false;
            if (!out && wg >= groups) return groups + 1;
        }
        if (out && pieces > 1) {
            for (int32_t k = 0; k < pieces; k++) {
                int4 &b = out->work[3 * (first_seg + k) + 2];
                b.x = (int32_t)out->slots;
                b.z = pieces;
            }
            out->slots += pieces;
        }
    }
    return wg + (used ? 1 : 0);
}
}  // namespace

void prefill_split_plan(const int4 *chunks, int32_t n, AttnParams &p, int32_t groups, PrefillSplit &out,
                        bool allow_split) {
    constexpr int KT = kPrefillKT;
    const int32_t G = p.num_heads / p.num_kv_heads, tpw = kPrefillRows / G;
    std::vector<PfItem> items;
    int64_t n_items = 0;
    for (int32_t c = 0; c < n; c++) n_items += (int64_t)p.num_kv_heads * ((chunks[c].z + tpw - 1) / tpw);
    items.reserve(n_items);
    int64_t total = 0;
    for (int32_t c = 0; c < n; c++) {
        const int4 ch = chunks[c];
        const int32_t kv_len = ch.y + ch.z;
        const int32_t ws = p.window > 0 ? std::max(0, kv_len - p.window) : 0;
        for (int32_t kvh = 0; kvh < p.num_kv_heads; kvh++)
            for (int32_t tok0 = 0; tok0 < ch.z; tok0 += tpw) {
                const int32_t tok_end = std::min(tok0 + tpw, ch.z);
                const int32_t key_end = p.causal ? ch.y + tok_end : kv_len;
                const int32_t t_lo = ws / KT, t_hi = std::max(t_lo, (key_end + KT - 1) / KT);
                items.push_back({ch, kvh, tok0, t_lo, t_hi});
                total += t_hi - t_lo + kSegCost;
            }
    }
    groups = std::max<int32_t>(1, groups);
    out.work.clear();
    out.range.clear();
    out.slots = 0;

    // Grid order: one item per workgroup, dispatched by the hardware in id
    // order as CUs free up.  All token blocks of one (chunk, kv head) get ids of
    // one residue mod 8, so they run side by side on one XCD and its L2 serves
    // their shared K/V; longest chunks first, the heaviest token blocks of a
    // group first.  Its makespan is estimated by list scheduling on `groups` CUs.
    std::vector<int32_t> order(n);
    for (int32_t c = 0; c < n; c++) order[c] = c;
    std::stable_sort(order.begin(), order.end(), [&](int32_t a, int32_t b) {
        return chunks[a].y + chunks[a].z > chunks[b].y + chunks[b].z;
    });
    int32_t nx = 0;
    for (int32_t c = 0; c < n; c++) nx = std::max(nx, (chunks[c].z + tpw - 1) / tpw);
    const int64_t ngroups = (int64_t)n * p.num_kv_heads;
    const int64_t grid_ids = (int64_t)kXcds * nx * ((ngroups + kXcds - 1) / kXcds);
    // item index of (chunk c, kv head, token block) in `items`
    std::vector<int64_t> item_base(n + 1, 0);
    for (int32_t c = 0; c < n; c++)
        item_base[c + 1] = item_base[c] + (int64_t)p.num_kv_heads * ((chunks[c].z + tpw - 1) / tpw);
    std::vector<int64_t> grid_item(grid_ids, -1);
    for (int64_t b = 0; b < grid_ids; b++) {
        const int64_t xcd = b % kXcds, r = b / kXcds;
        const int64_t grp = xcd + kXcds * (r / nx);
        if (grp >= ngroups) continue;
        const int32_t c = order[grp / p.num_kv_heads], kvh = (int32_t)(grp % p.num_kv_heads);
        const int32_t nb = (chunks[c].z + tpw - 1) / tpw, tb = nx - 1 - (int32_t)(r % nx);
        if (tb < nb) grid_item[b] = item_base[c] + (int64_t)kvh * nb + tb;
    }
    // The grid order's makespan by list scheduling, run only when it can
    // matter: it is at least grid_lb (the mean load, and the longest item), so
    // a static deal below that bound is taken without it.
    int64_t grid_lb = (total + groups - 1) / groups;
    for (const PfItem &it : items) grid_lb = std::max<int64_t>(grid_lb, it.t_hi - it.t_lo + kSegCost);
    auto grid_estimate = [&]() {
        int64_t makespan = 0;
        // each CU's finish time, a binary min-heap (all 0 to start)
        std::vector<int64_t> cu(groups, 0);
        for (int64_t b = 0; b < grid_ids; b++) {
            const int64_t it = grid_item[b];
            if (it < 0) continue;
            const int64_t t = cu[0] + items[it].t_hi - items[it].t_lo + kSegCost;
            makespan = std::max(makespan, t);
            for (int32_t i = 0;;) {  // the earliest CU takes it: sift its new time down
                const int32_t l = 2 * i + 1, r = l + 1;
                int32_t m = l < groups && cu[l] < t ? l : -1;
                if (r < groups && cu[r] < t && cu[r] < cu[l]) m = r;
                if (m < 0) {
                    cu[i] = t;
                    break;
                }
                cu[i] = cu[m];
                i = m;
            }
        }
        return makespan;
    };

    // Static grid: the grid order's items, each on the same XCD as there (all
    // token blocks of one (chunk, kv head) share that XCD's L2), dealt to the
    // XCD's workgroups, each item onto the least-loaded one (workgroup b runs
    // on XCD b mod 8).  A workgroup runs its items in the order dealt and
    // requests the next item's descriptors and first block-table entries while
    // the current one runs, so only its first item waits for them: the
    // estimate credits kPrefetchCost tiles for each later item.  Two deal
    // orders are planned:
    //  * grid order (longest chunks first, a group's token blocks side by side):
    //    the hardware's dispatch planned ahead;
    //  * longest item first: better balance when items differ in length, but a
    //    group's blocks end up apart and lose their shared L2 (measured 12%
    //    slower on 64 chunks of one context length), so it is taken only when
    //    its estimate is at least 1% shorter.
    // the chosen deal's items, workgroup by workgroup in the order dealt:
    // workgroup b's are static_items[static_off[b] .. static_off[b + 1])
    std::vector<int64_t> static_items;
    std::vector<int32_t> static_off;
    int64_t static_makespan = INT64_MAX;
    if (groups % kXcds == 0 && grid_ids <= INT32_MAX) {
        const int32_t per_xcd = groups / kXcds;
        std::vector<std::vector<int64_t>> by_xcd(kXcds);
        for (int64_t b = 0; b < grid_ids; b++)
            if (grid_item[b] >= 0) by_xcd[b % kXcds].push_back(grid_item[b]);
        std::vector<int64_t> icost(items.size());
        for (size_t i = 0; i < items.size(); i++) icost[i] = (int64_t)items[i].t_hi - items[i].t_lo + kSegCost;
        // The deals below return their estimated makespan; with `trace` they
        // also record each (workgroup, item) in the order dealt (workgroup i of
        // XCD x is i * 8 + x).
        // A deal onto the least-loaded workgroup takes the lowest index among
        // equals.
        std::vector<int64_t> load(groups);
        std::vector<int32_t> cnt(groups);
        // A deal runs XCD by XCD on contiguous copies of the XCD's loads and
        // counts (xl, xc: entry i is workgroup i * 8 + x), its workgroups in a
        // binary min-heap on (load, workgroup)
        std::vector<int64_t> xl(per_xcd);
        std::vector<int32_t> xc(per_xcd), heap(per_xcd);
        auto before = [&](int32_t a, int32_t b) { return xl[a] < xl[b] || (xl[a] == xl[b] && a < b); };
        auto heap_init = [&]() {
            std::fill(xl.begin(), xl.end(), 0);
            std::fill(xc.begin(), xc.end(), 0);
            for (int32_t i = 0; i < per_xcd; i++) heap[i] = i;  // all loads 0: already a heap
        };
        auto xcd_done = [&](int32_t x) {
            for (int32_t i = 0; i < per_xcd; i++) load[i * kXcds + x] = xl[i], cnt[i * kXcds + x] = xc[i];
        };
        auto sift_down = [&]() {  // the top's load grew
            int32_t i = 0;
            for (;;) {
                const int32_t l = 2 * i + 1, r = l + 1;
                int32_t m = i;
                if (l < per_xcd && before(heap[l], heap[m])) m = l;
                if (r < per_xcd && before(heap[r], heap[m])) m = r;
                if (m == i) return;
                std::swap(heap[i], heap[m]);
                i = m;
            }
        };
        // each deal records its (workgroup, item) pairs in the order dealt
        using Record = std::vector<std::pair<int32_t, int64_t>>;
        Record rec[3];
        for (Record &r : rec) r.reserve(items.size());
        auto put = [&](int32_t wg, int64_t it, Record *trace) {
            load[wg] += icost[it] - (cnt[wg] ? kPrefetchCost : 0);
            cnt[wg]++;
            if (trace) trace->emplace_back(wg, it);
        };
        // the same onto entry i of XCD x's copies
        auto xput = [&](int32_t x, int32_t i, int64_t it, Record *trace) {
            xl[i] += icost[it] - (xc[i] ? kPrefetchCost : 0);
            xc[i]++;
            if (trace) trace->emplace_back(i * kXcds + x, it);
        };
        // an XCD's items longest first, ties in grid order (a stable counting
        // sort on the small integer costs; a comparison sort past 2^16 tiles)
        std::vector<int64_t> by_cost;
        std::vector<int32_t> tally;
        auto longest_first = [&](const std::vector<int64_t> &in) -> const std::vector<int64_t> & {
            by_cost.resize(in.size());
            int64_t top = 0;
            for (int64_t it : in) top = std::max(top, icost[it]);
            if (top > (1 << 16)) {
                by_cost = in;
                std::stable_sort(by_cost.begin(), by_cost.end(), [&](int64_t a, int64_t b) { return icost[a] > icost[b]; });
                return by_cost;
            }
            tally.assign(top + 2, 0);
            for (int64_t it : in) tally[top - icost[it] + 1]++;  // slot by descending cost
            for (int64_t k = 1; k <= top + 1; k++) tally[k] += tally[k - 1];
            for (int64_t it : in) by_cost[tally[top - icost[it]]++] = it;
            return by_cost;
        };
        auto deal = [&](bool sorted, Record *trace) -> int64_t {
            int64_t worst = 0;
            for (int32_t x = 0; x < kXcds; x++) {
                const std::vector<int64_t> &seq = sorted ? longest_first(by_xcd[x]) : by_xcd[x];
                heap_init();
                for (int64_t it : seq) {
                    const int32_t i = heap[0];
                    xput(x, i, it, trace);
                    sift_down();
                    worst = std::max(worst, xl[i]);
                }
                xcd_done(x);
            }
            return worst;
        };
        // Paired groups: a (chunk, kv head)'s token blocks run side by side, each
        // on its own workgroup of the XCD, so its K/V streams from HBM about
        // once for all of them.  Groups are sorted by cost and the heaviest is
        // paired with the lightest, block i of one with block n - 1 - i of the
        // other (its heaviest with the other's lightest) on one workgroup, and
        // each pair's blocks go to the least-loaded workgroups of the XCD.
        std::vector<int32_t> gstart, gorder, sorder;
        std::vector<int64_t> gcost, scost;
        auto deal_paired = [&](Record *trace) -> int64_t {
            int64_t worst = 0;
            for (int32_t x = 0; x < kXcds; x++) {
                // this XCD's groups: runs of items of one (chunk, kv head), in grid order
                const std::vector<int64_t> &xs = by_xcd[x];
                gstart.clear();
                gcost.clear();
                for (size_t i = 0; i < xs.size(); i++) {
                    if (i == 0 || items[xs[i - 1]].chunk.x != items[xs[i]].chunk.x ||
                        items[xs[i - 1]].kvh != items[xs[i]].kvh) {
                        gstart.push_back((int32_t)i);
                        gcost.push_back(0);
                    }
                    gcost.back() += icost[xs[i]];
                }
                const int32_t ng = (int32_t)gstart.size();
                heap_init();
                gstart.push_back((int32_t)xs.size());
                gorder.resize(ng);
                for (int32_t g = 0; g < ng; g++) gorder[g] = g;
                std::stable_sort(gorder.begin(), gorder.end(), [&](int32_t a, int32_t b) { return gcost[a] > gcost[b]; });
                for (int32_t lo = 0, hi = ng; lo < hi; lo++) {
                    // the pair (lo, hi - 1), or group lo alone when it is the last;
                    // slot k holds block k of group lo, then the blocks i of the
                    // other with n - 1 - (i mod n) = k
                    const int32_t ga = gorder[lo], na = gstart[ga + 1] - gstart[ga];
                    const int32_t gb = hi - 1 > lo ? gorder[--hi] : -1;
                    const int32_t nb = gb < 0 ? 0 : gstart[gb + 1] - gstart[gb];
                    scost.assign(na, 0);
                    for (int32_t k = 0; k < na; k++) scost[k] = icost[xs[gstart[ga] + k]];
                    for (int32_t i = 0; i < nb; i++) scost[na - 1 - (i % na)] += icost[xs[gstart[gb] + i]];
                    // the pair's slots onto the least-loaded workgroups of this XCD,
                    // heaviest slot first
                    // (a stable counting sort on the slot costs when their range is small)
                    sorder.resize(na);
                    int64_t smin = scost[0], smax = scost[0];
                    for (int32_t k = 1; k < na; k++) smin = std::min(smin, scost[k]), smax = std::max(smax, scost[k]);
                    if (smax - smin <= 4 * (int64_t)na + 64) {
                        tally.assign(smax - smin + 2, 0);
                        for (int32_t k = 0; k < na; k++) tally[smax - scost[k] + 1]++;
                        for (int64_t v = 1; v <= smax - smin + 1; v++) tally[v] += tally[v - 1];
                        for (int32_t k = 0; k < na; k++) sorder[tally[smax - scost[k]]++] = k;
                    } else {
                        for (int32_t k = 0; k < na; k++) sorder[k] = k;
                        std::stable_sort(sorder.begin(), sorder.end(), [&](int32_t u, int32_t v) { return scost[u] > scost[v]; });
                    }
                    for (int32_t k : sorder) {
                        const int32_t w = heap[0];
                        xput(x, w, xs[gstart[ga] + k], trace);
                        for (int32_t i = na - 1 - k; i < nb; i += na) xput(x, w, xs[gstart[gb] + i], trace);
                        sift_down();
                        worst = std::max(worst, xl[w]);
                    }
                }
                xcd_done(x);
            }
            return worst;
        };
        static_makespan = deal(false, &rec[0]);
        const int64_t sorted_makespan = deal(true, &rec[1]);
        const int64_t paired_makespan = deal_paired(&rec[2]);
        int deal_pick = 0;  // 0 grid order, 1 longest first, 2 paired groups
        if ((double)sorted_makespan < 0.99 * (double)static_makespan) deal_pick = 1;
        const int64_t best_other = deal_pick == 1 ? sorted_makespan : static_makespan;
        // paired groups keep their L2 sharing: taken when its estimate is no longer
        if ((double)paired_makespan <= kPairedSlack * (double)best_other) deal_pick = 2;
        // the chosen deal's record: its loads again, then its items grouped by
        // workgroup (a counting sort keeps each workgroup's order dealt)
        const Record &dealt = rec[deal_pick];
        static_makespan = deal_pick == 2 ? paired_makespan : (deal_pick == 1 ? sorted_makespan : static_makespan);
        std::fill(load.begin(), load.end(), 0);
        std::fill(cnt.begin(), cnt.end(), 0);
        for (const auto &d : dealt) put(d.first, d.second, nullptr);
        static_off.assign(groups + 1, 0);
        for (int32_t b = 0; b < groups; b++) static_off[b + 1] = static_off[b] + cnt[b];
        static_items.resize(dealt.size());
        std::vector<int32_t> fill(static_off.begin(), static_off.end() - 1);
        for (const auto &d : dealt) static_items[fill[d.first]++] = d.second;
        // With few items per workgroup (at most 4 on average) dealing onto the
        // least-loaded workgroup leaves slack, so a local search follows: the
        // most-loaded workgroup of an XCD gives one of its items to another
        // workgroup of the XCD, or swaps it for a shorter one there, taking the
        // change that lowers the larger of the two loads the most, until no
        // change lowers it.  Items stay on their XCD.
        // Lists are kept at most kCap items per workgroup (no move into a full one).
        constexpr int32_t kCap = 16;
        bool fits = (int64_t)dealt.size() <= 4 * (int64_t)groups && per_xcd > 1;
        for (int32_t b = 0; fits && b < groups; b++) fits = cnt[b] <= kCap;
        if (fits) {
            std::vector<int64_t> wl((size_t)groups * kCap);
            std::vector<int32_t> wn(groups);
            for (int32_t b = 0; b < groups; b++) {
                wn[b] = cnt[b];
                std::copy(static_items.begin() + static_off[b], static_items.begin() + static_off[b + 1], wl.begin() + (size_t)b * kCap);
            }
            auto at = [&](int32_t b, int32_t k) -> int64_t & { return wl[(size_t)b * kCap + k]; };
            bool moved = false;
            for (int32_t x = 0; x < kXcds; x++) {
                for (int32_t iter = 0; iter < 4 * per_xcd; iter++) {
                    int32_t A = x;
                    for (int32_t b = x + kXcds; b < groups; b += kXcds)
                        if (load[b] > load[A]) A = b;
                    const int64_t LA = load[A];
                    int64_t best = LA;
                    int32_t bk = -1, bB = -1, bj = -1;  // item k of A to workgroup B (for its item j; -1: a move)
                    for (int32_t k = 0; k < wn[A]; k++) {
                        const int64_t a = icost[at(A, k)];
                        const int64_t la_mv = LA - a + (wn[A] > 1 ? kPrefetchCost : 0);
                        for (int32_t B = x; B < groups; B += kXcds) {
                            const int64_t LB = load[B];
                            // a move or swap leaves B above LB (items cost more than
                            // the prefetch credit; a swap takes a shorter item)
                            if (B == A || LB + 1 >= best) continue;
                            if (wn[B] < kCap) {
                                const int64_t mv = std::max(la_mv, LB + a - (wn[B] ? kPrefetchCost : 0));
                                if (mv < best) best = mv, bk = k, bB = B, bj = -1;
                            }
                            for (int32_t j = 0; j < wn[B]; j++) {
                                const int64_t c = icost[at(B, j)];
                                if (c >= a) continue;
                                const int64_t sw = std::max(LA - a + c, LB - c + a);
                                if (sw < best) best = sw, bk = k, bB = B, bj = j;
                            }
                        }
                    }
                    if (bk < 0) break;
                    const int64_t it = at(A, bk);
                    if (bj < 0) {  // A's items close up; the item joins B's end
                        for (int32_t k = bk; k + 1 < wn[A]; k++) at(A, k) = at(A, k + 1);
                        wn[A]--;
                        load[A] -= icost[it] - (wn[A] ? kPrefetchCost : 0);
                        load[bB] += icost[it] - (wn[bB] ? kPrefetchCost : 0);
                        at(bB, wn[bB]++) = it;
                    } else {  // the two items trade places
                        const int64_t other = at(bB, bj);
                        at(A, bk) = other;
                        at(bB, bj) = it;
                        load[A] += icost[other] - icost[it];
                        load[bB] += icost[it] - icost[other];
                    }
                    moved = true;
                }
            }
            if (moved) {
                static_makespan = 0;
                for (int32_t b = 0; b < groups; b++) {
                    static_off[b + 1] = static_off[b] + wn[b];
                    std::copy(wl.begin() + (size_t)b * kCap, wl.begin() + (size_t)b * kCap + wn[b], static_items.begin() + static_off[b]);
                    static_makespan = std::max(static_makespan, load[b]);
                }
            }
        }
    }

    const int64_t grid_makespan = static_makespan < grid_lb ? grid_lb : grid_estimate();
    // The balanced split: the smallest capacity that fits the line into
    // `groups` workgroups, searched upward from its lower bound.  It pays for
    // its partials and, with many items per workgroup, loses the side-by-side
    // L2 sharing of the grid order: it is taken only when it clearly shortens
    // the estimated makespan, so the search is skipped when even its bound
    // cannot, unless no other schedule applies.
    int64_t lo = std::max<int64_t>((total + groups - 1) / groups, kSegCost + kSplitCost + kMinPiece);
    const double best_whole = (double)std::min(grid_makespan, static_makespan);
    const bool split_can_win = allow_split && (double)lo <= 0.95 * best_whole;
    const bool other_applies = static_makespan < grid_makespan || grid_ids <= INT32_MAX;
    if (split_can_win || !other_applies) {
        int64_t hi = std::max<int64_t>(lo, total + kSegCost);
        while (lo < hi) {
            const int64_t mid = (lo + hi) / 2;
            if (pf_fill(items, mid, groups, nullptr, nullptr) <= groups) hi = mid; else lo = mid + 1;
        }
    }
    const bool split_wins = split_can_win && (double)lo <= 0.95 * best_whole;
    if (!split_wins && static_makespan < grid_makespan) {
        out.range.assign(groups, make_int2(0, 0));
        for (int32_t b = 0; b < groups; b++) {
            const int32_t first = (int32_t)(out.work.size() / 3);
            for (int32_t k = static_off[b]; k < static_off[b + 1]; k++) {
                const PfItem &it = items[static_items[k]];
                out.work.push_back(it.chunk);
                out.work.push_back(make_int4(it.kvh, it.tok0, it.t_lo, it.t_hi));
                out.work.push_back(make_int4(0, 0, 1, 0));
            }
            out.range[b] = make_int2(first, (int32_t)(out.work.size() / 3));
        }
        p.pf_groups = groups;
        return;
    }
    if (grid_ids <= INT32_MAX && !split_wins) {
        out.range.assign(grid_ids, make_int2(0, 0));
        for (int64_t b = 0; b < grid_ids; b++) {
            if (grid_item[b] < 0) continue;
            const PfItem &it = items[grid_item[b]];
            const int32_t k = (int32_t)(out.work.size() / 3);
            out.work.push_back(it.chunk);
            out.work.push_back(make_int4(it.kvh, it.tok0, it.t_lo, it.t_hi));
            out.work.push_back(make_int4(0, 0, 1, 0));
            out.range[b] = make_int2(k, k + 1);
        }
        p.pf_groups = (int32_t)grid_ids;
        return;
    }
    std::vector<int32_t> first(groups + 1, 0);
    const int32_t parts = pf_fill(items, lo, groups, &out, &first);
    first[parts] = (int32_t)(out.work.size() / 3);
    // workgroup b runs on XCD b % 8: consecutive parts on one XCD
    const int32_t per = (parts + kXcds - 1) / kXcds;
    const int32_t wgs = parts <= kXcds ? parts : kXcds * per;
    out.range.assign(wgs, make_int2(0, 0));
    for (int32_t b = 0; b < wgs; b++) {
        const int32_t part = parts <= kXcds ? b : (b % kXcds) * per + b / kXcds;
        if (part < parts) out.range[b] = make_int2(first[part], first[part + 1]);
    }
    p.pf_groups = wgs;
}

}  // namespace pam
