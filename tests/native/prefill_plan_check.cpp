// Host-only check of the dense prefill work list (prefill_split_plan): built by
// tests/test_prefill_plan.py with hipcc and run on the CPU (no kernel launches).
// For random chunk sets, group sizes, windows and CU counts it checks that
//  * every workgroup range holds whole segments and every segment belongs to
//    exactly one workgroup;
//  * each item (chunk, kv head, token block) is covered by its segments in
//    order, tiles [t_lo, t_hi) exactly, with the item's key range:
//    t_lo = window start / 32, t_hi = ceil(last key + 1, 32);
//  * a split item's pieces carry the same first slot and piece count, pieces
//    are numbered 0..n-1, and slot ranges of split items do not overlap;
//  * the split schedule uses at most one workgroup per CU (rounded up to 8).
#include <cstdio>
#include <map>
#include <random>
#include <set>
#include <tuple>

#include "../../pagedattentionmetal_amd/csrc/kernels/prefill.hip"

using namespace pam;

static int check(const std::vector<int4> &ch, int H, int Hkv, int W, int causal, int groups) {
    AttnParams p{};
    p.num_heads = H;
    p.num_kv_heads = Hkv;
    p.window = W;
    p.causal = causal;
    PrefillSplit ps;
    prefill_split_plan(ch.data(), (int)ch.size(), p, groups, ps);
    const int tpw = 256 / (H / Hkv);
    const int nseg = (int)ps.work.size() / 3;
    if ((int)ps.work.size() != 3 * nseg || p.pf_groups != (int)ps.range.size()) return 1;
    std::vector<int> owner(nseg, -1);
    for (int b = 0; b < (int)ps.range.size(); b++)
        for (int s = ps.range[b].x; s < ps.range[b].y; s++) {
            if (s < 0 || s >= nseg || owner[s] != -1) return 2;
            owner[s] = b;
        }
    std::map<std::tuple<int, int, int>, std::vector<int>> segs;  // item -> segments
    for (int s = 0; s < nseg; s++) {
        if (owner[s] < 0) return 3;
        const int4 c = ps.work[3 * s], a = ps.work[3 * s + 1];
        int cix = -1;
        for (int i = 0; i < (int)ch.size(); i++)
            if (ch[i].x == c.x && ch[i].y == c.y && ch[i].z == c.z && ch[i].w == c.w) cix = i;
        if (cix < 0) return 4;
        segs[{cix, a.x, a.y}].push_back(s);
    }
    std::set<int> slots_used;
    size_t items = 0;
    for (int c = 0; c < (int)ch.size(); c++) {
        const int kv_len = ch[c].y + ch[c].z, ws = W > 0 ? std::max(0, kv_len - W) : 0;
        for (int h = 0; h < Hkv; h++)
            for (int t0 = 0; t0 < ch[c].z; t0 += tpw) {
                items++;
                const int te = std::min(t0 + tpw, ch[c].z), ke = causal ? ch[c].y + te : kv_len;
                const int lo = ws / 32, hi = std::max(lo, (ke + 31) / 32);
                auto it = segs.find({c, h, t0});
                if (it == segs.end()) return 5;
                const std::vector<int> &v = it->second;
                int cur = lo;
                const int pieces = ps.work[3 * v[0] + 2].z, slot0 = ps.work[3 * v[0] + 2].x;
                if (pieces != (int)v.size()) return 6;
                for (int k = 0; k < (int)v.size(); k++) {
                    const int4 a = ps.work[3 * v[k] + 1], b = ps.work[3 * v[k] + 2];
                    if (a.z != cur || a.w < a.z || b.y != k || b.z != pieces || b.x != slot0) return 7;
                    cur = a.w;
                }
                if (cur != hi) return 8;
                if (pieces > 1) {
                    for (int k = 0; k < pieces; k++)
                        if (!slots_used.insert(slot0 + k).second || slot0 + k >= ps.slots) return 9;
                }
            }
    }
    if (segs.size() != items) return 10;
    if (ps.slots > 0 && (int)ps.range.size() > (groups + 7) / 8 * 8) return 11;
    return 0;
}

int main() {
    std::mt19937 rng(5);
    int failures = 0, split_plans = 0, multi_plans = 0;
    for (int trial = 0; trial < 3000; trial++) {
        const int n = 1 + rng() % 10, Hkv = 1 << (rng() % 4), G = 1 << (rng() % 4);
        std::vector<int4> ch;
        int row_base = 0;
        for (int i = 0; i < n; i++) {
            const int len = 1 + rng() % 3000, ctx = rng() % 5000;
            ch.push_back(make_int4(i, ctx, len, row_base));
            row_base += len;
        }
        const int W = rng() % 3 == 0 ? 1 + rng() % 4000 : 0;
        const int causal = rng() % 4 != 0, groups = 1 + rng() % 300;
        const int rc = check(ch, G * Hkv, Hkv, W, causal, groups);
        if (rc) {
            std::printf("trial %d: check %d failed (n %d, G %d, Hkv %d, W %d, causal %d, groups %d)\n", trial, rc, n,
                        G, Hkv, W, causal, groups);
            failures++;
        }
        AttnParams p{};
        p.num_heads = G * Hkv;
        p.num_kv_heads = Hkv;
        p.window = W;
        p.causal = causal;
        PrefillSplit ps;
        prefill_split_plan(ch.data(), (int)ch.size(), p, groups, ps);
        split_plans += ps.slots > 0;
        bool several = false;
        for (const int2 &r : ps.range) several |= r.y - r.x > 1;
        multi_plans += ps.slots == 0 && several;  // static grid, or a balanced split that cut nothing
    }
    // c3's chunks on 192 workgroups (the one-launch mixed step's prefill part):
    // 512 whole items, 2.7 per workgroup.  Dealt longest-first onto the
    // least-loaded workgroup its largest load is 217 tiles (12 per item, less 4
    // for each later item of a workgroup); the local search that follows the
    // deal brings it to 197.
    {
        const int ctx[8] = {2412, 1645, 1012, 369, 1595, 2566, 2747, 1490};
        std::vector<int4> ch;
        for (int i = 0; i < 8; i++) ch.push_back(make_int4(i, ctx[i], 512, 512 * i));
        const int rc = check(ch, 32, 8, 0, 1, 192);
        AttnParams p{};
        p.num_heads = 32;
        p.num_kv_heads = 8;
        p.causal = 1;
        PrefillSplit ps;
        prefill_split_plan(ch.data(), 8, p, 192, ps);
        long worst = 0;
        for (const int2 &r : ps.range) {
            long load = 0;
            for (int s = r.x; s < r.y; s++) load += ps.work[3 * s + 1].w - ps.work[3 * s + 1].z + 12 - (s > r.x ? 4 : 0);
            worst = std::max(worst, load);
        }
        std::printf("c3 chunks on 192 workgroups: check %d, %zu workgroups, %d slots, largest load %ld tiles\n", rc,
                    ps.range.size(), ps.slots, worst);
        if (rc || ps.slots != 0 || ps.range.size() != 192 || worst > 197) failures++;
    }
    std::printf("%d failures, %d of 3000 plans split items, %d run several whole items per workgroup\n", failures,
                split_plans, multi_plans);
    return failures ? 1 : 0;
}
