// Draft-tree builders that produce the verify trees of the tree-verify path.
//
//  * cartesian_tree: build_cartesian_tree (crates/speculate/src/methods/medusa.rs:172-193).
//    Layer 0 is the root; layer d+1 attaches every candidate of step d under
//    every node of layer d, in BFS order, so parents always precede children.
//  * prune_cartesian: prune_cartesian_tree (crates/speculate/src/methods/eagle.rs:763-845).
//    Every non-root node is scored by the f32 sum of the per-step log-probs of
//    the candidates on its root path (summed from the node upwards), the
//    max_total - 1 best survive (stable descending order, so equal scores keep
//    BFS order), their ancestors are added back, and the survivors are
//    re-emitted sorted stably by depth with re-indexed parents.
#include <algorithm>
#include <string>
#include <vector>

#include "sd_model.hpp"

namespace sd {

DraftTreeC cartesian_tree(uint32_t root, const uint32_t *cand, const uint32_t *branching, size_t depth) {
    DraftTreeC t;
    t.tokens.push_back(root);
    t.parents.push_back(0);
    std::vector<uint32_t> prev{0}, next;
    size_t off = 0;
    for (size_t d = 0; d < depth; d++) {
        const uint32_t b = branching[d];
        next.clear();
        for (uint32_t p : prev)
            for (uint32_t c = 0; c < b; c++) {
                next.push_back((uint32_t)t.tokens.size());
                t.tokens.push_back(cand[off + c]);
                t.parents.push_back(p);
            }
        off += b;
        prev.swap(next);
    }
    return t;
}

size_t cartesian_size(const uint32_t *branching, size_t depth) {
    size_t n = 1, layer = 1;
    for (size_t d = 0; d < depth; d++) {
        layer *= branching[d];
        n += layer;
        if (n > (size_t)1 << 24) throw ArgError("Cartesian tree too large");
    }
    return n;
}

DraftTreeC prune_cartesian(const DraftTreeC &full, const float *log_probs, const uint32_t *branching, size_t depth,
                           size_t max_total) {
    const size_t n = full.size();
    if (n <= max_total) return full;
    // per-step offsets into the back-to-back log-prob table
    std::vector<size_t> off(depth + 1, 0);
    for (size_t d = 0; d < depth; d++) off[d + 1] = off[d] + branching[d];

    // sibling rank of every node = its candidate index at its step
    std::vector<uint32_t> rank(n, 0), seen(n, 0);
    for (size_t i = 1; i < n; i++) rank[i] = seen[full.parents[i]]++;
    std::vector<int> dep(n, 0);
    for (size_t i = 1; i < n; i++) dep[i] = dep[full.parents[i]] + 1;

    struct Sc {
        uint32_t node;
        float s;
    };
    std::vector<Sc> scores;
    scores.reserve(n - 1);
    for (size_t i = 1; i < n; i++) {
        const int d = dep[i];
        if ((size_t)d > depth) throw ArgError("tree deeper than the log-prob table");
        float s = 0.f;
        size_t cur = i;
        for (int dd = d - 1; dd >= 0; dd--) {
            if (rank[cur] >= branching[dd]) throw ArgError("node rank exceeds the branching of its step");
            s += log_probs[off[dd] + rank[cur]];
            cur = full.parents[cur];
        }
        scores.push_back(Sc{(uint32_t)i, s});
    }
    // descending; incomparable (NaN) pairs count as equal and keep their order
    std::stable_sort(scores.begin(), scores.end(), [](const Sc &a, const Sc &b) { return a.s > b.s; });
    const size_t want = std::min(max_total > 0 ? max_total - 1 : 0, scores.size());
    std::vector<char> keep(n, 0);
    keep[0] = 1;
    for (size_t j = 0; j < want; j++) keep[scores[j].node] = 1;
    for (size_t i = n - 1; i >= 1; i--)
        if (keep[i]) keep[full.parents[i]] = 1;

    std::vector<uint32_t> order;
    for (size_t i = 0; i < n; i++)
        if (keep[i]) order.push_back((uint32_t)i);
    std::stable_sort(order.begin(), order.end(), [&](uint32_t a, uint32_t b) { return dep[a] < dep[b]; });
    std::vector<uint32_t> new_index(n, 0);
    for (size_t k = 0; k < order.size(); k++) new_index[order[k]] = (uint32_t)k;
    DraftTreeC out;
    for (uint32_t old : order) {
        out.tokens.push_back(full.tokens[old]);
        out.parents.push_back(old == 0 ? 0 : new_index[full.parents[old]]);
    }
    // the re-emitted table must satisfy parent < self (DraftTree::from_parent_table)
    for (size_t i = 1; i < out.size(); i++)
        if (out.parents[i] >= i) throw SamplingError("pruned tree invalid: parent not before child");
    return out;
}

}  // namespace sd
