// block_allocator.cpp - see block_allocator.h (KVCacheManager.swift:47-379).
#include "block_allocator.h"

#include <algorithm>
#include <cstdlib>

namespace pam {

BlockAllocator::BlockAllocator(int32_t max_blocks, int32_t block_size)
    : max_blocks_(max_blocks), block_size_(block_size), ref_(max_blocks > 0 ? max_blocks : 0, 0) {
    // Deque((0..<maxBlocks).reversed()) : back of the deque is block 0
    for (int32_t b = max_blocks - 1; b >= 0; b--) free_.push_back(b);
}

void BlockAllocator::allocate_sequence(int64_t id) {
    if (seqs_.count(id)) throw SequenceExistsError();
    seqs_.emplace(id, LogicalSequence{});
}

const LogicalSequence &BlockAllocator::sequence(int64_t id) const {
    auto it = seqs_.find(id);
    if (it == seqs_.end()) throw SequenceNotFoundError();
    return it->second;
}

int32_t BlockAllocator::allocate_block() {
    if (policy_ == EvictionPolicy::kBestFit) return allocate_best_fit();
    const int32_t b = free_.back();  // removeLast
    free_.pop_back();
    return b;
}

// KVCacheManager.swift:250-265: first free block whose held size is closest to a
// full block (default: a full block).
int32_t BlockAllocator::allocate_best_fit() {
    size_t best = 0;
    int64_t best_delta = INT64_MAX;
    for (size_t i = 0; i < free_.size(); i++) {
        auto it = free_sizes_.find(free_[i]);
        const int64_t held = it == free_sizes_.end() ? block_size_ : it->second;
        const int64_t delta = std::llabs(held - block_size_);
        if (delta < best_delta) {
            best_delta = delta;
            best = i;
        }
    }
    const int32_t b = free_[best];
    free_.erase(free_.begin() + (std::ptrdiff_t)best);
    free_sizes_.erase(b);
    return b;
}

void BlockAllocator::copy_on_write(LogicalSequence &seq, int32_t index, BlockCopies *copies) {
    if (free_.empty()) throw OutOfMemoryError();
    const int32_t old_block = seq.block_table[index];
    const int32_t new_block = allocate_block();
    if (copies) copies->emplace_back(old_block, new_block);
    ref_[old_block] -= 1;
    ref_[new_block] = 1;
    seq.block_table[index] = new_block;
}

// KVCacheManager.swift:115-174.  Works on a copy of the sequence that is stored
// back only on success; allocator state a copy-on-write already changed stays
// changed on a later out-of-memory, exactly as in the reference.
void BlockAllocator::append_tokens(int64_t id, int64_t count, const uint64_t *hashes, int32_t n_hashes,
                                   BlockCopies *copies) {
    if (count < 0) throw invalid_request("count must be non-negative");
    if (count == 0) return;
    auto it = seqs_.find(id);
    if (it == seqs_.end()) throw SequenceNotFoundError();
    LogicalSequence seq = it->second;
    const int64_t bs = block_size_;
    const int64_t cur = seq.length, next = cur + count;
    const int64_t now = (cur + bs - 1) / bs, after = (next + bs - 1) / bs;
    const int64_t extra = after - now;
    if (now > 0 && cur % bs != 0) {
        const int32_t last = seq.block_table[(size_t)(now - 1)];
        if (ref_[last] > 1) copy_on_write(seq, (int32_t)(now - 1), copies);
    }
    if (extra > 0) {
        if ((int64_t)free_.size() < extra) throw OutOfMemoryError();
        for (int64_t i = 0; i < extra; i++) {
            const bool hashed = hashes != nullptr && i < n_hashes;
            if (hashed) {
                auto hit = prefix_.find(hashes[i]);
                if (hit != prefix_.end()) {
                    seq.block_table.push_back(hit->second);
                    ref_[hit->second] += 1;
                    prefix_hits_ += 1;
                    continue;
                }
            }
            const int32_t b = allocate_block();
            seq.block_table.push_back(b);
            ref_[b] = 1;
            if (hashed) prefix_[hashes[i]] = b;
        }
    }
    seq.length = next;
    it->second = std::move(seq);
}

// KVCacheManager.swift:200-214
void BlockAllocator::ensure_exclusive(int64_t id, int32_t logical_block, BlockCopies *copies) {
    auto it = seqs_.find(id);
    if (it == seqs_.end()) throw SequenceNotFoundError();
    LogicalSequence &seq = it->second;
    if (logical_block < 0 || logical_block >= (int32_t)seq.block_table.size())
        throw invalid_request("block index out of range");
    if (ref_[seq.block_table[logical_block]] > 1) copy_on_write(seq, logical_block, copies);
}

// KVCacheManager.swift:216-239
void BlockAllocator::free_sequence(int64_t id) {
    auto it = seqs_.find(id);
    if (it == seqs_.end()) return;
    const LogicalSequence seq = std::move(it->second);
    seqs_.erase(it);
    const size_t total = seq.block_table.size();
    const int64_t rem = seq.length % block_size_;
    const int32_t last_tokens = rem == 0 ? block_size_ : (int32_t)rem;
    for (size_t i = 0; i < total; i++) {
        const int32_t b = seq.block_table[i];
        ref_[b] -= 1;
        if (ref_[b] <= 0) {
            switch (policy_) {
                case EvictionPolicy::kFifo: free_.push_front(b); break;
                case EvictionPolicy::kLifo: free_.push_back(b); break;
                case EvictionPolicy::kBestFit:
                    free_sizes_[b] = i + 1 < total ? block_size_ : last_tokens;
                    free_.push_back(b);
                    break;
            }
        }
    }
}

// KVCacheManager.swift:65-67 + 267-283
void BlockAllocator::set_policy(EvictionPolicy p) {
    policy_ = p;
    if (p == EvictionPolicy::kFifo || p == EvictionPolicy::kLifo) {
        std::reverse(free_.begin(), free_.end());
        free_sizes_.clear();
    } else {
        for (int32_t b : free_)
            if (!free_sizes_.count(b)) free_sizes_[b] = block_size_;
        std::vector<int32_t> v(free_.begin(), free_.end());
        std::stable_sort(v.begin(), v.end(), [&](int32_t a, int32_t b) {
            auto fa = free_sizes_.find(a), fb = free_sizes_.find(b);
            const int32_t sa = fa == free_sizes_.end() ? 0 : fa->second;
            const int32_t sb = fb == free_sizes_.end() ? 0 : fb->second;
            return sa > sb;
        });
        free_.assign(v.begin(), v.end());
    }
}

// KVCacheManager.swift:353-378
AllocatorStats BlockAllocator::stats() const {
    AllocatorStats s{};
    s.total_blocks = max_blocks_;
    s.free_blocks = (int64_t)free_.size();
    s.used_blocks = max_blocks_ - s.free_blocks;
    s.active_sequences = (int64_t)seqs_.size();
    int64_t partial = 0;
    for (const auto &kv : seqs_) {
        const int64_t rem = kv.second.length % block_size_;
        if (rem > 0 && rem < block_size_) partial++;
    }
    s.partially_filled_blocks = partial;
    const int64_t active = seqs_.empty() ? 1 : (int64_t)seqs_.size();
    s.fragmentation_ratio = (float)partial / (float)active;
    s.prefix_cache_hits = prefix_hits_;
    s.prefix_cache_entries = (int64_t)prefix_.size();
    int64_t shared = 0;
    for (int32_t r : ref_)
        if (r > 1) shared++;
    s.shared_blocks = shared;
    return s;
}

}  // namespace pam
