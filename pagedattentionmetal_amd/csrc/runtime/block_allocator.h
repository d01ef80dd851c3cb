// block_allocator.h - host-side paged block bookkeeping.
//
// Restates KVCacheManager's block logic (Sources/PagedAttentionMetal/KVCacheManager.swift):
// the free list is a deque initialised to reversed(0..<maxBlocks) (:101) and
// allocation takes from its back (:241-248), so a fresh cache hands out blocks
// 0, 1, 2, ...; frees go to the front (FIFO), the back (LIFO) or the back with a
// held-size note (best fit, :216-239, :250-265).  Prefix hashes map to shared,
// ref-counted blocks (:150-168); appending into a shared partial tail block
// copies it first (:134-140, :176-194).  Data movement is not done here: every
// copy-on-write is returned to the caller as a (src, dst) block pair, which the
// device cache turns into HBM-to-HBM copies on its stream.
#pragma once
#include <cstdint>
#include <deque>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace pam {

// KVCacheError (KVCacheManager.swift:6-11) and PagedAttentionError
// (PagedAttentionTypes.swift:5-64) surface as this exception with the text the
// C ABI hands back through pam_last_error.
struct PamError : std::runtime_error {
    explicit PamError(const std::string &m) : std::runtime_error(m) {}
};
// A request larger than the allocation-free decode's fixed scratch: always
// reported as an error, also under graceful degradation.
struct ScratchLimitError : PamError {
    explicit ScratchLimitError(const std::string &m) : PamError(m) {}
};
// A failure reported by the GPU after work was enqueued (never retried).
struct ExecutionError : PamError {
    explicit ExecutionError(const std::string &m) : PamError(m) {}
};
struct OutOfMemoryError : PamError {
    OutOfMemoryError() : PamError("KVCacheError.outOfMemory") {}
};
struct SequenceNotFoundError : PamError {
    SequenceNotFoundError() : PamError("KVCacheError.sequenceNotFound") {}
};
struct SequenceExistsError : PamError {
    SequenceExistsError() : PamError("KVCacheError.sequenceAlreadyExists") {}
};
inline PamError invalid_request(const std::string &m) { return PamError("KVCacheError.invalidRequest: " + m); }
inline PamError invalid_configuration(const std::string &m) {
    return PamError("Invalid paged attention configuration: " + m);
}
inline PamError buffer_too_small(const std::string &name, int64_t expected, int64_t actual) {
    return PamError(name + " buffer is too small: expected at least " + std::to_string(expected) + " bytes, got " +
                    std::to_string(actual) + ".");
}

enum class EvictionPolicy : int32_t { kFifo = 0, kLifo = 1, kBestFit = 2 };

struct LogicalSequence {
    std::vector<int32_t> block_table;
    int64_t length = 0;
};

using BlockCopies = std::vector<std::pair<int32_t, int32_t>>;

struct AllocatorStats {
    int64_t total_blocks, used_blocks, free_blocks, active_sequences;
    int64_t partially_filled_blocks;
    float fragmentation_ratio;
    int64_t prefix_cache_hits, prefix_cache_entries, shared_blocks;
};

class BlockAllocator {
   public:
    BlockAllocator(int32_t max_blocks, int32_t block_size);

    void allocate_sequence(int64_t id);
    // appends count tokens; hashes (may be null) name the new blocks for prefix reuse
    void append_tokens(int64_t id, int64_t count, const uint64_t *hashes, int32_t n_hashes, BlockCopies *copies);
    void ensure_exclusive(int64_t id, int32_t logical_block, BlockCopies *copies);
    void free_sequence(int64_t id);
    void register_block_hash(uint64_t hash, int32_t block) { prefix_[hash] = block; }
    void set_policy(EvictionPolicy p);
    EvictionPolicy policy() const { return policy_; }

    const LogicalSequence &sequence(int64_t id) const;
    bool has_sequence(int64_t id) const { return seqs_.count(id) != 0; }
    int32_t available() const { return (int32_t)free_.size(); }
    int32_t max_blocks() const { return max_blocks_; }
    int32_t block_size() const { return block_size_; }
    int32_t ref_count(int32_t block) const { return ref_[block]; }
    AllocatorStats stats() const;

   private:
    int32_t allocate_block();
    int32_t allocate_best_fit();
    void copy_on_write(LogicalSequence &seq, int32_t index, BlockCopies *copies);

    int32_t max_blocks_, block_size_;
    EvictionPolicy policy_ = EvictionPolicy::kFifo;
    std::deque<int32_t> free_;
    std::unordered_map<int32_t, int32_t> free_sizes_;
    std::unordered_map<int64_t, LogicalSequence> seqs_;
    std::unordered_map<uint64_t, int32_t> prefix_;
    std::vector<int32_t> ref_;
    int64_t prefix_hits_ = 0;
};

}  // namespace pam
