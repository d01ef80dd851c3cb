// scheduler.h - ContinuousBatchingScheduler (Sources/PagedAttentionMetal/Scheduler.swift:42-177).
//
// Same policy, including its documented quirks: completed sequences stay in
// the table (so addRequest returns -1 once maxSequences entries exist, :59-70),
// step() serves waiting requests first, then unfinished running ones, then
// paused ones, each in arrival order (:78-114), and handleMemoryPressure pauses
// the newest running sequence for as long as the availability callback reports
// too few blocks (:135-152) - the caller frees the victims afterwards.
#pragma once
#include <cstdint>
#include <functional>
#include <map>
#include <mutex>
#include <vector>

namespace pam {

enum class SeqStatus : int32_t { kWaiting = 0, kRunning = 1, kPaused = 2, kCompleted = 3 };

struct SchedulerSequence {
    int32_t id;
    int32_t prompt_length;
    int32_t max_new_tokens;
    int32_t arrival_order;
    int32_t generated = 0;
    SeqStatus status = SeqStatus::kWaiting;
    bool done() const { return generated >= max_new_tokens; }
    int32_t current_length() const { return prompt_length + generated; }
};

class Scheduler {
   public:
    Scheduler(int32_t max_batch, int32_t max_sequences) : max_batch_(max_batch), max_sequences_(max_sequences) {}
    int32_t add_request(int32_t prompt, int32_t max_new);
    void complete(int32_t id);
    std::vector<int32_t> step();
    void mark_prefilled(int32_t id);
    void mark_decoded(int32_t id);
    void preempt(int32_t id);
    std::vector<int32_t> handle_memory_pressure(int32_t required, const std::function<int32_t()> &available);
    int32_t count(SeqStatus s);
    bool get(int32_t id, SchedulerSequence *out);

   private:
    std::vector<SchedulerSequence *> sorted_with(SeqStatus s, bool only_unfinished);
    std::mutex mu_;
    int32_t max_batch_, max_sequences_;
    int32_t next_id_ = 0, arrivals_ = 0;
    std::map<int32_t, SchedulerSequence> seqs_;
};

}  // namespace pam
