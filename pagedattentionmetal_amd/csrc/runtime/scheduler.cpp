// scheduler.cpp - see scheduler.h (Scheduler.swift:42-177).
#include "scheduler.h"

#include <algorithm>

namespace pam {

int32_t Scheduler::add_request(int32_t prompt, int32_t max_new) {
    std::lock_guard<std::mutex> g(mu_);
    if ((int32_t)seqs_.size() >= max_sequences_) return -1;
    const int32_t id = next_id_++;
    SchedulerSequence s{};
    s.id = id;
    s.prompt_length = prompt;
    s.max_new_tokens = max_new;
    s.arrival_order = arrivals_++;
    seqs_.emplace(id, s);
    return id;
}

void Scheduler::complete(int32_t id) {
    std::lock_guard<std::mutex> g(mu_);
    auto it = seqs_.find(id);
    if (it != seqs_.end()) it->second.status = SeqStatus::kCompleted;
}

std::vector<SchedulerSequence *> Scheduler::sorted_with(SeqStatus st, bool only_unfinished) {
    std::vector<SchedulerSequence *> v;
    for (auto &kv : seqs_)
        if (kv.second.status == st && (!only_unfinished || !kv.second.done())) v.push_back(&kv.second);
    std::sort(v.begin(), v.end(),
              [](const SchedulerSequence *a, const SchedulerSequence *b) { return a->arrival_order < b->arrival_order; });
    return v;
}

std::vector<int32_t> Scheduler::step() {
    std::lock_guard<std::mutex> g(mu_);
    auto waiting = sorted_with(SeqStatus::kWaiting, false);
    auto running = sorted_with(SeqStatus::kRunning, true);
    auto paused = sorted_with(SeqStatus::kPaused, false);
    std::vector<int32_t> batch;
    const size_t n_wait = std::min(waiting.size(), (size_t)std::max(max_batch_, 0));
    for (size_t i = 0; i < n_wait; i++) {
        waiting[i]->status = SeqStatus::kRunning;
        batch.push_back(waiting[i]->id);
    }
    for (size_t i = 0; i < running.size() && (int32_t)batch.size() < max_batch_; i++) batch.push_back(running[i]->id);
    for (size_t i = 0; i < paused.size() && (int32_t)batch.size() < max_batch_; i++) {
        paused[i]->status = SeqStatus::kRunning;
        batch.push_back(paused[i]->id);
    }
    return batch;
}

void Scheduler::mark_prefilled(int32_t id) {
    std::lock_guard<std::mutex> g(mu_);
    auto it = seqs_.find(id);
    if (it != seqs_.end()) it->second.status = SeqStatus::kRunning;
}

void Scheduler::mark_decoded(int32_t id) {
    std::lock_guard<std::mutex> g(mu_);
    auto it = seqs_.find(id);
    if (it != seqs_.end()) it->second.generated += 1;
}

void Scheduler::preempt(int32_t id) {
    std::lock_guard<std::mutex> g(mu_);
    auto it = seqs_.find(id);
    if (it != seqs_.end()) it->second.status = SeqStatus::kPaused;
}

std::vector<int32_t> Scheduler::handle_memory_pressure(int32_t required, const std::function<int32_t()> &available) {
    std::lock_guard<std::mutex> g(mu_);
    std::vector<int32_t> out;
    while (available() < required) {
        SchedulerSequence *victim = nullptr;
        for (auto &kv : seqs_)
            if (kv.second.status == SeqStatus::kRunning &&
                (victim == nullptr || kv.second.arrival_order > victim->arrival_order))
                victim = &kv.second;
        if (victim == nullptr) break;
        victim->status = SeqStatus::kPaused;
        out.push_back(victim->id);
    }
    return out;
}

int32_t Scheduler::count(SeqStatus s) {
    std::lock_guard<std::mutex> g(mu_);
    int32_t n = 0;
    for (auto &kv : seqs_)
        if (kv.second.status == s) n++;
    return n;
}

bool Scheduler::get(int32_t id, SchedulerSequence *out) {
    std::lock_guard<std::mutex> g(mu_);
    auto it = seqs_.find(id);
    if (it == seqs_.end()) return false;
    *out = it->second;
    return true;
}

}  // namespace pam
