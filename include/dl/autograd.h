#pragma once
// Grad-mode scopes.  Mirrors include/dl/autograd.h:11-34 of the reference (is_grad_enabled, GradModeGuard,
// NoGradGuard): a thread-local recording switch that a scope sets and restores.  This library records no graph on
// any path (the decode path of the reference runs under NoGrad, src/nn/decoder.cpp:128), so the mode only
// reports what callers set; the guards exist so that the reference's inference code compiles and runs unchanged
// (examples/decoder_model.h:32).

#include "dl/types.h"

namespace dl {

/// The calling thread's recording mode: true until a guard turns it off.
DL_API bool is_grad_enabled();

/// Sets the calling thread's mode for the scope and restores the previous mode on exit.
class DL_API GradModeGuard {
public:
    explicit GradModeGuard(bool enabled);
    ~GradModeGuard();
    GradModeGuard(const GradModeGuard&) = delete;
    GradModeGuard& operator=(const GradModeGuard&) = delete;

private:
    bool previous_;
};

/// Turns recording off for the scope (the reference's inference guard).
class DL_API NoGradGuard {
public:
    NoGradGuard();
    ~NoGradGuard();
    NoGradGuard(const NoGradGuard&) = delete;
    NoGradGuard& operator=(const NoGradGuard&) = delete;

private:
    GradModeGuard mode_;
};

} // namespace dl
