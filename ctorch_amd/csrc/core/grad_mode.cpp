// Thread-local grad mode (reference src/autograd/engine.cpp:11-18): the switch the reference's NoGradGuard scopes.
#include "dl/autograd.h"

namespace dl {

namespace {
thread_local bool grad_enabled = true;
}

bool is_grad_enabled() { return grad_enabled; }

GradModeGuard::GradModeGuard(bool enabled) : previous_(grad_enabled) { grad_enabled = enabled; }
GradModeGuard::~GradModeGuard() { grad_enabled = previous_; }

NoGradGuard::NoGradGuard() : mode_(false) {}
NoGradGuard::~NoGradGuard() = default;

} // namespace dl
