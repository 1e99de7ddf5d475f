// validate.h -- validate-only mode of the launchers (host side).
//
// A layer driver (mi_dit_block_ops, mi_qwen3_layer_ops) calls every entry
// point of its chain twice: first with the calling thread's dry-run flag set,
// so each entry validates its operands and picks its kernel exactly as it
// would for the real call but launches nothing, then for real. A bad operand
// anywhere in the chain is therefore reported before the first kernel runs.
// The flag is per host thread, so concurrent callers on other threads are
// unaffected.
#pragma once

namespace mi {

bool dry_run();
void set_dry_run(bool on);

// sets the calling thread's dry-run flag for one scope
struct DryRunScope {
    bool prev;

    DryRunScope() : prev(dry_run()) { set_dry_run(true); }
    ~DryRunScope() { set_dry_run(prev); }
    DryRunScope(const DryRunScope &)             = delete;
    DryRunScope & operator=(const DryRunScope &) = delete;
};

}  // namespace mi

// every kernel launch of the library goes through this
#define MI_LAUNCH(...)                     \
    do {                                   \
        if (!::mi::dry_run()) {            \
            hipLaunchKernelGGL(__VA_ARGS__); \
        }                                  \
    } while (0)
