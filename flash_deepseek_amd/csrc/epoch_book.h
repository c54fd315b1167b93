// epoch_book.h -- host-side bookkeeping of the batch-1 layer kernel's call
// epochs (plain C++, no HIP: the CPU tests compile it on its own).
//
// Every fdm_moe_layer launch carries a fresh non-zero epoch; values handed
// between its workgroups are tagged with it, and a wait inside the kernel
// that gives up writes it into a device error flag.  The host reports each
// such epoch once, when the caller synchronises.
#pragma once

namespace fdm {

struct EpochBook {
  unsigned epoch = 0;     // last epoch handed to a launch
  unsigned reported = 0;  // last error epoch reported to the caller

  // The next launch's epoch: never 0 (device flags start at 0), so a wrap
  // of the counter skips it.
  unsigned next() {
    if (++epoch == 0) ++epoch;
    return epoch;
  }

  // err_flag: the device error flag after a synchronisation (0 = no wait
  // ever gave up).  True once per timed-out epoch.
  bool new_error(unsigned err_flag) {
    if (err_flag == 0 || err_flag == reported) return false;
    reported = err_flag;
    return true;
  }
};

}  // namespace fdm
