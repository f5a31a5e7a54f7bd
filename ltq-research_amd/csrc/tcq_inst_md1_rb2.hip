// Instantiations of the Viterbi launcher for parity mode 1, radix block 2 (S = 1024, 4 states per lane, G <= 4; every
// label count). Split by radix block so the units compile in parallel.
#include "tcq_launch.h"
namespace ltq {
template int launch<10, 2, 1, 4>(const TcqArgs&, hipStream_t);
template int launch_tb<10, 2, 1, 4>(const TcqArgs&, const TcqArgs&, hipStream_t);
template int launch<10, 2, 1, 8>(const TcqArgs&, hipStream_t);
template int launch_tb<10, 2, 1, 8>(const TcqArgs&, const TcqArgs&, hipStream_t);
template int launch<10, 2, 1, 16>(const TcqArgs&, hipStream_t);
template int launch_tb<10, 2, 1, 16>(const TcqArgs&, const TcqArgs&, hipStream_t);
template int launch<10, 2, 1, 32>(const TcqArgs&, hipStream_t);
template int launch_tb<10, 2, 1, 32>(const TcqArgs&, const TcqArgs&, hipStream_t);
}  // namespace ltq
