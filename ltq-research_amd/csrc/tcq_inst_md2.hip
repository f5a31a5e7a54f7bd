// Instantiations of the Viterbi launcher for parity mode 2 (S = 1024, every label count).
#include "tcq_launch.h"
namespace ltq {
template int launch<10, 2, 4>(const TcqArgs&, hipStream_t);
template int launch<10, 2, 8>(const TcqArgs&, hipStream_t);
template int launch<10, 2, 16>(const TcqArgs&, hipStream_t);
template int launch<10, 2, 32>(const TcqArgs&, hipStream_t);
}  // namespace ltq
