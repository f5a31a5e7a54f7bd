// Instantiations of the Viterbi launcher for parity mode 1 (S = 1024, every label count).
#include "tcq_launch.h"
namespace ltq {
template int launch<10, 1, 4>(const TcqArgs&, hipStream_t);
template int launch<10, 1, 8>(const TcqArgs&, hipStream_t);
template int launch<10, 1, 16>(const TcqArgs&, hipStream_t);
template int launch<10, 1, 32>(const TcqArgs&, hipStream_t);
}  // namespace ltq
