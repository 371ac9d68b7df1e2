#include "launch.hpp"
