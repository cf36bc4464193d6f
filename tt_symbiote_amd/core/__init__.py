from .module import (HIPModule, StatefulHIPModule, StatefulTTNNModule, StatelessHIPModule,
                     StatelessTTNNModule, TTNNModule)
from .run_config import DispatchManager, NormalRun, get_run_implementation

__all__ = ["HIPModule", "StatelessHIPModule", "StatefulHIPModule", "TTNNModule",
           "StatelessTTNNModule", "StatefulTTNNModule", "DispatchManager", "NormalRun",
           "get_run_implementation"]
