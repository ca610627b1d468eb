"""ytm_amd -- MI355X-native Tsetlin Machine hot path with the cutm API of Mayur1009/YTM.

    from ytm_amd import MultiClassTM   # instead of: from cutm import MultiClassTM
    from ytm_amd.binarizer import Binarizer, ThermometerBinarizer   # instead of: tm_utils.binarizer
"""
from . import binarizer as binarizer
from .binarizer import Binarizer as Binarizer
from .binarizer import ThermometerBinarizer as ThermometerBinarizer
from .multiclass import MultiClassTM as MultiClassTM
from .multioutput import MultiOutputTM as MultiOutputTM

__all__ = ["MultiClassTM", "MultiOutputTM", "Binarizer", "ThermometerBinarizer", "binarizer"]
