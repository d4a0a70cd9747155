"""Input data: the N-MNIST event-camera dataset (.bin files of 40-bit AER events) and
its conversion to the network's InputEvents."""
from salt_amd.data.nmnist import (CHANNEL_NAMES, CLASS_NAMES, IMG_SIZE, NMNISTDataset,
                                  NMNISTSplit, decode_aer, decode_bin_file, list_files)
from salt_amd.data.events import grid_input_events, split_input_events, take_input_events

__all__ = ["CHANNEL_NAMES", "CLASS_NAMES", "IMG_SIZE", "NMNISTDataset", "NMNISTSplit",
           "decode_aer", "decode_bin_file", "list_files", "grid_input_events",
           "split_input_events", "take_input_events"]
