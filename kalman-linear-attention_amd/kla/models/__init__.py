from kla.models.sequence_model import Block, SequenceModel, build_mixer, register_mixer

__all__ = ["Block", "SequenceModel", "build_mixer", "register_mixer"]
